// Per-head RMS normalization (FP32 statistics and gains) and split-half RoPE
// of the Q and K parts of a packed QKV projection output.
//
// A head (dim = 128) belongs to one 16-lane slice of a wavefront, lane t
// holding elements 8t .. 8t + 7 of its Q and of its K vector (one 16-byte
// load of fp16, two of fp32); a one-wavefront workgroup handles 4 heads of
// one row. The sum of squares has a
// fixed order: each lane adds its eight squares in order, then the 16
// partials meet in an xor butterfly (offsets 8, 4, 2, 1); IEEE addition is
// commutative, so every lane of the slice ends with the same total. The
// normalized vector goes through the wave's LDS so each lane can read the
// partner element of the rotation (the other half of the rotary prefix).
#include "w8a8_device.h"
#include "w8a8_host.h"

namespace w8a8 {

constexpr int kRopeDim = 128;
constexpr int kRopeHeadsPerBlock = 4;   // one wavefront per workgroup

struct RopeParams {
  const void* packed;
  int64_t ldp, rows;
  int heads, rot_dim, half;
  const void* freqs;
  const float* q_gain;
  const float* k_gain;
  float eps, inv_dim;
  void* q_out;
  void* k_out;
};

template <int DT>
__device__ __forceinline__ float load_elem(const void* base, int64_t i) {
  if constexpr (DT == kF32) return reinterpret_cast<const float*>(base)[i];
  else return h2f(reinterpret_cast<const uint16_t*>(base)[i]);
}

// Four consecutive values of type DT starting at element i (16-byte aligned
// for fp32, 8-byte for fp16).
template <int DT>
__device__ __forceinline__ void load4(const void* base, int64_t i, float (&v)[4]) {
  if constexpr (DT == kF32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + i);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  } else {
    const uint2 a = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(base) + i);
    v[0] = h2f((uint16_t)(a.x & 0xffffu)); v[1] = h2f((uint16_t)(a.x >> 16));
    v[2] = h2f((uint16_t)(a.y & 0xffffu)); v[3] = h2f((uint16_t)(a.y >> 16));
  }
}

// VEC: rot_dim / 2 is a multiple of 8, so a lane's eight elements are all
// rotated or all not, lie on one side, and use eight consecutive 2x2
// matrices (one contiguous block of freqs); otherwise each element finds its
// own.
template <int IN, int FQ, int OUT, bool VEC>
__global__ __launch_bounds__(64) void rms_rope_kernel(RopeParams p) {
  __shared__ float lds[kRopeHeadsPerBlock * 2 * kRopeDim];
  const int tid = threadIdx.x, t = tid & 15, slice = tid >> 4;
  // Workgroup (row, c) handles heads 4 c .. 4 c + 3 of one row; a slice
  // normalizes and rotates its head's Q and K vectors, which share the row's
  // rotation matrices. Workgroups come in groups of 8 rows x parts with
  // row = 8 g + (id % 8): workgroups are dealt to the 8 XCDs in turn, so the
  // parts of a row run on one XCD at nearly the same time and its rotation
  // matrices are fetched into that XCD's L2 once (53504 rows x 24 heads:
  // 274 -> 267 us against a (rows, parts) grid, whose parts of a row were a
  // whole pass apart).
  const int parts = (p.heads + kRopeHeadsPerBlock - 1) / kRopeHeadsPerBlock;
  const int64_t grp = (int64_t)blockIdx.x / (8 * parts);
  const int rem = (int)((int64_t)blockIdx.x - grp * 8 * parts);
  const int64_t row = grp * 8 + (rem & 7);
  if (row >= p.rows) return;   // the last group's missing rows (no barrier follows)
  const int head_raw = (rem >> 3) * kRopeHeadsPerBlock + slice;
  const bool active = head_raw < p.heads;
  const int head = active ? head_raw : 0;
  const int width = p.heads * kRopeDim;
  const int col = head * kRopeDim + 8 * t;
  const int d0 = 8 * t;

  float x[2][8];
  {
    const char* prow = reinterpret_cast<const char*>(p.packed) + row * p.ldp * (IN == kF32 ? 4 : 2);
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int c = v * width + col;
      if constexpr (IN == kF32) {
        const float4* s4 = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(prow) + c);
        const float4 a = s4[0], b = s4[1];
        x[v][0] = a.x; x[v][1] = a.y; x[v][2] = a.z; x[v][3] = a.w;
        x[v][4] = b.x; x[v][5] = b.y; x[v][6] = b.z; x[v][7] = b.w;
      } else {
        const uint4 a = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(prow) + c);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[v][2 * i] = h2f((uint16_t)(w[i] & 0xffffu));
          x[v][2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
        }
      }
    }
  }
  // Gains and (VEC) the lane's rotation matrices are loaded with x, so one
  // memory round trip serves the whole vector.
  float4 g4[2][2];
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    const float4* g = reinterpret_cast<const float4*>(v ? p.k_gain : p.q_gain);
    g4[v][0] = g[2 * t];
    g4[v][1] = g[2 * t + 1];
  }
  const char* frow = reinterpret_cast<const char*>(p.freqs) + row * (int64_t)p.half * 4 * (FQ == kF32 ? 4 : 2);
  const int side0 = d0 >= p.half ? 1 : 0;
  const int p0 = d0 - side0 * p.half;
  const bool rotated = d0 < p.rot_dim;
  float diag[VEC ? 8 : 1], offd[VEC ? 8 : 1];
  if constexpr (VEC) {
    if (rotated) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float m[4];   // F[p0 + i][0][0], [0][1], [1][0], [1][1]
        load4<FQ>(frow, (p0 + i) * 4, m);
        diag[i] = side0 ? m[3] : m[0];
        offd[i] = side0 ? m[2] : m[1];
      }
    }
  }
  float n[2][8];
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float sq = x[v][i] * x[v][i];
      ss = ss + sq;
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) ss = ss + __shfl_xor(ss, off, 64);
    const float mean = ss * p.inv_dim;
    const float inv = 1.0f / __builtin_sqrtf(mean + p.eps);
    const float gv[8] = {g4[v][0].x, g4[v][0].y, g4[v][0].z, g4[v][0].w,
                         g4[v][1].x, g4[v][1].y, g4[v][1].z, g4[v][1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s1 = x[v][i] * inv;
      n[v][i] = s1 * gv[i];
    }
  }
  float* vlds = lds + slice * 2 * kRopeDim;
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    float4* w4 = reinterpret_cast<float4*>(vlds + v * kRopeDim + d0);
    w4[0] = make_float4(n[v][0], n[v][1], n[v][2], n[v][3]);
    w4[1] = make_float4(n[v][4], n[v][5], n[v][6], n[v][7]);
  }
  wave_lds_sync();
  float o[2][8];
  if constexpr (VEC) {
    if (rotated) {
      const int other0 = side0 ? d0 - p.half : d0 + p.half;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const float4* r4 = reinterpret_cast<const float4*>(vlds + v * kRopeDim + other0);
        const float4 a4 = r4[0], b4 = r4[1];
        const float part[8] = {a4.x, a4.y, a4.z, a4.w, b4.x, b4.y, b4.z, b4.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float a = n[v][i] * diag[i];
          o[v][i] = __builtin_fmaf(part[i], offd[i], a);
        }
      }
    } else {
#pragma unroll
      for (int v = 0; v < 2; ++v)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[v][i] = n[v][i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d = d0 + i;
      if (d < p.rot_dim) {
        const int side = d >= p.half ? 1 : 0;
        const int pair = d - side * p.half;
        const int other = side ? d - p.half : d + p.half;
        const int f = pair * 4 + side * 2;
        const float dg = load_elem<FQ>(frow, f + side);
        const float od = load_elem<FQ>(frow, f + 1 - side);
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          const float a = n[v][i] * dg;
          o[v][i] = __builtin_fmaf(vlds[v * kRopeDim + other], od, a);
        }
      } else {
#pragma unroll
        for (int v = 0; v < 2; ++v) o[v][i] = n[v][i];
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    char* orow = reinterpret_cast<char*>(v ? p.k_out : p.q_out) + row * (int64_t)width * (OUT == kF32 ? 4 : 2);
    if constexpr (OUT == kF32) {
      float4* d = reinterpret_cast<float4*>(reinterpret_cast<float*>(orow) + col);
      d[0] = make_float4(o[v][0], o[v][1], o[v][2], o[v][3]);
      d[1] = make_float4(o[v][4], o[v][5], o[v][6], o[v][7]);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)f2h_of_f32(o[v][2 * i]) | ((uint32_t)f2h_of_f32(o[v][2 * i + 1]) << 16);
      *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(orow) + col) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

template <int IN, int FQ, int OUT>
static int launch_rope(const RopeParams& p, hipStream_t s) {
  const int parts = (p.heads + kRopeHeadsPerBlock - 1) / kRopeHeadsPerBlock;
  const dim3 grid((unsigned)(((p.rows + 7) / 8) * 8 * parts));
  const dim3 block(64);
  if (p.half % 8 == 0)
    hipLaunchKernelGGL((rms_rope_kernel<IN, FQ, OUT, true>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((rms_rope_kernel<IN, FQ, OUT, false>), grid, block, 0, s, p);
  return launch_status("w8a8_rms_rope");
}

template <int IN, int FQ>
static int launch_rope_out(int out, const RopeParams& p, hipStream_t s) {
  return out == W8A8_F32 ? launch_rope<IN, FQ, kF32>(p, s) : launch_rope<IN, FQ, kF16>(p, s);
}

}  // namespace w8a8

extern "C" int w8a8_rms_rope(const W8A8RmsRopeArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_rms_rope: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8RmsRopeArgs), "w8a8_rms_rope: struct_size %u != %zu", a->struct_size,
               sizeof(W8A8RmsRopeArgs));
  W8A8_REQUIRE(a->in_dtype == W8A8_F16 || a->in_dtype == W8A8_F32, "w8a8_rms_rope: in_dtype %d not F16/F32",
               a->in_dtype);
  W8A8_REQUIRE(a->freq_dtype == W8A8_F16 || a->freq_dtype == W8A8_F32, "w8a8_rms_rope: freq_dtype %d not F16/F32",
               a->freq_dtype);
  W8A8_REQUIRE(a->out_dtype == W8A8_F16 || a->out_dtype == W8A8_F32, "w8a8_rms_rope: out_dtype %d not F16/F32",
               a->out_dtype);
  W8A8_REQUIRE(a->dim == kRopeDim, "w8a8_rms_rope: dim %d != 128 (full-head RMS over 128)", a->dim);
  W8A8_REQUIRE(a->rot_dim > 0 && a->rot_dim <= a->dim && a->rot_dim % 2 == 0,
               "w8a8_rms_rope: rot_dim %d must be even in (0, dim]", a->rot_dim);
  W8A8_REQUIRE(a->rows >= 0 && a->heads > 0, "w8a8_rms_rope: rows >= 0 and heads > 0 required");
  W8A8_REQUIRE(a->rows < ((int64_t)1 << 31) && a->heads <= 4096, "w8a8_rms_rope: rows or heads out of range");
  // One workgroup of 64 threads per (row, 4 heads), rows padded to a multiple
  // of 8: the launch's work-item count must fit 32 bits.
  W8A8_REQUIRE(((a->rows + 7) / 8) * 8 * ((a->heads + kRopeHeadsPerBlock - 1) / kRopeHeadsPerBlock) * 64 <
                   ((int64_t)1 << 32),
               "w8a8_rms_rope: rows x heads too large for one launch");
  if (a->rows == 0) return W8A8_OK;
  const int es = a->in_dtype == W8A8_F32 ? 4 : 2;
  W8A8_REQUIRE(a->packed && a->freqs && a->q_gain && a->k_gain && a->q_out && a->k_out, "w8a8_rms_rope: null buffer");
  W8A8_REQUIRE(a->ldp >= 2 * (int64_t)a->heads * a->dim, "w8a8_rms_rope: ldp %lld below 2*heads*dim",
               (long long)a->ldp);
  W8A8_REQUIRE(aligned16(a->packed) && (a->ldp * es) % 16 == 0 && aligned16(a->q_out) && aligned16(a->k_out),
               "w8a8_rms_rope: packed/outputs must be 16-byte aligned with 16-byte row strides");
  W8A8_REQUIRE(aligned16(a->freqs) && aligned16(a->q_gain) && aligned16(a->k_gain),
               "w8a8_rms_rope: freqs and gains must be 16-byte aligned");
  RopeParams p;
  p.packed = a->packed;
  p.ldp = a->ldp;
  p.rows = a->rows;
  p.heads = a->heads;
  p.rot_dim = a->rot_dim;
  p.half = a->rot_dim / 2;
  p.freqs = a->freqs;
  p.q_gain = a->q_gain;
  p.k_gain = a->k_gain;
  p.eps = a->eps;
  // fp32(1/dim), the constant the reference multiplies the sum by.
  p.inv_dim = (float)(1.0 / (double)a->dim);
  p.q_out = a->q_out;
  p.k_out = a->k_out;
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  if (a->in_dtype == W8A8_F16) {
    return a->freq_dtype == W8A8_F16 ? launch_rope_out<kF16, kF16>(a->out_dtype, p, s)
                                     : launch_rope_out<kF16, kF32>(a->out_dtype, p, s);
  }
  return a->freq_dtype == W8A8_F16 ? launch_rope_out<kF32, kF16>(a->out_dtype, p, s)
                                   : launch_rope_out<kF32, kF32>(a->out_dtype, p, s);
}
