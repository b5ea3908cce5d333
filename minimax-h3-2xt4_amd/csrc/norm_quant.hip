// DiT modulated RMSNorm, optionally fused with ConvRot256 and the per-row
// INT8 quantizer: the QKV / FC1 input preparation in one pass over x.
//
// One wavefront per row, lane l owning the 16-element units u = l + 64 j
// (elements [16u, 16u + 16)) as in the row quantizer, so loads and the int8
// store are 128-bit and contiguous across the wave. The sum of squares has a
// fixed order that does not depend on the launch: each lane adds its squares
// in (unit, element) order, then the 64 lane partials meet in an xor
// butterfly (offsets 32, 16, ..., 1); IEEE addition is commutative, so every
// lane ends with the same total. rsqrtf is replaced by a correctly rounded
// square root followed by a correctly rounded division.
#include "w8a8_device.h"
#include "w8a8_host.h"

namespace w8a8 {

constexpr int kNormWaves = 4;

struct NormParams {
  const void* x;
  int64_t ldx, rows, cols;
  const float* weight;
  const float* shift;
  const float* mscale;
  int64_t ld_mod;
  int32_t mod_rows;
  float eps, inv_cols;
  const int32_t* labels;
  void* y;
  int64_t ldy;
  int8_t* q;
  int64_t ldq;
  float* qscale;
  const uint32_t* signs;   // ConvRot sign words (0 or 0x80000000 per column), or null
};

// MODE: 0 norm only, 1 quantize, 2 ConvRot256 (fp32) + quantize,
// 3 ConvRot256 rounded to the storage dtype + quantize; 2 or 3 | kNormSigned
// (4): the rotation takes the sign words (diag(s) then H), a compile-time
// choice so that the kernels without signs hold no registers for them.
constexpr int kNormSigned = 4;
template <int MODE>
constexpr int rot_of() { return (MODE & 3) == 2 ? 1 : (MODE & 3) == 3 ? 2 : 0; }

__device__ __forceinline__ void load16_f32(const float* p, float (&v)[16]) {
  const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 t = q[i];
    v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
  }
}

// Table flags of a kernel: kGain (weight present), kMod (shift/scale
// tables present), kAnyTables (decide per call from the pointers).
enum NormTables { kGain = 1, kMod = 2, kAnyTables = 4 };

// v: x on entry; on return the normalized, modulated value rounded to DT
// (as fp32), with its storage bits packed in bits.
template <int DT, int TB>
__device__ __forceinline__ void modulate16(float (&v)[16], uint32_t (&bits)[8], float inv, const float* w,
                                           const float* sh, const float* sc, int64_t c0) {
  const bool gain = (TB & kGain) || ((TB & kAnyTables) && w);
  const bool mod = (TB & kMod) || ((TB & kAnyTables) && sh);
  float wv[16], shv[16], scv[16];
  if (gain) load16_f32(w + c0, wv);
  if (mod) {
    load16_f32(sc + c0, scv);
    load16_f32(sh + c0, shv);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float t = v[i] * inv;
    if (gain) t = t * wv[i];
    if (mod) {
      const float f = 1.0f + scv[i];
      t = t * f;
      t = t + shv[i];
    }
    uint16_t h;
    if constexpr (DT == kF16) {
      h = f2h_of_f32(t);
      v[i] = h2f(h);
    } else {
      h = f2bf(t);
      v[i] = bf2f(h);
    }
    if (i & 1) bits[i >> 1] |= (uint32_t)h << 16;
    else bits[i >> 1] = h;
  }
}

// Waves per workgroup of the norm-only kernel with AdaLN tables: the
// workgroup stages the gain and its first row's shift and scale rows in LDS,
// and its waves whose row carries that label read them there (the rows of a
// segment share the label). 16384 x 3072: 55 -> 41 us. With the rotation the
// tables' LDS costs more occupancy than the loads they save (61 -> 73 us).
constexpr int kNormStageWaves = 8;
constexpr int kNormStageMaxCols = 4096;   // 48 KB of tables

// Dynamic LDS of a W-wave workgroup: the rotation slots, then (STAGE) the
// gain, scale and shift rows.
template <int MODE, int W, bool STAGE>
constexpr int norm_lds_floats(int cols) { return (rot_of<MODE>() ? W * kRotWave : 0) + (STAGE ? 3 * cols : 0); }

template <int DT, int MODE, int J, int TB, int W = kNormWaves, bool STAGE = false>
__global__ __launch_bounds__(64 * W) void norm_quant_kernel(NormParams p) {
  constexpr int ROT = rot_of<MODE>();
  static_assert(!STAGE || (TB == (kGain | kMod) && ROT == 0), "staged tables: norm-only DiT form");
  extern __shared__ __attribute__((aligned(16))) float dsm[];
  float* const lds = dsm;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row0 = (int64_t)blockIdx.x * W;
  const int64_t row = row0 + wave;
  float* const tw = dsm + (ROT ? W * kRotWave : 0);
  float* const tsc = tw + p.cols;
  float* const tsh = tsc + p.cols;
  int l0 = -1;
  if constexpr (STAGE) {
    // Every thread reaches the barrier before any row bound is applied.
    l0 = min(max(p.labels[row0], 0), p.mod_rows - 1);
    const float4* gw = reinterpret_cast<const float4*>(p.weight);
    const float4* gsc = reinterpret_cast<const float4*>(p.mscale + (int64_t)l0 * p.ld_mod);
    const float4* gsh = reinterpret_cast<const float4*>(p.shift + (int64_t)l0 * p.ld_mod);
    const int n4 = (int)(p.cols >> 2);
    for (int i = threadIdx.x; i < n4; i += 64 * W) {
      reinterpret_cast<float4*>(tw)[i] = gw[i];
      reinterpret_cast<float4*>(tsc)[i] = gsc[i];
      reinterpret_cast<float4*>(tsh)[i] = gsh[i];
    }
    __syncthreads();
  }
  if (row >= p.rows) return;
  const int units = (int)(p.cols >> 4);
  const int jcount = (units + 63) >> 6;
  const uint16_t* xrow = reinterpret_cast<const uint16_t*>(p.x) + row * p.ldx;
  uint16_t* yrow = p.y ? reinterpret_cast<uint16_t*>(p.y) + row * p.ldy : nullptr;
  const float* sh = nullptr;
  const float* sc = nullptr;
  bool staged = false;
  if ((TB & kMod) || ((TB & kAnyTables) && p.shift)) {
    const int l = min(max(p.labels[row], 0), p.mod_rows - 1);
    staged = STAGE && l == l0;
    sh = p.shift + (int64_t)l * p.ld_mod;
    sc = p.mscale + (int64_t)l * p.ld_mod;
  }
  float* buf = ROT ? rot_slot(lds, wave, lane) : nullptr;
  const int t = lane & 15;

  // Normalize one unit (v holds x), store y, rotate for the quantizer.
  auto finish = [&](int u, float (&v)[16], float inv, bool store_y) {
    uint32_t bits[8];
    if (STAGE && staged) modulate16<DT, TB>(v, bits, inv, tw, tsh, tsc, (int64_t)u * 16);
    else modulate16<DT, TB>(v, bits, inv, p.weight, sh, sc, (int64_t)u * 16);
    if (store_y && yrow) {
      uint4* dst = reinterpret_cast<uint4*>(yrow + (int64_t)u * 16);
      dst[0] = make_uint4(bits[0], bits[1], bits[2], bits[3]);
      dst[1] = make_uint4(bits[4], bits[5], bits[6], bits[7]);
    }
    if constexpr (ROT != 0) {
      constexpr bool SG = (MODE & kNormSigned) != 0;
      convrot256_lanes<true, SG>(v, buf, t, SG ? p.signs + 256 * (u >> 4) : nullptr);
      if constexpr (ROT == 2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = round_to<DT>(v[i]);
      }
    }
  };
  auto store_q = [&](int u, const float (&v)[16], float s, float rcp) {
    *reinterpret_cast<uint4*>(p.q + row * p.ldq + (int64_t)u * 16) = quant16(v, s, rcp);
  };
  // ss + x*x with one rounding: the square of a 16-bit float is exact in
  // fp32 (at most 22 significant bits, no overflow or underflow), so the FMA
  // equals the separately rounded product and sum.
  auto add_squares = [](float ss, const float (&v)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) ss = __builtin_fmaf(v[i], v[i], ss);
    return ss;
  };
  auto inv_rms = [&](float ss) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss = ss + __shfl_xor(ss, off, 64);
    const float mean = ss * p.inv_cols;
    const float d = mean + p.eps;
    return 1.0f / __builtin_sqrtf(d);
  };

  if constexpr (J > 0) {
    float v[J][16];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int u = lane + 64 * j;
      if (u < units) {
        load16<DT>(xrow + (int64_t)u * 16, v[j]);
        ss = add_squares(ss, v[j]);
      }
    }
    const float inv = inv_rms(ss);
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int u = lane + 64 * j;
      if (u < units) {
        finish(u, v[j], inv, true);
        if constexpr (MODE != 0) {
#pragma unroll
          for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[j][i]));
        }
      }
    }
    if constexpr (MODE != 0) {
      amax = wave_max(amax);
      const float s = row_scale_of(amax);
      const float rcp = 1.0f / s;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int u = lane + 64 * j;
        if (u < units) store_q(u, v[j], s, rcp);
      }
      if (lane == 0) p.qscale[row] = s;
    }
  } else {
    // Rows too wide for registers: sum of squares, then absmax, then the
    // stores, each pass re-reading x.
    float ss = 0.0f;
    for (int j = 0; j < jcount; ++j) {
      const int u = lane + 64 * j;
      if (u < units) {
        float v[16];
        load16<DT>(xrow + (int64_t)u * 16, v);
        ss = add_squares(ss, v);
      }
    }
    const float inv = inv_rms(ss);
    float s = 0.0f, rcp = 0.0f;
    if constexpr (MODE != 0) {
      float amax = 0.0f;
      for (int j = 0; j < jcount; ++j) {
        const int u = lane + 64 * j;
        if (u < units) {
          float v[16];
          load16<DT>(xrow + (int64_t)u * 16, v);
          finish(u, v, inv, false);
#pragma unroll
          for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
        }
      }
      amax = wave_max(amax);
      s = row_scale_of(amax);
      rcp = 1.0f / s;
    }
    for (int j = 0; j < jcount; ++j) {
      const int u = lane + 64 * j;
      if (u < units) {
        float v[16];
        load16<DT>(xrow + (int64_t)u * 16, v);
        finish(u, v, inv, true);
        if constexpr (MODE != 0) store_q(u, v, s, rcp);
      }
    }
    if constexpr (MODE != 0) {
      if (lane == 0) p.qscale[row] = s;
    }
  }
}

template <int DT, int MODE, int TB, int W = kNormWaves, bool STAGE = false>
static void launch_norm_j(const NormParams& p, hipStream_t stream) {
  const int jneed = (int)(((p.cols >> 4) + 63) / 64);
  const dim3 grid((unsigned)((p.rows + W - 1) / W)), block(64 * W);
  const size_t lds = 4 * (size_t)max(norm_lds_floats<MODE, W, STAGE>((int)p.cols), 1);
#define W8A8_NLAUNCH(JJ) hipLaunchKernelGGL((norm_quant_kernel<DT, MODE, JJ, TB, W, STAGE>), grid, block, lds, stream, p)
  switch (jneed) {
    case 1: W8A8_NLAUNCH(1); break;
    case 2: W8A8_NLAUNCH(2); break;
    case 3: W8A8_NLAUNCH(3); break;
    case 4: W8A8_NLAUNCH(4); break;
    case 5: case 6: W8A8_NLAUNCH(6); break;
    case 7: case 8: W8A8_NLAUNCH(8); break;
    default: W8A8_NLAUNCH(0); break;
  }
#undef W8A8_NLAUNCH
}

// Rows held in registers for the DiT (gain + AdaLN tables) and plain
// RMSNorm (gain only) forms; other table combinations take the streaming
// kernel with the tables decided per call.
template <int DT, int MODE>
static int launch_norm(const NormParams& p, hipStream_t stream) {
  if (MODE == 0 && p.weight && p.shift && p.cols <= kNormStageMaxCols) {
    if constexpr (MODE == 0) launch_norm_j<DT, MODE, kGain | kMod, kNormStageWaves, true>(p, stream);
  } else if (p.weight && p.shift) {
    launch_norm_j<DT, MODE, kGain | kMod>(p, stream);
  } else if (p.weight) {
    launch_norm_j<DT, MODE, kGain>(p, stream);
  } else {
    const dim3 grid((unsigned)((p.rows + kNormWaves - 1) / kNormWaves)), block(64 * kNormWaves);
    hipLaunchKernelGGL((norm_quant_kernel<DT, MODE, 0, kAnyTables>), grid, block,
                       4 * (size_t)max(norm_lds_floats<MODE, kNormWaves, false>(0), 1), stream, p);
  }
  return launch_status("w8a8_norm_quantize");
}

}  // namespace w8a8

extern "C" int w8a8_norm_quantize(const W8A8NormArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_norm_quantize: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8NormArgs), "w8a8_norm_quantize: struct_size %u != %zu",
               a->struct_size, sizeof(W8A8NormArgs));
  W8A8_REQUIRE(a->x_dtype == W8A8_F16 || a->x_dtype == W8A8_BF16, "w8a8_norm_quantize: x_dtype %d not F16/BF16",
               a->x_dtype);
  W8A8_REQUIRE(a->rows >= 0 && a->cols >= 0, "w8a8_norm_quantize: negative shape");
  W8A8_REQUIRE(a->y != nullptr || a->q != nullptr, "w8a8_norm_quantize: neither y nor q requested");
  W8A8_REQUIRE(a->convrot == 0 || a->convrot == 256, "w8a8_norm_quantize: convrot must be 0 or 256");
  W8A8_REQUIRE(a->round_rotated == 0 || a->round_rotated == 1, "w8a8_norm_quantize: round_rotated must be 0 or 1");
  const int group = (a->q && a->convrot) ? 256 : 16;
  W8A8_REQUIRE(a->cols % group == 0, "w8a8_norm_quantize: cols %lld not a multiple of %d", (long long)a->cols,
               group);
  W8A8_REQUIRE(a->cols <= ((int64_t)1 << 30), "w8a8_norm_quantize: cols too large");
  W8A8_REQUIRE((a->mod_shift == nullptr) == (a->mod_scale == nullptr),
               "w8a8_norm_quantize: mod_shift and mod_scale go together");
  if (a->rows == 0) return W8A8_OK;
  W8A8_REQUIRE(a->cols > 0, "w8a8_norm_quantize: zero-width rows have no norm");
  W8A8_REQUIRE(a->x != nullptr && aligned16(a->x) && a->ldx >= a->cols && (a->ldx * 2) % 16 == 0,
               "w8a8_norm_quantize: x must be 16-byte aligned with ldx >= cols and a 16-byte row stride");
  if (a->y) {
    W8A8_REQUIRE(aligned16(a->y) && a->ldy >= a->cols && (a->ldy * 2) % 16 == 0,
                 "w8a8_norm_quantize: y must be 16-byte aligned with ldy >= cols and a 16-byte row stride");
  }
  if (a->q) {
    W8A8_REQUIRE(a->q_scale != nullptr, "w8a8_norm_quantize: q requires q_scale");
    W8A8_REQUIRE(aligned16(a->q) && a->ldq >= a->cols && a->ldq % 16 == 0,
                 "w8a8_norm_quantize: q must be 16-byte aligned with ldq >= cols, a multiple of 16");
  }
  W8A8_REQUIRE(a->weight == nullptr || aligned16(a->weight), "w8a8_norm_quantize: weight must be 16-byte aligned");
  if (a->mod_shift) {
    W8A8_REQUIRE(a->labels != nullptr && a->mod_rows >= 1, "w8a8_norm_quantize: modulation needs labels, mod_rows");
    W8A8_REQUIRE(aligned16(a->mod_shift) && aligned16(a->mod_scale) && a->ld_mod >= a->cols && a->ld_mod % 4 == 0,
                 "w8a8_norm_quantize: tables must be 16-byte aligned with ld_mod >= cols, a multiple of 4");
  }
  NormParams p;
  p.x = a->x;
  p.ldx = a->ldx;
  p.rows = a->rows;
  p.cols = a->cols;
  p.weight = a->weight;
  p.shift = a->mod_shift;
  p.mscale = a->mod_scale;
  p.ld_mod = a->ld_mod;
  p.mod_rows = a->mod_rows;
  p.eps = a->eps;
  // fp32(1/cols), the constant the reference multiplies the sum by.
  p.inv_cols = (float)(1.0 / (double)a->cols);
  p.labels = a->labels;
  p.y = a->y;
  p.ldy = a->ldy;
  p.q = a->q;
  p.ldq = a->ldq;
  p.qscale = a->q_scale;
  W8A8_REQUIRE(a->convrot_signs == nullptr || (a->q && a->convrot && aligned16(a->convrot_signs)),
               "w8a8_norm_quantize: convrot_signs needs q, convrot and a 16-byte aligned array");
  p.signs = a->convrot_signs;
  hipStream_t stream = reinterpret_cast<hipStream_t>(a->stream);
  const int mode = (a->q == nullptr ? 0 : a->convrot == 0 ? 1 : a->round_rotated ? 3 : 2) |
                   (a->convrot_signs ? kNormSigned : 0);
  if (a->x_dtype == W8A8_F16) {
    switch (mode) {
      case 0: return launch_norm<kF16, 0>(p, stream);
      case 1: return launch_norm<kF16, 1>(p, stream);
      case 2: return launch_norm<kF16, 2>(p, stream);
      case 3: return launch_norm<kF16, 3>(p, stream);
      case 6: return launch_norm<kF16, 6>(p, stream);
      default: return launch_norm<kF16, 7>(p, stream);
    }
  }
  switch (mode) {
    case 0: return launch_norm<kBF16, 0>(p, stream);
    case 1: return launch_norm<kBF16, 1>(p, stream);
    case 2: return launch_norm<kBF16, 2>(p, stream);
    case 3: return launch_norm<kBF16, 3>(p, stream);
    case 6: return launch_norm<kBF16, 6>(p, stream);
    default: return launch_norm<kBF16, 7>(p, stream);
  }
}
