// FC2 prologue: FP32 SwiGLU -> ConvRot256 -> row absmax -> INT8, fused.
//
// One workgroup of W wavefronts per row: 4 W 16-lane slots each own one
// 256-column group per pass (lane t of a slot loads gate/up elements
// [16t, 16t + 16) of the group with 128-bit loads). The rotated FP32 values
// stay in registers until the row maximum is known, so the only HBM traffic
// is the FP16 gate|up row in and the int8 row out (plus the fp32 scale).
// Many rows take the fewest waves (1, 2, 4 or 8) that leave each wave at
// most three passes (the launcher lists the timings behind the rule; at
// width 8192 that is W = 4, two passes); up to one row per CU takes W = 16,
// so a lane transforms a quarter of the groups with four waves per SIMD
// issuing (one row of width 14336: 13.0 -> 8.6 us; at two rows per CU the
// 16-wave workgroups no longer gain).
#include <atomic>

#include "w8a8_device.h"
#include "w8a8_host.h"

namespace w8a8 {

constexpr int kSwigluMaxPasses = 4;  // register-resident up to 16 W groups per row

template <int DT>
constexpr int sw_bytes() { return DT == kF32 ? 4 : 2; }

// Dynamic LDS of a W-wave workgroup: the rotation slots, then the waves'
// maxima.
template <int W>
constexpr int swiglu_lds_bytes() { return (W * kRotWave + W) * 4; }

// P > 0: the row's rotated values stay in registers (P passes of 4 W
// groups). P == 0: streaming, the row is transformed twice (maximum, then
// quantize).
template <int DT, int P, int W, bool SG>
__global__ __launch_bounds__(64 * W) void swiglu_quant_kernel(
    const void* __restrict__ x, int64_t ldx, int64_t rows, int64_t width,
    const float* __restrict__ row_max_in, float* __restrict__ row_max_out,
    float* __restrict__ group_max, int8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ scale, const uint32_t* __restrict__ signs) {
  constexpr int kWaves = W, kSlots = 4 * kWaves;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* const lds = smem;
  float* const wmax = smem + kWaves * kRotWave;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t row = blockIdx.x;
  const int groups = (int)(width >> 8);
  const int slot = tid >> 4;
  const int t = tid & 15;
  float* buf = rot_slot(lds, wave, lane);
  const char* xrow = reinterpret_cast<const char*>(x) + row * ldx * sw_bytes<DT>();

  // v[i] <- rotated element 16 t + i of group g.
  auto transform = [&](int g, float (&v)[16]) {
    float gv[16], uv[16];
    load16<DT>(xrow + ((int64_t)g * 256 + 16 * t) * sw_bytes<DT>(), gv);
    load16<DT>(xrow + (width + (int64_t)g * 256 + 16 * t) * sw_bytes<DT>(), uv);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = DT == kF16 ? swiglu_fp16_gate(gv[i], uv[i]) : swiglu(gv[i], uv[i]);
    convrot256_lanes<true, SG>(v, buf, t, SG ? signs + 256 * g : nullptr);
  };
  auto group_absmax = [&](int g, const float (&v)[16]) {
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(v[j]));
    m = seg16_max(m);
    if (group_max && t == 0) group_max[row * groups + g] = m;
    return m;
  };
  auto store_group = [&](int g, const float (&v)[16], float s, float rcp) {
    *reinterpret_cast<uint4*>(q + row * ldq + (int64_t)g * 256 + 16 * t) = quant16(v, s, rcp);
  };
  auto row_reduce = [&](float m) {
    m = wave_max(m);
    if (lane == 0) wmax[wave] = m;
    __syncthreads();
    float r = wmax[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) r = fmaxf(r, wmax[w]);
    return r;
  };

  if constexpr (P > 0) {
    // Every pass's gate and up loads are issued before the first transform,
    // so the row's memory latency is paid once, not once per pass. Slots
    // past the last group load (and transform) that group again, unused:
    // the code stays straight-line, so the waits before each pass count
    // exactly.
    uint4 graw[P][4], uraw[P][4];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int g = min(slot + kSlots * p, groups - 1);
      raw16<DT>(xrow + ((int64_t)g * 256 + 16 * t) * sw_bytes<DT>(), graw[p]);
      raw16<DT>(xrow + (width + (int64_t)g * 256 + 16 * t) * sw_bytes<DT>(), uraw[p]);
    }
    float v[P][16];
    float local = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int g = slot + kSlots * p;
      float gv[16], uv[16];
      unpack16<DT>(graw[p], gv);
      unpack16<DT>(uraw[p], uv);
#pragma unroll
      for (int i = 0; i < 16; ++i)
        v[p][i] = DT == kF16 ? swiglu_fp16_gate(gv[i], uv[i]) : swiglu(gv[i], uv[i]);
      convrot256_lanes<true, SG>(v[p], buf, t, SG ? signs + 256 * min(g, groups - 1) : nullptr);
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(v[p][j]));
      m = seg16_max(m);
      if (g < groups) {
        if (group_max && t == 0) group_max[row * groups + g] = m;
        local = fmaxf(local, m);
      }
    }
    const float rmax = row_reduce(local);
    if (row_max_out && tid == 0) row_max_out[row] = rmax;
    if (q) {
      const float s = row_scale_of(row_max_in ? row_max_in[row] : rmax);
      const float rcp = 1.0f / s;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int g = slot + kSlots * p;
        if (g < groups) store_group(g, v[p], s, rcp);
      }
      if (tid == 0) scale[row] = s;
    }
  } else {
    float local = 0.0f;
    const bool need_max = !row_max_in || row_max_out || group_max;
    if (need_max) {
      for (int g = slot; g < groups; g += kSlots) {
        float v[16];
        transform(g, v);
        local = fmaxf(local, group_absmax(g, v));
      }
    }
    const float rmax = row_reduce(local);
    if (row_max_out && tid == 0) row_max_out[row] = rmax;
    if (q) {
      const float s = row_scale_of(row_max_in ? row_max_in[row] : rmax);
      const float rcp = 1.0f / s;
      for (int g = slot; g < groups; g += kSlots) {
        float v[16];
        transform(g, v);
        store_group(g, v, s, rcp);
      }
      if (tid == 0) scale[row] = s;
    }
  }
}

template <int DT, int W, bool SG>
static void launch_swiglu_w(const W8A8SwigluArgs* a, hipStream_t stream) {
  const int groups = (int)(a->width >> 8);
  const int passes = (groups + 4 * W - 1) / (4 * W);
  const dim3 grid((unsigned)a->rows), block(64 * W);
#define W8A8_SLAUNCH(PP)                                                                                 \
  hipLaunchKernelGGL((swiglu_quant_kernel<DT, PP, W, SG>), grid, block, swiglu_lds_bytes<W>(), stream, a->x, \
                     a->ldx, a->rows, a->width, a->row_max, a->row_max_out, a->group_max, a->q, a->ldq,  \
                     a->scale, a->convrot_signs)
  switch (passes) {
    case 1: W8A8_SLAUNCH(1); break;
    case 2: W8A8_SLAUNCH(2); break;
    case 3: W8A8_SLAUNCH(3); break;
    case 4: W8A8_SLAUNCH(4); break;
    default: W8A8_SLAUNCH(0); break;
  }
#undef W8A8_SLAUNCH
  static_assert(kSwigluMaxPasses == 4, "dispatch covers P = 1..4");
}

// The 16-wave variants' LDS exceeds the 64 KB default: raise their limit once
// per device.
template <int DT, bool SG>
static int enable_wide_swiglu(int dev) {
  static std::atomic<uint64_t> done{0};
  const uint64_t bit = 1ull << dev;
  if (done.load(std::memory_order_acquire) & bit) return W8A8_OK;
  const void* fns[] = {reinterpret_cast<const void*>(&swiglu_quant_kernel<DT, 0, 16, SG>),
                       reinterpret_cast<const void*>(&swiglu_quant_kernel<DT, 1, 16, SG>),
                       reinterpret_cast<const void*>(&swiglu_quant_kernel<DT, 2, 16, SG>),
                       reinterpret_cast<const void*>(&swiglu_quant_kernel<DT, 3, 16, SG>),
                       reinterpret_cast<const void*>(&swiglu_quant_kernel<DT, 4, 16, SG>)};
  for (const void* f : fns) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, swiglu_lds_bytes<16>());
    if (e != hipSuccess) {
      set_error("w8a8_swiglu_quantize: cannot enable %d bytes of LDS: %s", swiglu_lds_bytes<16>(),
                hipGetErrorString(e));
      return W8A8_ERR_LAUNCH;
    }
  }
  done.fetch_or(bit, std::memory_order_acq_rel);
  return W8A8_OK;
}

template <int DT, bool SG>
static int launch_swiglu(const W8A8SwigluArgs* a, hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("w8a8_swiglu_quantize: hipGetDevice failed");
    return W8A8_ERR_LAUNCH;
  }
  // Waves per row: 16 while the rows fit the CUs one each; otherwise the
  // fewest (a power of two) that leave each wave at most three passes of
  // its 4 groups. Timed on one box at 16384 rows (W = 1 / 2 / 4 / 8):
  // width 2048 41 / 56 / 88 / 156 us, 4096 87 / 78 / 116 / 187, 6144
  // 248 / 141 / 159 / 227, 8192 341 / 197 / 187 / 262, 16384
  // 664 / 631 / 402 / 391, 20480 824 / 790 / 770 / 558 (bit-identical).
  const int64_t groups = a->width >> 8;
  if (a->rows <= (int64_t)device_cus(dev) || groups > 4 * 8 * 3) {
    const int rc = enable_wide_swiglu<DT, SG>(dev);
    if (rc != W8A8_OK) return rc;
    launch_swiglu_w<DT, 16, SG>(a, stream);
  } else if (groups <= 4 * 1 * 3) {
    launch_swiglu_w<DT, 1, SG>(a, stream);
  } else if (groups <= 4 * 2 * 3) {
    launch_swiglu_w<DT, 2, SG>(a, stream);
  } else if (groups <= 4 * 4 * 3) {
    launch_swiglu_w<DT, 4, SG>(a, stream);
  } else {
    launch_swiglu_w<DT, 8, SG>(a, stream);
  }
  return launch_status("w8a8_swiglu_quantize");
}

}  // namespace w8a8

extern "C" int w8a8_swiglu_quantize(const W8A8SwigluArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_swiglu_quantize: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8SwigluArgs),
               "w8a8_swiglu_quantize: struct_size %u != %zu", a->struct_size, sizeof(W8A8SwigluArgs));
  W8A8_REQUIRE(a->x_dtype == W8A8_F16 || a->x_dtype == W8A8_F32,
               "w8a8_swiglu_quantize: x_dtype %d not F16/F32", a->x_dtype);
  const int es = a->x_dtype == W8A8_F16 ? 2 : 4;
  W8A8_REQUIRE(a->rows >= 0 && a->width >= 0, "w8a8_swiglu_quantize: negative shape");
  W8A8_REQUIRE(a->width % 256 == 0, "w8a8_swiglu_quantize: width %lld not a multiple of 256",
               (long long)a->width);
  W8A8_REQUIRE(a->rows <= 0x7fffffffLL && a->width <= ((int64_t)1 << 28), "w8a8_swiglu_quantize: shape too large");
  if (a->rows == 0) return W8A8_OK;
  W8A8_REQUIRE(a->width > 0, "w8a8_swiglu_quantize: zero width");
  W8A8_REQUIRE(a->x != nullptr, "w8a8_swiglu_quantize: null x");
  W8A8_REQUIRE(a->q || a->row_max_out || a->group_max, "w8a8_swiglu_quantize: no output requested");
  W8A8_REQUIRE(!a->q || a->scale, "w8a8_swiglu_quantize: q requires scale");
  W8A8_REQUIRE(a->ldx >= 2 * a->width, "w8a8_swiglu_quantize: ldx below 2*width");
  W8A8_REQUIRE(aligned16(a->x) && (a->ldx * es) % 16 == 0, "w8a8_swiglu_quantize: x must be 16-byte aligned");
  if (a->q) {
    W8A8_REQUIRE(a->ldq >= a->width && a->ldq % 16 == 0 && aligned16(a->q),
                 "w8a8_swiglu_quantize: q must be 16-byte aligned with ldq >= width, ldq %% 16 == 0");
  }
  W8A8_REQUIRE(a->convrot_signs == nullptr || aligned16(a->convrot_signs),
               "w8a8_swiglu_quantize: convrot_signs must be 16-byte aligned");
  hipStream_t stream = reinterpret_cast<hipStream_t>(a->stream);
  // The sign words select their own kernels (compile-time), so the kernels
  // without them hold no registers for the sign path.
  if (a->convrot_signs)
    return a->x_dtype == W8A8_F16 ? launch_swiglu<kF16, true>(a, stream) : launch_swiglu<kF32, true>(a, stream);
  return a->x_dtype == W8A8_F16 ? launch_swiglu<kF16, false>(a, stream) : launch_swiglu<kF32, false>(a, stream);
}
