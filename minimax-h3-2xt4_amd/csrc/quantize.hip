// Dynamic per-row absmax INT8 quantization, optionally after ConvRot256.
//
// One wavefront per row. Lane l owns the 16-element units u = l + 64 j
// (elements [16u, 16u + 16)), loaded with 128-bit loads and stored as one
// 128-bit int8 store, so each wave instruction touches a contiguous span.
// With ConvRot256 a 256-column group is owned by 16 consecutive lanes and
// rotated through a wave-private LDS transpose (w8a8_device.h).
#include <atomic>

#include "w8a8_device.h"
#include "w8a8_host.h"

namespace w8a8 {

constexpr int kQuantWaves = 4;
constexpr int kQuantMaxJ = 8;  // units per lane kept in registers

template <int DT>
constexpr int dt_bytes() { return DT == kF32 ? 4 : 2; }

// The ROT bit of a rotation that takes the sign words (diag(s) then H).
constexpr int kSigned = 4;

// ROT: 0 no rotation, 1 ConvRot256 kept in FP32, 2 ConvRot256 rounded to
// the input dtype, each rotation | kSigned with signs. J > 0: the row (at
// most J units per lane) stays in registers between the absmax and the
// quantization. J == 0: streaming, the row is read twice.
template <int DT, int ROT, int J>
__global__ __launch_bounds__(256) void quantize_rows_kernel(
    const void* __restrict__ x, int64_t ldx, int64_t rows, int64_t cols,
    const float* __restrict__ row_max, int8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ scale, float* __restrict__ row_max_out, const uint32_t* __restrict__ signs) {
  constexpr int RM = ROT & 3;
  constexpr bool SG = (ROT & kSigned) != 0;
  __shared__ float lds[RM ? kQuantWaves * kRotWave : 1];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + wave;
  if (row >= rows) return;
  const int units = (int)(cols >> 4);
  const int jcount = (units + 63) >> 6;
  const char* xrow = reinterpret_cast<const char*>(x) + row * ldx * dt_bytes<DT>();
  float* buf = RM ? rot_slot(lds, wave, lane) : nullptr;
  const int t = lane & 15;

  // The sign words of unit u's 256-column group (ConvRot with signs).
  auto smask = [&](int u) { return SG ? signs + 256 * (u >> 4) : nullptr; };
  auto load_unit = [&](int u, float (&v)[16]) {
    load16<DT>(xrow + (int64_t)u * 16 * dt_bytes<DT>(), v);
    if constexpr (RM != 0) {
      convrot256_lanes<true, SG>(v, buf, t, smask(u));
      if constexpr (RM == 2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = round_to<DT>(v[i]);
      }
    }
  };
  auto store_unit = [&](int u, const float (&v)[16], float s, float rcp) {
    *reinterpret_cast<uint4*>(q + row * ldq + (int64_t)u * 16) = quant16(v, s, rcp);
  };

  if constexpr (J > 0) {
    // Every unit's loads are issued before the first is transformed, so the
    // row's memory latency is paid once, not once per unit (each rotation's
    // LDS transpose orders the wave's memory accesses).
    // Lanes past the row's last unit load that unit again (unused), so the
    // loads are unconditional and the waits before each unit count exactly.
    uint4 raw[J][4];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int u = min(lane + 64 * j, units - 1);
      raw16<DT>(xrow + (int64_t)u * 16 * dt_bytes<DT>(), raw[j]);
    }
    // Straight-line over all J units (a 256-column group is wholly in or
    // out of the row, so the rotation's 16 lanes agree); units past the row
    // are left out of the maximum and never stored.
    // ConvRot256 rounded to fp16 (KEEP16): the rotated units are kept as
    // packed fp16 pairs (exactly the rounded values), half the registers,
    // and the maximum is taken on the fp32 rotation and rounded once:
    // rounding is monotonic and odd, so that is the maximum of the rounded
    // magnitudes (fmaxf skips NaN either way).
    constexpr bool KEEP16 = RM == 2 && DT == kF16;
    float v[KEEP16 ? 1 : J][16];
    uint32_t h16[KEEP16 ? J : 1][8];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float (&vj)[16] = v[KEEP16 ? 0 : j];
      unpack16<DT>(raw[j], vj);
      if constexpr (RM != 0) {
        convrot256_lanes<true, SG>(vj, buf, t, smask(min(lane + 64 * j, units - 1)));
        if constexpr (RM == 2 && !KEEP16) {
#pragma unroll
          for (int i = 0; i < 16; ++i) vj[i] = round_to<DT>(vj[i]);
        }
      }
      float m = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(vj[i]));
      amax = lane + 64 * j < units ? fmaxf(amax, m) : amax;
      if constexpr (KEEP16) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          h16[j][i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{vj[2 * i], vj[2 * i + 1]}, v2h));
      }
    }
    if constexpr (KEEP16) amax = round_to<DT>(amax);
    amax = row_max ? row_max[row] : wave_max(amax);
    if (row_max_out != nullptr && lane == 0) row_max_out[row] = amax;
    if (q == nullptr) return;  // maximum phase only
    const float s = row_scale_of(amax);
    const float rcp = 1.0f / s;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int u = lane + 64 * j;
      if (u < units) {
        if constexpr (KEEP16) {
          float w[16];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            w[2 * i] = h2f((uint16_t)(h16[j][i] & 0xffffu));
            w[2 * i + 1] = h2f((uint16_t)(h16[j][i] >> 16));
          }
          store_unit(u, w, s, rcp);
        } else {
          store_unit(u, v[j], s, rcp);
        }
      }
    }
    if (lane == 0) scale[row] = s;
  } else {
    float amax = 0.0f;
    if (row_max) {
      amax = row_max[row];
    } else {
      for (int j = 0; j < jcount; ++j) {
        const int u = lane + 64 * j;
        if (u < units) {
          float v[16];
          load_unit(u, v);
#pragma unroll
          for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
        }
      }
      amax = wave_max(amax);
    }
    if (row_max_out != nullptr && lane == 0) row_max_out[row] = amax;
    if (q == nullptr) return;  // maximum phase only
    const float s = row_scale_of(amax);
    const float rcp = 1.0f / s;
    for (int j = 0; j < jcount; ++j) {
      const int u = lane + 64 * j;
      if (u < units) {
        float v[16];
        load_unit(u, v);
        store_unit(u, v, s, rcp);
      }
    }
    if (lane == 0) scale[row] = s;
  }
}

// Few rows (decode / short prefill): one workgroup of W wavefronts per row,
// thread t owning units u = t + 64 W j (J units, kept in registers), so a
// row is spread over W wavefronts instead of one: W = 16 for up to one row
// per CU (four waves per SIMD), W = 4 beyond.
template <int ROT, int W>
constexpr int row_wg_lds_bytes() { return (((ROT & 3) ? W * kRotWave : 0) + W) * 4; }

template <int DT, int ROT, int J, int W>
__global__ __launch_bounds__(64 * W) void quantize_row_wg_kernel(
    const void* __restrict__ x, int64_t ldx, int64_t cols, const float* __restrict__ row_max,
    int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale, float* __restrict__ row_max_out,
    const uint32_t* __restrict__ signs) {
  constexpr int RM = ROT & 3;
  constexpr bool SG = (ROT & kSigned) != 0;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* const lds = smem;
  float* const wmax = smem + (RM ? W * kRotWave : 0);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t row = blockIdx.x;
  const int units = (int)(cols >> 4);
  const char* xrow = reinterpret_cast<const char*>(x) + row * ldx * dt_bytes<DT>();
  float* buf = RM ? rot_slot(lds, wave, lane) : nullptr;
  const int t = lane & 15;
  float v[J][16];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int u = tid + 64 * W * j;
    if (u < units) {
      load16<DT>(xrow + (int64_t)u * 16 * dt_bytes<DT>(), v[j]);
      if constexpr (RM != 0) {
        convrot256_lanes<true, SG>(v[j], buf, t, SG ? signs + 256 * (u >> 4) : nullptr);
        if constexpr (RM == 2) {
#pragma unroll
          for (int i = 0; i < 16; ++i) v[j][i] = round_to<DT>(v[j][i]);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[j][i]));
    }
  }
  amax = wave_max(amax);
  if (lane == 0) wmax[wave] = amax;
  __syncthreads();
  if (row_max) {
    amax = row_max[row];
  } else {
    amax = wmax[0];
#pragma unroll
    for (int w = 1; w < W; ++w) amax = fmaxf(amax, wmax[w]);
  }
  if (row_max_out != nullptr && tid == 0) row_max_out[row] = amax;
  if (q == nullptr) return;  // maximum phase only
  const float s = row_scale_of(amax);
  const float rcp = 1.0f / s;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int u = tid + 64 * W * j;
    if (u < units) *reinterpret_cast<uint4*>(q + row * ldq + (int64_t)u * 16) = quant16(v[j], s, rcp);
  }
  if (tid == 0) scale[row] = s;
}

template <int DT, int ROT>
static int launch_quantize(const W8A8QuantArgs* a, hipStream_t stream) {
  // Below 2048 rows a wavefront per row leaves most of the GPU idle, and
  // rows wider than 4096 columns hold too many registers per wave (or, past
  // 8192, read the row twice): spread each row over a workgroup (up to 16384
  // columns). Timed on one box: 1024 x 3072 7.5 -> 5.6 us, 4096 x 8192
  // 34.2 -> 25.6 us, 1024 x 14336 36.6 -> 14.4 us; 4096 x 3072 stays on a
  // wavefront per row (12.6 against 17.1 us).
  if (a->cols <= 16384 && (a->rows < 2048 || (a->cols > 4096 && a->rows < 8192))) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
      set_error("w8a8_quantize_rows: hipGetDevice failed");
      return W8A8_ERR_LAUNCH;
    }
    const dim3 g((unsigned)a->rows);
    if (a->rows <= (int64_t)device_cus(dev)) {
      // 16 waves, one unit per thread. With the rotation the LDS exceeds the
      // 64 KB default: raise the limit once per device.
      constexpr int kLds = row_wg_lds_bytes<ROT, 16>();
      static std::atomic<uint64_t> enabled{0};
      const uint64_t bit = 1ull << dev;
      if (!(enabled.load(std::memory_order_acquire) & bit)) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&quantize_row_wg_kernel<DT, ROT, 1, 16>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
        if (e != hipSuccess) {
          set_error("w8a8_quantize_rows: cannot enable %d bytes of LDS: %s", kLds, hipGetErrorString(e));
          return W8A8_ERR_LAUNCH;
        }
        enabled.fetch_or(bit, std::memory_order_acq_rel);
      }
      hipLaunchKernelGGL((quantize_row_wg_kernel<DT, ROT, 1, 16>), g, dim3(1024), kLds, stream, a->x, a->ldx,
                         a->cols, a->row_max, a->q, a->ldq, a->scale, a->row_max_out, a->convrot_signs);
      return launch_status("w8a8_quantize_rows");
    }
    const int jw = (int)((a->cols / 16 + 255) / 256);
    const dim3 b(256);
    constexpr int kLds4 = row_wg_lds_bytes<ROT, 4>();
#define W8A8_WLAUNCH(JJ)                                                                                    \
  hipLaunchKernelGGL((quantize_row_wg_kernel<DT, ROT, JJ, 4>), g, b, kLds4, stream, a->x, a->ldx, a->cols, \
                     a->row_max, a->q, a->ldq, a->scale, a->row_max_out, a->convrot_signs)
    switch (jw) {
      case 1: W8A8_WLAUNCH(1); break;
      case 2: W8A8_WLAUNCH(2); break;
      case 3: W8A8_WLAUNCH(3); break;
      default: W8A8_WLAUNCH(4); break;
    }
#undef W8A8_WLAUNCH
    return launch_status("w8a8_quantize_rows");
  }
  const int units = (int)(a->cols >> 4);
  const int jneed = (units + 63) / 64;
  const dim3 grid((unsigned)((a->rows + kQuantWaves - 1) / kQuantWaves));
  const dim3 block(64 * kQuantWaves);
#define W8A8_QLAUNCH(JJ)                                                                      \
  hipLaunchKernelGGL((quantize_rows_kernel<DT, ROT, JJ>), grid, block, 0, stream, a->x, a->ldx, \
                     a->rows, a->cols, a->row_max, a->q, a->ldq, a->scale, a->row_max_out, a->convrot_signs)
  switch (jneed) {
    case 1: W8A8_QLAUNCH(1); break;
    case 2: W8A8_QLAUNCH(2); break;
    case 3: W8A8_QLAUNCH(3); break;
    case 4: W8A8_QLAUNCH(4); break;
    case 5: case 6: W8A8_QLAUNCH(6); break;
    case 7: case 8: W8A8_QLAUNCH(8); break;
    default: W8A8_QLAUNCH(0); break;
  }
#undef W8A8_QLAUNCH
  static_assert(kQuantMaxJ == 8, "dispatch covers J = 1..8");
  return launch_status("w8a8_quantize_rows");
}

}  // namespace w8a8

extern "C" int w8a8_quantize_rows(const W8A8QuantArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_quantize_rows: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8QuantArgs),
               "w8a8_quantize_rows: struct_size %u != %zu", a->struct_size, sizeof(W8A8QuantArgs));
  const int es = (a->x_dtype == W8A8_F16 || a->x_dtype == W8A8_BF16) ? 2 : a->x_dtype == W8A8_F32 ? 4 : 0;
  W8A8_REQUIRE(es != 0, "w8a8_quantize_rows: x_dtype %d not F16/BF16/F32", a->x_dtype);
  W8A8_REQUIRE(a->rows >= 0 && a->cols >= 0, "w8a8_quantize_rows: negative shape");
  W8A8_REQUIRE(a->convrot == 0 || a->convrot == 256, "w8a8_quantize_rows: convrot must be 0 or 256");
  W8A8_REQUIRE(a->cols % (a->convrot ? 256 : 16) == 0,
               "w8a8_quantize_rows: cols %lld not a multiple of %d", (long long)a->cols, a->convrot ? 256 : 16);
  W8A8_REQUIRE(a->cols <= ((int64_t)1 << 30), "w8a8_quantize_rows: cols too large");
  if (a->rows == 0 || a->cols == 0) {
    W8A8_REQUIRE(a->cols != 0 || a->rows == 0, "w8a8_quantize_rows: zero-width rows have no scale");
    return W8A8_OK;
  }
  W8A8_REQUIRE(a->x != nullptr, "w8a8_quantize_rows: null x");
  W8A8_REQUIRE((a->q == nullptr) == (a->scale == nullptr), "w8a8_quantize_rows: q and scale go together");
  W8A8_REQUIRE(a->q != nullptr || a->row_max_out != nullptr, "w8a8_quantize_rows: no output requested");
  W8A8_REQUIRE(a->row_max_out == nullptr || a->row_max == nullptr,
               "w8a8_quantize_rows: row_max_out reports the row's own maximum (no external row_max)");
  W8A8_REQUIRE(a->ldx >= a->cols && (a->q == nullptr || a->ldq >= a->cols),
               "w8a8_quantize_rows: leading dimension below cols");
  W8A8_REQUIRE(aligned16(a->x) && (a->ldx * es) % 16 == 0 &&
               (a->q == nullptr || (aligned16(a->q) && a->ldq % 16 == 0)),
               "w8a8_quantize_rows: x/q must be 16-byte aligned with 16-byte row strides");
  W8A8_REQUIRE(a->convrot_signs == nullptr || (a->convrot && aligned16(a->convrot_signs)),
               "w8a8_quantize_rows: convrot_signs needs convrot and a 16-byte aligned array");
  hipStream_t stream = reinterpret_cast<hipStream_t>(a->stream);
  W8A8_REQUIRE(a->round_rotated == 0 || a->round_rotated == 1, "w8a8_quantize_rows: round_rotated must be 0 or 1");
  const int mode = (a->convrot == 0 ? 0 : (a->round_rotated && a->x_dtype != W8A8_F32) ? 2 : 1) |
                   (a->convrot_signs ? kSigned : 0);
  switch (a->x_dtype * 8 + mode) {
    case W8A8_F16 * 8 + 0: return launch_quantize<kF16, 0>(a, stream);
    case W8A8_F16 * 8 + 1: return launch_quantize<kF16, 1>(a, stream);
    case W8A8_F16 * 8 + 2: return launch_quantize<kF16, 2>(a, stream);
    case W8A8_F16 * 8 + 5: return launch_quantize<kF16, 5>(a, stream);
    case W8A8_F16 * 8 + 6: return launch_quantize<kF16, 6>(a, stream);
    case W8A8_BF16 * 8 + 0: return launch_quantize<kBF16, 0>(a, stream);
    case W8A8_BF16 * 8 + 1: return launch_quantize<kBF16, 1>(a, stream);
    case W8A8_BF16 * 8 + 2: return launch_quantize<kBF16, 2>(a, stream);
    case W8A8_BF16 * 8 + 5: return launch_quantize<kBF16, 5>(a, stream);
    case W8A8_BF16 * 8 + 6: return launch_quantize<kBF16, 6>(a, stream);
    case W8A8_F32 * 8 + 0: return launch_quantize<kF32, 0>(a, stream);
    case W8A8_F32 * 8 + 5: return launch_quantize<kF32, 5>(a, stream);
    default: return launch_quantize<kF32, 1>(a, stream);
  }
}
