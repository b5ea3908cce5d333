// INT8 GEMM on gfx950 i8 MFMA (v_mfma_i32_16x16x64_i8) with a fused
// dequantization / bias / residual epilogue, and the standalone epilogue.
//
// C[m][n] = sum_k A[m][k] * B[n][k], A = activations [M,K], B = weights
// [N,K], both K-contiguous. Workgroup tile 256x256, K step 64, four
// wavefronts each owning a 128x128 quadrant (8x8 MFMA tiles of 16x16,
// 256 int32 accumulators per lane). The MFMA's A operand is the weight tile
// and its B operand the activation tile, so each lane ends with four
// consecutive output columns of one row (vector stores in the epilogue).
// Global->LDS goes through registers with a two-buffer LDS pipeline (one
// barrier per K step); the LDS rows (64 bytes) have their 16-byte chunks
// XOR-swizzled so that the 16 lanes reading one fragment column hit distinct
// banks.
#include "w8a8_device.h"
#include "w8a8_host.h"

namespace w8a8 {

struct GemmParams {
  const int8_t* a;
  const int8_t* b;
  int64_t lda, ldb;
  int m, n, k;
  const float* row_scale;
  const float* col_scale;
  int col_stride;
  int bias_dtype;  // 0 none, kF16, kF32
  const void* bias;
  const uint16_t* residual;
  int64_t ldr;
  void* out;
  int64_t ldc;
};

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kTileBytes = kBM * kBK;  // one operand tile per buffer

// 16-byte chunk swizzle of LDS row r (depends on r & 15 only).
__device__ __forceinline__ int chunk_swizzle(int r) {
  return (((r >> 1) ^ (r >> 3)) & 1) | (((r >> 2) & 1) << 1);
}

// Workgroup id -> output tile. Consecutive workgroup ids are dispatched
// round-robin over the 8 XCDs; remap so each XCD owns a contiguous range of
// logical tiles, then raster in groups of 8 row-tiles so concurrently running
// tiles share A rows and B rows in that XCD's L2.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  constexpr int kGroupM = 8;
  const int group = kGroupM * tiles_n;
  const int first_m = (pid / group) * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in = pid - (pid / group) * group;
  tm = first_m + in % gsize;
  tn = in / gsize;
}

__device__ __forceinline__ float load_bias(const GemmParams& p, int n) {
  if (p.bias_dtype == kF16) return h2f(reinterpret_cast<const uint16_t*>(p.bias)[n]);
  if (p.bias_dtype == kF32) return reinterpret_cast<const float*>(p.bias)[n];
  return 0.0f;
}

// Epilogue of four consecutive columns n..n+3 of row m (valid of them in
// range). Shared by the fused GEMM epilogue and the standalone dequantize.
template <int EPI, int OUT>
__device__ __forceinline__ void epilogue4(const GemmParams& p, int m, int n, int valid, const int (&c)[4],
                                          float a) {
  if constexpr (EPI == kEpiInt32) {
    int* o = reinterpret_cast<int*>(p.out) + (int64_t)m * p.ldc + n;
    if (valid == 4) {
      *reinterpret_cast<int4*>(o) = make_int4(c[0], c[1], c[2], c[3]);
    } else {
      for (int v = 0; v < valid; ++v) o[v] = c[v];
    }
  } else {
    float y[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int nn = v < valid ? n + v : n;
      const float w = p.col_scale[(int64_t)nn * p.col_stride];
      y[v] = dequant1<EPI>(c[v], a, w);
      if (p.bias_dtype) y[v] = y[v] + load_bias(p, nn);
    }
    if constexpr (OUT == kF32) {
      float* o = reinterpret_cast<float*>(p.out) + (int64_t)m * p.ldc + n;
      if (valid == 4) *reinterpret_cast<float4*>(o) = make_float4(y[0], y[1], y[2], y[3]);
      else for (int v = 0; v < valid; ++v) o[v] = y[v];
    } else {
      uint16_t h[4];
      if constexpr (OUT == kF16) {
        if (p.residual) {
          const uint16_t* r = p.residual + (int64_t)m * p.ldr + n;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float branch = h2f(f2h(y[v]));
            const float res = v < valid ? h2f(r[v]) : 0.0f;
            h[v] = f2h(res + branch);
          }
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) h[v] = f2h(y[v]);
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) h[v] = f2bf(y[v]);
      }
      uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + (int64_t)m * p.ldc + n;
      if (valid == 4) {
        *reinterpret_cast<uint2*>(o) =
            make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
      } else {
        for (int v = 0; v < valid; ++v) o[v] = h[v];
      }
    }
  }
}

template <int EPI, int OUT>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_i8_256x256(GemmParams p) {
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * 2 * kTileBytes];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tiles_m = (p.m + kBM - 1) / kBM, tiles_n = (p.n + kBN - 1) / kBN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;

  // Global -> LDS: thread (lrow, lchunk) moves 16 bytes of rows
  // lrow + 64 s (s = 0..3) of each operand tile per K step.
  const int lrow = tid >> 2, lchunk = tid & 3;
  const int st_off = lrow * kBK + ((lchunk ^ chunk_swizzle(lrow)) << 4);
  const int8_t* ga[4];
  const int8_t* gb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int ra = min(m0 + 64 * s + lrow, p.m - 1);
    const int rb = min(n0 + 64 * s + lrow, p.n - 1);
    ga[s] = p.a + (int64_t)ra * p.lda + lchunk * 16;
    gb[s] = p.b + (int64_t)rb * p.ldb + lchunk * 16;
  }
  const int ktiles = (p.k + kBK - 1) / kBK;

  v4i ra[4], rb[4];
  auto gload = [&](int kt) {
    const int kof = kt * kBK;
    const bool kin = kof + lchunk * 16 < p.k;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      ra[s] = kin ? *reinterpret_cast<const v4i*>(ga[s] + kof) : v4i{0, 0, 0, 0};
      rb[s] = kin ? *reinterpret_cast<const v4i*>(gb[s] + kof) : v4i{0, 0, 0, 0};
    }
  };
  auto sstore = [&](int buf) {
    int8_t* sa = smem + buf * 2 * kTileBytes;
    int8_t* sb = sa + kTileBytes;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      *reinterpret_cast<v4i*>(sa + s * 64 * kBK + st_off) = ra[s];
      *reinterpret_cast<v4i*>(sb + s * 64 * kBK + st_off) = rb[s];
    }
  };

  // Fragment reads: lane (fr = lane % 16, fc = lane / 16) reads row fr,
  // 16-byte chunk fc of each 16-row block.
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 15, fc = lane >> 4;
  const int frag = fr * kBK + ((fc ^ chunk_swizzle(fr)) << 4);
  const int a_off = wm * 128 * kBK + frag;
  const int b_off = wn * 128 * kBK + frag;

  v4i acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) gload(kt + 1);
    const int8_t* sa = smem + cur * 2 * kTileBytes;
    const int8_t* sb = sa + kTileBytes;
    v4i fa[8], fb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) fb[i] = *reinterpret_cast<const v4i*>(sa + a_off + i * 16 * kBK);
#pragma unroll
    for (int i = 0; i < 8; ++i) fa[i] = *reinterpret_cast<const v4i*>(sb + b_off + i * 16 * kBK);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
        acc[nb][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[nb], fb[mb], acc[nb][mb], 0, 0, 0);
    if (kt + 1 < ktiles) sstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds C[m][n..n+3] with m = mbase + fr,
  // n = nbase + 4 fc for each (nb, mb) MFMA tile.
  const int mw = m0 + wm * 128, nw = n0 + wn * 128;
  float as[8];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const int m = mw + mb * 16 + fr;
    as[mb] = (EPI != kEpiInt32 && m < p.m) ? p.row_scale[m] : 0.0f;
  }
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    const int n = nw + nb * 16 + 4 * fc;
    const int valid = min(4, p.n - n);
    if (valid <= 0) continue;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const int m = mw + mb * 16 + fr;
      if (m >= p.m) continue;
      const int c[4] = {acc[nb][mb][0], acc[nb][mb][1], acc[nb][mb][2], acc[nb][mb][3]};
      epilogue4<EPI, OUT>(p, m, n, valid, c, as[mb]);
    }
  }
}

// Standalone epilogue: thread -> 4 consecutive columns of one row.
template <int EPI, int OUT>
__global__ __launch_bounds__(256) void dequant_kernel(GemmParams p, const int32_t* __restrict__ acc,
                                                      int64_t ldacc) {
  const int quads = (p.n + 3) >> 2;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.m * quads) return;
  const int m = (int)(idx / quads);
  const int n = (int)(idx - (int64_t)m * quads) * 4;
  const int valid = min(4, p.n - n);
  const int32_t* src = acc + (int64_t)m * ldacc + n;
  int c[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) c[v] = v < valid ? src[v] : 0;
  epilogue4<EPI, OUT>(p, m, n, valid, c, p.row_scale[m]);
}

static int check_epilogue(int epi, int out_dtype, int bias_dtype, const void* bias, const void* residual,
                          int64_t ldr, int64_t n, const float* row_scale, const float* col_scale,
                          int64_t col_stride, const void* out, int64_t ldc) {
  W8A8_REQUIRE(out != nullptr, "null output");
  W8A8_REQUIRE(aligned16(out) && ldc % 4 == 0 && ldc >= n, "out must be 16-byte aligned, ldc %% 4 == 0, ldc >= n");
  if (epi == W8A8_EPI_INT32) {
    W8A8_REQUIRE(out_dtype == W8A8_I32, "EPI_INT32 requires out_dtype I32");
    W8A8_REQUIRE(bias == nullptr && residual == nullptr, "EPI_INT32 takes no bias or residual");
    return W8A8_OK;
  }
  W8A8_REQUIRE(epi == W8A8_EPI_ROW || epi == W8A8_EPI_COLUMN, "unknown epilogue %d", epi);
  W8A8_REQUIRE(out_dtype == W8A8_F16 || out_dtype == W8A8_BF16 || out_dtype == W8A8_F32,
               "dequantized out_dtype must be F16, BF16 or F32");
  W8A8_REQUIRE(row_scale && col_scale, "row_scale and col_scale required");
  W8A8_REQUIRE(col_stride == 0 || col_stride == 1, "col_scale_stride must be 0 (scalar) or 1");
  W8A8_REQUIRE(bias == nullptr || bias_dtype == W8A8_F16 || bias_dtype == W8A8_F32,
               "bias_dtype must be F16 or F32");
  if (residual) {
    W8A8_REQUIRE(out_dtype == W8A8_F16, "residual requires F16 output");
    W8A8_REQUIRE(((uintptr_t)residual & 7u) == 0 && ldr % 4 == 0 && ldr >= n,
                 "residual must be 8-byte aligned with ldr %% 4 == 0, ldr >= n");
  }
  return W8A8_OK;
}

template <int EPI>
static void launch_gemm_out(int out, const GemmParams& p, dim3 grid, hipStream_t s) {
  switch (out) {
    case kF16: hipLaunchKernelGGL((gemm_i8_256x256<EPI, kF16>), grid, dim3(256), 0, s, p); break;
    case kBF16: hipLaunchKernelGGL((gemm_i8_256x256<EPI, kBF16>), grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL((gemm_i8_256x256<EPI, kF32>), grid, dim3(256), 0, s, p); break;
  }
}

template <int EPI>
static void launch_dequant_out(int out, const GemmParams& p, const int32_t* acc, int64_t ldacc, dim3 grid,
                               hipStream_t s) {
  switch (out) {
    case kF16: hipLaunchKernelGGL((dequant_kernel<EPI, kF16>), grid, dim3(256), 0, s, p, acc, ldacc); break;
    case kBF16: hipLaunchKernelGGL((dequant_kernel<EPI, kBF16>), grid, dim3(256), 0, s, p, acc, ldacc); break;
    default: hipLaunchKernelGGL((dequant_kernel<EPI, kF32>), grid, dim3(256), 0, s, p, acc, ldacc); break;
  }
}

}  // namespace w8a8

extern "C" int w8a8_gemm(const W8A8GemmArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_gemm: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8GemmArgs), "w8a8_gemm: struct_size %u != %zu", a->struct_size,
               sizeof(W8A8GemmArgs));
  W8A8_REQUIRE(a->m >= 0 && a->n >= 0 && a->k >= 0, "w8a8_gemm: negative shape");
  W8A8_REQUIRE(a->m < (1LL << 31) && a->n < (1LL << 31) && a->k < (1LL << 31), "w8a8_gemm: shape too large");
  W8A8_REQUIRE(a->k * 128 * 128 < (1LL << 31), "w8a8_gemm: k=%lld could overflow int32 accumulation",
               (long long)a->k);
  W8A8_REQUIRE(a->k % 16 == 0, "w8a8_gemm: k %lld not a multiple of 16", (long long)a->k);
  if (a->m == 0 || a->n == 0) return W8A8_OK;
  int rc = check_epilogue(a->epilogue, a->out_dtype, a->bias_dtype, a->bias, a->residual, a->ldr, a->n,
                          a->row_scale, a->col_scale, a->col_scale_stride, a->out, a->ldc);
  if (rc != W8A8_OK) return rc;
  W8A8_REQUIRE(a->k == 0 || (a->a && a->b), "w8a8_gemm: null operand");
  W8A8_REQUIRE(aligned16(a->a) && aligned16(a->b) && a->lda % 16 == 0 && a->ldb % 16 == 0 && a->lda >= a->k &&
                   a->ldb >= a->k,
               "w8a8_gemm: operands must be 16-byte aligned with lda, ldb %% 16 == 0 and >= k");
  GemmParams p{};
  p.a = a->a; p.b = a->b; p.lda = a->lda; p.ldb = a->ldb;
  p.m = (int)a->m; p.n = (int)a->n; p.k = (int)a->k;
  p.row_scale = a->row_scale; p.col_scale = a->col_scale; p.col_stride = (int)a->col_scale_stride;
  p.bias_dtype = a->bias ? a->bias_dtype : 0; p.bias = a->bias;
  p.residual = reinterpret_cast<const uint16_t*>(a->residual); p.ldr = a->ldr;
  p.out = a->out; p.ldc = a->ldc;
  const int64_t tiles = ((a->m + kBM - 1) / kBM) * ((a->n + kBN - 1) / kBN);
  W8A8_REQUIRE(tiles < (1LL << 31), "w8a8_gemm: too many tiles");
  const dim3 grid((unsigned)tiles);
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  switch (a->epilogue) {
    case W8A8_EPI_INT32: hipLaunchKernelGGL((gemm_i8_256x256<kEpiInt32, kI32>), grid, dim3(256), 0, s, p); break;
    case W8A8_EPI_ROW: launch_gemm_out<kEpiRow>(a->out_dtype, p, grid, s); break;
    default: launch_gemm_out<kEpiColumn>(a->out_dtype, p, grid, s); break;
  }
  return launch_status("w8a8_gemm");
}

extern "C" int w8a8_dequantize(const W8A8DequantArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_dequantize: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8DequantArgs), "w8a8_dequantize: struct_size %u != %zu",
               a->struct_size, sizeof(W8A8DequantArgs));
  W8A8_REQUIRE(a->epilogue == W8A8_EPI_ROW || a->epilogue == W8A8_EPI_COLUMN,
               "w8a8_dequantize: epilogue must be ROW or COLUMN");
  W8A8_REQUIRE(a->m >= 0 && a->n >= 0 && a->m < (1LL << 31) && a->n < (1LL << 31), "w8a8_dequantize: bad shape");
  if (a->m == 0 || a->n == 0) return W8A8_OK;
  int rc = check_epilogue(a->epilogue, a->out_dtype, a->bias_dtype, a->bias, a->residual, a->ldr, a->n,
                          a->row_scale, a->col_scale, a->col_scale_stride, a->out, a->ldc);
  if (rc != W8A8_OK) return rc;
  W8A8_REQUIRE(a->acc && a->ldacc >= a->n, "w8a8_dequantize: null acc or ldacc < n");
  GemmParams p{};
  p.m = (int)a->m; p.n = (int)a->n;
  p.row_scale = a->row_scale; p.col_scale = a->col_scale; p.col_stride = (int)a->col_scale_stride;
  p.bias_dtype = a->bias ? a->bias_dtype : 0; p.bias = a->bias;
  p.residual = reinterpret_cast<const uint16_t*>(a->residual); p.ldr = a->ldr;
  p.out = a->out; p.ldc = a->ldc;
  const int64_t threads = a->m * ((a->n + 3) / 4);
  const dim3 grid((unsigned)((threads + 255) / 256));
  W8A8_REQUIRE((threads + 255) / 256 < (1LL << 31), "w8a8_dequantize: too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  if (a->epilogue == W8A8_EPI_ROW) launch_dequant_out<kEpiRow>(a->out_dtype, p, a->acc, a->ldacc, grid, s);
  else launch_dequant_out<kEpiColumn>(a->out_dtype, p, a->acc, a->ldacc, grid, s);
  return launch_status("w8a8_dequantize");
}
