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
#include <atomic>

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
  int vec_out;  // out rows allow 4-element vector stores (16-byte base, ldc % 4 == 0)
  int vec16;    // out (and residual) rows are 16-byte aligned: staged full-row stores
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
    if (valid == 4 && p.vec_out) {
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
      if (valid == 4 && p.vec_out) *reinterpret_cast<float4*>(o) = make_float4(y[0], y[1], y[2], y[3]);
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
      if (valid == 4 && p.vec_out) {
        *reinterpret_cast<uint2*>(o) =
            make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
      } else {
        for (int v = 0; v < valid; ++v) o[v] = h[v];
      }
    }
  }
}

// Epilogue of one wavefront's 128x128 quadrant: lane holds C[m][n..n+3]
// with m = mw + 16 mb + fr and n = nw + 16 nb + 4 fc for MFMA tile
// T = 8 nb + mb. Expanded by template recursion so every accumulator index is
// a constant and the accumulators never need addressable storage.
template <int EPI, int OUT, int T>
__device__ __forceinline__ void store_tiles(const GemmParams& p, v4i (&acc)[8][8], const float (&as)[8], int mw,
                                            int nw, int fr, int fc) {
  constexpr int NB = T / 8, MB = T % 8;
  const int n = nw + NB * 16 + 4 * fc;
  const int m = mw + MB * 16 + fr;
  const int valid = min(4, p.n - n);
  if (valid > 0 && m < p.m) {
    const int c[4] = {acc[NB][MB][0], acc[NB][MB][1], acc[NB][MB][2], acc[NB][MB][3]};
    epilogue4<EPI, OUT>(p, m, n, valid, c, as[MB]);
  }
  if constexpr (T + 1 < 64) store_tiles<EPI, OUT, T + 1>(p, acc, as, mw, nw, fr, fc);
}

template <int EPI, int OUT>
__device__ __forceinline__ void store_quadrant(const GemmParams& p, v4i (&acc)[8][8], int mw, int nw, int fr,
                                               int fc) {
  float as[8];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const int m = mw + mb * 16 + fr;
    as[mb] = (EPI != kEpiInt32 && m < p.m) ? p.row_scale[m] : 0.0f;
  }
  store_tiles<EPI, OUT, 0>(p, acc, as, mw, nw, fr, fc);
}

// The same for a 4x4 grid of 32x32 tiles (v_mfma_i32_32x32x32_i8 layout):
// lane (fr = lane % 32, fh = lane / 32) holds, for register group g = 0..3,
// C[m][n..n+3] with m = mw + 32 mb + fr and n = nw + 32 nb + 8 g + 4 fh.
template <int EPI, int OUT, int T>
__device__ __forceinline__ void store_tiles32(const GemmParams& p, v16i (&acc)[4][4], const float (&as)[4], int mw,
                                              int nw, int fr, int fh) {
  constexpr int NB = T / 16, MB = (T / 4) % 4, G = T % 4;
  const int n = nw + NB * 32 + 8 * G + 4 * fh;
  const int m = mw + MB * 32 + fr;
  const int valid = min(4, p.n - n);
  if (valid > 0 && m < p.m) {
    const int c[4] = {acc[NB][MB][4 * G], acc[NB][MB][4 * G + 1], acc[NB][MB][4 * G + 2], acc[NB][MB][4 * G + 3]};
    epilogue4<EPI, OUT>(p, m, n, valid, c, as[MB]);
  }
  if constexpr (T + 1 < 64) store_tiles32<EPI, OUT, T + 1>(p, acc, as, mw, nw, fr, fh);
}

template <int EPI, int OUT>
__device__ __forceinline__ void store_quadrant32(const GemmParams& p, v16i (&acc)[4][4], int mw, int nw, int fr,
                                                 int fh) {
  float as[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int m = mw + mb * 32 + fr;
    as[mb] = (EPI != kEpiInt32 && m < p.m) ? p.row_scale[m] : 0.0f;
  }
  store_tiles32<EPI, OUT, 0>(p, acc, as, mw, nw, fr, fh);
}

// Output element bits of one accumulator (storage dtype OUT; with a residual
// the FP16 branch is stored and the residual is added on write-out).
template <int EPI, int OUT>
__device__ __forceinline__ uint32_t out_bits(int c, float a, float w, float b, bool has_bias) {
  if constexpr (EPI == kEpiInt32) {
    return (uint32_t)c;
  } else {
    float y = dequant1<EPI>(c, a, w);
    if (has_bias) y = y + b;
    if constexpr (OUT == kF32) return __builtin_bit_cast(uint32_t, y);
    else if constexpr (OUT == kF16) return f2h(y);
    else return f2bf(y);
  }
}

// Staged epilogue of a full 128x128 quadrant: the wave writes its dequantized
// outputs into a private 32 KB LDS slice (rows of 128 elements, 16-byte
// chunks XOR-swizzled by row), then writes whole row segments to HBM with
// 16-byte stores (4 rows x 256 B per instruction for 2-byte outputs), adding
// the FP16 residual read with the same coalesced pattern. 4-byte outputs go
// in two passes of 64 rows. Requires a full tile and 16-byte aligned rows.
template <int EPI, int OUT>
__device__ __forceinline__ void store_quadrant32_staged(const GemmParams& p, v16i (&acc)[4][4],
                                                        const float (&wsc)[4][4][4], int mw, int nw, int lane,
                                                        int8_t* stage) {
  constexpr int ES = (OUT == kF16 || OUT == kBF16) ? 2 : 4;
  constexpr int RB = 128 * ES;          // bytes per quadrant row
  constexpr int CPR = RB / 16;          // 16-byte chunks per row
  constexpr int ROWS = 32768 / RB;      // rows per pass (128 or 64)
  constexpr int PASSES = 128 / ROWS;    // 1 or 2
  const int fr = lane & 31, fh = lane >> 5;
  const bool has_bias = EPI != kEpiInt32 && p.bias_dtype != 0;
  float as[4];
  float bsc[4][4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) as[mb] = EPI != kEpiInt32 ? p.row_scale[mw + mb * 32 + fr] : 0.0f;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) bsc[nb][g][v] = has_bias ? load_bias(p, nw + nb * 32 + 8 * g + 4 * fh + v) : 0.0f;
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    // Stage rows [pass * ROWS, pass * ROWS + ROWS) of the quadrant.
#pragma unroll
    for (int mbl = 0; mbl < 4 / PASSES; ++mbl) {
      const int mb = pass * (4 / PASSES) + mbl;
      const int row = mbl * 32 + fr;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint32_t bits[4];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            bits[v] = out_bits<EPI, OUT>(acc[nb][mb][4 * g + v], as[mb], wsc[nb][g][v], bsc[nb][g][v], has_bias);
          const int byte = (nb * 32 + 8 * g + 4 * fh) * ES;
          const int chunk = byte >> 4;
          int8_t* dst = stage + row * RB + ((chunk ^ (row & 15)) << 4) + (byte & 15);
          if constexpr (ES == 2)
            *reinterpret_cast<uint2*>(dst) = make_uint2(bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16));
          else
            *reinterpret_cast<uint4*>(dst) = make_uint4(bits[0], bits[1], bits[2], bits[3]);
        }
    }
    wave_lds_sync();
    // Write out: each instruction covers 64 chunks = 64 / CPR rows.
#pragma unroll 4
    for (int it = 0; it < ROWS * CPR / 64; ++it) {
      const int row = it * (64 / CPR) + lane / CPR;
      const int chunk = lane % CPR;
      const uint4 val = *reinterpret_cast<const uint4*>(stage + row * RB + ((chunk ^ (row & 15)) << 4));
      const int64_t m = mw + pass * ROWS + row;
      const int n = nw + chunk * (16 / ES);
      char* o = reinterpret_cast<char*>(p.out) + (m * p.ldc + n) * ES;
      if constexpr (OUT == kF16) {
        if (p.residual) {
          const uint4 r = *reinterpret_cast<const uint4*>(p.residual + m * p.ldr + n);
          const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
          const uint32_t bw[4] = {val.x, val.y, val.z, val.w};
          uint32_t ow[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint16_t lo = f2h(h2f((uint16_t)(rw[i] & 0xffffu)) + h2f((uint16_t)(bw[i] & 0xffffu)));
            const uint16_t hi = f2h(h2f((uint16_t)(rw[i] >> 16)) + h2f((uint16_t)(bw[i] >> 16)));
            ow[i] = (uint32_t)lo | ((uint32_t)hi << 16);
          }
          *reinterpret_cast<uint4*>(o) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
          continue;
        }
      }
      *reinterpret_cast<uint4*>(o) = val;
    }
    wave_lds_sync();
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

  store_quadrant<EPI, OUT>(p, acc, m0 + wm * 128, n0 + wn * 128, fr, fc);
}

// 256x256 tile fed by gfx950 direct global->LDS loads
// (global_load_lds_dwordx4) into a kStages-deep LDS ring: K steps kt+1 ..
// kt+kStages-2 stay in flight while step kt is multiplied, with no staging
// registers. Each wave instruction writes 1 KB of LDS (16 rows x 64 bytes);
// lane i fills physical chunk i % 4 of its row, so it loads the logical
// chunk that the XOR swizzle places there. Requires K % 64 == 0.
constexpr int kStages = 5;
constexpr int kStageBytes = 2 * kTileBytes;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  // s_waitcnt vmcnt(N) with expcnt and lgkmcnt left unconstrained.
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ void dma16(const int8_t* g, int8_t* l) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}

// Workgroup barrier without a memory fence: the DMA completion is awaited
// explicitly (vmcnt) before it, and the empty asm keeps the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int EPI, int OUT>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_i8_256x256_dma(GemmParams p) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (p.m + kBM - 1) / kBM, tiles_n = (p.n + kBN - 1) / kBN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;

  const int drow = lane >> 2;
  const int dchunk = (lane & 3) ^ chunk_swizzle(drow);
  const int8_t* src_a[4];
  const int8_t* src_b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = (wave * 4 + j) * 16 + drow;
    src_a[j] = p.a + (int64_t)min(m0 + row, p.m - 1) * p.lda + dchunk * 16;
    src_b[j] = p.b + (int64_t)min(n0 + row, p.n - 1) * p.ldb + dchunk * 16;
  }
  const int ktiles = p.k / kBK;
  auto issue = [&](int kt, int buf) {
    int8_t* st = smem + buf * kStageBytes + wave * 4 * 1024;
    const int kof = kt * kBK;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(src_a[j] + kof, st + j * 1024);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(src_b[j] + kof, st + kTileBytes + j * 1024);
  };

  // v_mfma_i32_32x32x32_i8: lane (r = lane % 32, h = lane / 32) supplies
  // row r, 16-byte K chunk 2 s + h of the K sub-step s (0, 1) for both
  // operands. Each wave holds a 4x4 grid of 32x32 accumulator tiles.
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, fh = lane >> 5;
  const int frag0 = fr * kBK + (((0 + fh) ^ chunk_swizzle(fr & 15)) << 4);
  const int frag1 = fr * kBK + (((2 + fh) ^ chunk_swizzle(fr & 15)) << 4);
  const int a_row = wm * 128 * kBK, b_row = wn * 128 * kBK;

  v16i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16i{};

  // Column scales of this lane's 64 output columns, fetched before the K loop
  // so the epilogue never waits on them.
  const int mw = m0 + wm * 128, nw = n0 + wn * 128;
  float wsc[4][4][4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int n = min(nw + nb * 32 + 8 * g + 4 * fh + v, p.n - 1);
        wsc[nb][g][v] = EPI != kEpiInt32 ? p.col_scale[(int64_t)n * p.col_stride] : 0.0f;
      }

  // Software pipeline over K steps. Stage s is DMA'd in the middle of step
  // s - 4 into the buffer step s - 5 used (every wave finished reading it
  // before that barrier). Within step kt: the MFMAs of sub-step 0 run while
  // sub-step 1's fragments are read; then the barrier that publishes stage
  // kt+1; then the MFMAs of sub-step 1 run while the fragments of step
  // kt+1's sub-step 0 are read. Past the last K step the DMA re-reads the
  // last stage into a buffer that is never consumed, so every step issues
  // exactly one stage and the vmcnt bounds are constant.
  auto read_frags = [&](int buf, int frag, v4i (&fa)[4], v4i (&fb)[4]) {
    const int8_t* sa = smem + buf * kStageBytes;
    const int8_t* sb = sa + kTileBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i] = *reinterpret_cast<const v4i*>(sb + b_row + frag + i * 32 * kBK);
      fb[i] = *reinterpret_cast<const v4i*>(sa + a_row + frag + i * 32 * kBK);
    }
  };
  auto mfma16 = [&](const v4i (&fa)[4], const v4i (&fb)[4]) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        acc[nb][mb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[nb], fb[mb], acc[nb][mb], 0, 0, 0);
  };
  // 16 MFMAs with 8 fragment reads spread between them.
  auto interleave = [&]() {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };

#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) issue(min(s, ktiles - 1), s);
  wait_vmcnt<8 * (kStages - 2)>();  // stage 0 landed (stages 1..3 in flight)
  block_barrier();
  v4i fa0[4], fb0[4], fa1[4], fb1[4];
  read_frags(0, frag0, fa0, fb0);
  int cur = 0;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int nxt = cur + 1 == kStages ? 0 : cur + 1;
    const int freeb = cur == 0 ? kStages - 1 : cur - 1;
    mfma16(fa0, fb0);
    read_frags(cur, frag1, fa1, fb1);
    interleave();
    wait_vmcnt<8 * (kStages - 3)>();  // stage kt+1 landed (kt+2, kt+3 in flight)
    block_barrier();
    issue(min(kt + kStages - 1, ktiles - 1), freeb);
    mfma16(fa1, fb1);
    read_frags(nxt, frag0, fa0, fb0);
    interleave();
    cur = nxt;
  }
  wait_vmcnt<0>();  // no DMA may still target this workgroup's LDS at exit
  if (p.vec16 && m0 + kBM <= p.m && n0 + kBN <= p.n) {
    block_barrier();  // every wave is done with the ring; reuse it for staging
    store_quadrant32_staged<EPI, OUT>(p, acc, wsc, mw, nw, lane, smem + wave * 32768);
  } else {
    store_quadrant32<EPI, OUT>(p, acc, mw, nw, fr, fh);
  }
}

// Skinny GEMM for M <= 64 (text-encoder decode / short prefill): weight
// streaming. A 512-thread workgroup owns NR weight rows (NR = 16 or 32); its
// 8 wavefronts split K into contiguous ranges and multiply with
// v_mfma_i32_16x16x64_i8 (weight rows as the MFMA A operand, up to four
// 16-row activation blocks as B), loading both operands straight from memory
// into registers, 4 K steps per batch so many loads are in flight. The 8
// partial sums meet in LDS; the shared epilogue writes the outputs. The
// activation rows (<= 64 x K) stay L2-resident across workgroups.
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyMaxMB = 4;
constexpr int kSkinnyU = 4;

template <int EPI, int OUT, int NR>
__global__ __launch_bounds__(512) void gemm_i8_skinny(GemmParams p) {
  constexpr int NB = NR / 16;
  __shared__ int red[kSkinnyWaves][NR][kSkinnyMaxMB * 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * NR;
  const int mblocks = (p.m + 15) >> 4;
  const int ksteps = p.k >> 6;
  const int per = (ksteps + kSkinnyWaves - 1) / kSkinnyWaves;
  const int s0 = min(wave * per, ksteps), s1 = min(s0 + per, ksteps);
  const int fr = lane & 15, fc = lane >> 4;

  const int8_t* wrow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) wrow[nb] = p.b + (int64_t)min(n0 + nb * 16 + fr, p.n - 1) * p.ldb + fc * 16;
  const int8_t* arow[kSkinnyMaxMB];
#pragma unroll
  for (int mb = 0; mb < kSkinnyMaxMB; ++mb) arow[mb] = p.a + (int64_t)min(mb * 16 + fr, p.m - 1) * p.lda + fc * 16;

  v4i acc[NB][kSkinnyMaxMB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < kSkinnyMaxMB; ++mb) acc[nb][mb] = v4i{0, 0, 0, 0};

  for (int s = s0; s < s1; s += kSkinnyU) {
    v4i wf[kSkinnyU][NB], af[kSkinnyU][kSkinnyMaxMB];
#pragma unroll
    for (int u = 0; u < kSkinnyU; ++u) {
      const int kof = min(s + u, s1 - 1) * 64;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) wf[u][nb] = *reinterpret_cast<const v4i*>(wrow[nb] + kof);
#pragma unroll
      for (int mb = 0; mb < kSkinnyMaxMB; ++mb)
        if (mb < mblocks) af[u][mb] = *reinterpret_cast<const v4i*>(arow[mb] + kof);
    }
#pragma unroll
    for (int u = 0; u < kSkinnyU; ++u) {
      if (s + u < s1) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mb = 0; mb < kSkinnyMaxMB; ++mb)
            if (mb < mblocks)
              acc[nb][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[u][nb], af[u][mb], acc[nb][mb], 0, 0, 0);
      }
    }
  }
  // Lane holds C[m][n..n+3] for m = 16 mb + fr, n = 16 nb + 4 fc (local).
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < kSkinnyMaxMB; ++mb)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][nb * 16 + 4 * fc + v][mb * 16 + fr] = acc[nb][mb][v];
  __syncthreads();
  // Thread -> (m, 4 consecutive n): sum the 8 partials, then the epilogue.
  for (int idx = tid; idx < p.m * (NR / 4); idx += 512) {
    const int m = idx / (NR / 4);
    const int nl = (idx % (NR / 4)) * 4;
    const int n = n0 + nl;
    const int valid = min(4, p.n - n);
    if (valid <= 0) continue;
    int c[4] = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < kSkinnyWaves; ++w)
#pragma unroll
      for (int v = 0; v < 4; ++v) c[v] += red[w][nl + v][m];
    const float a = EPI != kEpiInt32 ? p.row_scale[m] : 0.0f;
    epilogue4<EPI, OUT>(p, m, n, valid, c, a);
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
  const int es = out_dtype == W8A8_F16 || out_dtype == W8A8_BF16 ? 2 : 4;
  W8A8_REQUIRE(((uintptr_t)out % es) == 0 && ldc >= n, "out must be element-aligned with ldc >= n");
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
    W8A8_REQUIRE(((uintptr_t)residual & 1u) == 0 && ldr >= n, "residual must be 2-byte aligned with ldr >= n");
  }
  return W8A8_OK;
}

// The DMA kernel's LDS ring exceeds the 64 KB default: raise the kernel's
// dynamic LDS limit once per device (an idempotent per-device record).
template <int EPI, int OUT>
static int enable_dma_lds() {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("w8a8_gemm: hipGetDevice failed");
    return W8A8_ERR_LAUNCH;
  }
  const uint64_t bit = 1ull << dev;
  if (done.load(std::memory_order_acquire) & bit) return W8A8_OK;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_i8_256x256_dma<EPI, OUT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kStages * kStageBytes);
  if (e != hipSuccess) {
    set_error("w8a8_gemm: cannot enable %d bytes of LDS: %s", kStages * kStageBytes, hipGetErrorString(e));
    return W8A8_ERR_LAUNCH;
  }
  done.fetch_or(bit, std::memory_order_acq_rel);
  return W8A8_OK;
}

template <int EPI, int OUT>
static int launch_tile(const GemmParams& p, dim3 grid, hipStream_t s) {
  if (p.k % kBK == 0) {
    const int rc = enable_dma_lds<EPI, OUT>();
    if (rc != W8A8_OK) return rc;
    hipLaunchKernelGGL((gemm_i8_256x256_dma<EPI, OUT>), grid, dim3(256), kStages * kStageBytes, s, p);
  } else {
    hipLaunchKernelGGL((gemm_i8_256x256<EPI, OUT>), grid, dim3(256), 0, s, p);
  }
  return W8A8_OK;
}

template <int EPI, int OUT>
static int launch_tile_or_skinny(const GemmParams& p, dim3 grid, hipStream_t s) {
  if (p.m <= kSkinnyMaxMB * 16 && p.k % 64 == 0) {
    // 32 weight rows per workgroup while that still fills 256 workgroups.
    if (p.n / 32 >= 256) {
      hipLaunchKernelGGL((gemm_i8_skinny<EPI, OUT, 32>), dim3((unsigned)((p.n + 31) / 32)), dim3(512), 0, s, p);
    } else {
      hipLaunchKernelGGL((gemm_i8_skinny<EPI, OUT, 16>), dim3((unsigned)((p.n + 15) / 16)), dim3(512), 0, s, p);
    }
    return W8A8_OK;
  }
  return launch_tile<EPI, OUT>(p, grid, s);
}

template <int EPI>
static int launch_gemm_out(int out, const GemmParams& p, dim3 grid, hipStream_t s) {
  switch (out) {
    case kF16: return launch_tile_or_skinny<EPI, kF16>(p, grid, s);
    case kBF16: return launch_tile_or_skinny<EPI, kBF16>(p, grid, s);
    default: return launch_tile_or_skinny<EPI, kF32>(p, grid, s);
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
  p.vec_out = aligned16(a->out) && a->ldc % 4 == 0;
  {
    const int es = (a->out_dtype == W8A8_F16 || a->out_dtype == W8A8_BF16) ? 2 : 4;
    p.vec16 = aligned16(a->out) && (a->ldc * es) % 16 == 0 &&
              (a->residual == nullptr || (aligned16(a->residual) && a->ldr % 8 == 0));
  }
  const int64_t tiles = ((a->m + kBM - 1) / kBM) * ((a->n + kBN - 1) / kBN);
  W8A8_REQUIRE(tiles < (1LL << 31), "w8a8_gemm: too many tiles");
  const dim3 grid((unsigned)tiles);
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  int rc2;
  switch (a->epilogue) {
    case W8A8_EPI_INT32: rc2 = launch_tile_or_skinny<kEpiInt32, kI32>(p, grid, s); break;
    case W8A8_EPI_ROW: rc2 = launch_gemm_out<kEpiRow>(a->out_dtype, p, grid, s); break;
    default: rc2 = launch_gemm_out<kEpiColumn>(a->out_dtype, p, grid, s); break;
  }
  if (rc2 != W8A8_OK) return rc2;
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
  p.vec_out = aligned16(a->out) && a->ldc % 4 == 0;
  const int64_t threads = a->m * ((a->n + 3) / 4);
  const dim3 grid((unsigned)((threads + 255) / 256));
  W8A8_REQUIRE((threads + 255) / 256 < (1LL << 31), "w8a8_dequantize: too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  if (a->epilogue == W8A8_EPI_ROW) launch_dequant_out<kEpiRow>(a->out_dtype, p, a->acc, a->ldacc, grid, s);
  else launch_dequant_out<kEpiColumn>(a->out_dtype, p, a->acc, a->ldacc, grid, s);
  return launch_status("w8a8_dequantize");
}
