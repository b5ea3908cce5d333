// Host-visible pieces of the INT8 GEMM: the kernel parameter block and the
// per-(epilogue, output dtype) launchers. The launchers are defined in
// gemm_kernels.h and instantiated one pair per object file by gemm_inst.hip;
// gemm_api.hip (the C ABI) only calls them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
  int cs_vec;       // col_scale has stride 1 and a 16-byte aligned base (float4 loads)
  int bias_dtype;   // 0 none, kF16, kF32
  const void* bias;
  const uint16_t* residual;
  int64_t ldr;
  const float* gate;      // DiT gate table [R, ldg] (with residual), or null
  const int32_t* labels;  // row -> gate-table row
  int64_t ldg;
  int gvec;               // gate rows allow float4 loads (16-byte base, ldg % 4 == 0)
  // RMS-RoPE epilogue (rope_heads > 0): output columns [0, 2 * rope_heads *
  // 128) are Q then K heads, normalized and rotated after the fp16 rounding.
  int rope_heads, rope_half, rope_rot, rope_f32, rope_pairs;
  float rope_eps;
  const void* rope_freqs;
  const float* rope_q_gain;
  const float* rope_k_gain;
  void* out;
  int64_t ldc;
  int vec_out;  // out rows allow 4-element vector stores (16-byte base, ldc % 4 == 0)
  int vec16;    // out (and residual) rows are 16-byte aligned: staged full-row stores
  // Split K (persistent kernel): ksplit workgroups share each output tile,
  // split s covering K stages [s*S/ksplit, (s+1)*S/ksplit) and writing its
  // partial tile at out + s * split_stride elements (1 / 0: no split).
  int ksplit;
  int64_t split_stride;
  // Caller's split-K workspace (may be null).
  void* ws;
  int64_t ws_bytes;
};

// Workspace of a split-K GEMM: the int32 partial planes (ksplit x m x n),
// which the finishing kernel adds (0 without a split).
inline int64_t split_partials_bytes(int64_t m, int64_t n, int ksplit) {
  return ksplit > 1 ? (int64_t)ksplit * m * n * 4 : 0;
}

// EPI: kEpiInt32 / kEpiRow / kEpiColumn; OUT: kI32 / kF16 / kBF16 / kF32.
template <int EPI, int OUT>
int launch_gemm(const GemmParams& p, hipStream_t s);

template <int EPI, int OUT>
void launch_dequant(const GemmParams& p, const int32_t* acc, int64_t ldacc, hipStream_t s);

// Split-K choice for an m x n x k GEMM on device dev: the number of K splits
// (1: none) and the workspace bytes it needs.
int gemm_ksplit(int64_t m, int64_t n, int64_t k, int dev, int64_t* workspace_bytes);

// Tile shape and K split of the persistent kernel: nb 4: 256 x 256, nb 3:
// 256 x 192, nb 2: 128 x 256 output tiles; K split ksplit ways.
struct GemmPlan {
  int nb;
  int ksplit;
};

inline int64_t plan_tiles(int64_t m, int64_t n, const GemmPlan& plan) {
  const int64_t bm = plan.nb == 2 ? 128 : 256, bn = plan.nb == 2 ? 256 : 64 * plan.nb;
  return ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
}

// The plan of least modelled time for an m x n x k GEMM (k a multiple of
// 128) on cus CUs, with at most max_split K splits. The cost is counted in
// K = 128 stages of a 256 x 256 tile (about 1 us on the power-limited
// clock): rounds of work items x (stages per item x the tile's relative
// cost + the tile's epilogue and the launch's fill and drain), plus the
// split partials' write-and-read traffic at about 6.5 TB/s. A 256 x 192
// stage costs 0.85 (0.80 of the cycles), a 128 x 256 stage 0.6 with an
// epilogue of 6 instead of 8: fitted to the fastest measured plan of eight
// shapes with M of 300..700 rows, where 256-row tiles leave most CUs idle
// or need large split partials. A plan replaces the one before it only
// when it is 10% faster (256 x 256 and unsplit first).
inline GemmPlan gemm_plan(int64_t m, int64_t n, int64_t k, int cus, int max_split = 8) {
  const int64_t kst = k / 128;
  GemmPlan best{4, 1};
  double best_t = -1.0;
  for (int nb = 4; nb >= 2; --nb) {
    const int64_t tiles = plan_tiles(m, n, GemmPlan{nb, 1});
    const double f = nb == 4 ? 1.0 : nb == 3 ? 0.85 : 0.6, e = nb == 2 ? 6.0 : 8.0;
    for (int ks = 1; ks <= max_split; ks *= 2) {
      if (ks > 1 && (tiles >= cus || kst / ks < 2)) break;
      const int64_t rounds = (tiles * ks + cus - 1) / cus;
      double t = (double)rounds * ((double)((kst + ks - 1) / ks) * f + e);
      if (ks > 1) t += (double)ks * m * n * 8 / 6.5e12 * 1e6;
      if (best_t < 0.0 || t < 0.9 * best_t) {
        best = GemmPlan{nb, ks};
        best_t = t;
      }
    }
  }
  return best;
}

// The int32 partial-sum pass of a split-K GEMM (the persistent kernel with
// the raw int32 epilogue, defined with the int32 instantiation).
int launch_gemm_partials(const GemmParams& p, const GemmPlan& plan, int dev, hipStream_t s);

}  // namespace w8a8
