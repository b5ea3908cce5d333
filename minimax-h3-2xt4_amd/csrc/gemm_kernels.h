// INT8 GEMM kernels on gfx950 i8 MFMA with a fused dequantization / bias /
// residual epilogue, the skinny-M weight-streaming GEMM and the standalone
// epilogue. Included only by gemm_inst.hip, which instantiates one
// (epilogue, output dtype) pair per object file so the variants compile in
// parallel.
//
// C[m][n] = sum_k A[m][k] * B[n][k], A = activations [M,K], B = weights
// [N,K], both K-contiguous. The MFMA's A operand is the weight tile and its B
// operand the activation tile, so each lane ends with four consecutive
// output columns of one row.
#pragma once

#include <atomic>
#include <type_traits>

#include "gemm_launch.h"
#include "w8a8_device.h"

namespace w8a8 {

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kTileBytes = kBM * kBK;  // one operand tile per K step

// 16-byte chunk swizzle of LDS row r (depends on r & 15 only): the 16 lanes
// reading one fragment column of 64-byte rows hit distinct banks.
__device__ __forceinline__ int chunk_swizzle(int r) {
  return (((r >> 1) ^ (r >> 3)) & 1) | (((r >> 2) & 1) << 1);
}

// Grouped raster: logical tile pid -> (tm, tn), walking groups of 8
// row-tiles column by column so neighbouring pids share A and B rows.
__device__ __forceinline__ void raster(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int kGroupM = 8;
  const int group = kGroupM * tiles_n;
  const int first_m = (pid / group) * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in = pid - (pid / group) * group;
  tm = first_m + in % gsize;
  tn = in / gsize;
}

// One workgroup per tile (the register-staged fallback): consecutive
// workgroup ids are dispatched round-robin over the 8 XCDs, so remap them
// to give each XCD a contiguous range of the raster.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  raster(pid, tiles_m, tiles_n, tm, tn);
}

__device__ __forceinline__ float load_bias(const GemmParams& p, int n) {
  if (p.bias_dtype == kF16) return h2f(reinterpret_cast<const uint16_t*>(p.bias)[n]);
  if (p.bias_dtype == kF32) return reinterpret_cast<const float*>(p.bias)[n];
  return 0.0f;
}

// Epilogue of four consecutive columns n..n+3 of row m (valid of them in
// range). Shared by the unstaged GEMM epilogues, the skinny GEMM and the
// standalone dequantize.
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
          const float* gr = p.gate ? p.gate + (int64_t)p.labels[m] * p.ldg + n : nullptr;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float branch = h2f(f2h_of_f32(y[v]));
            const float res = v < valid ? h2f(r[v]) : 0.0f;
            h[v] = gr ? f2h_of_f32(__builtin_fmaf(branch, gr[v < valid ? v : 0], res)) : f2h(res + branch);
          }
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) h[v] = f2h_of_f32(y[v]);
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

// Epilogue of one wavefront's 128x128 quadrant in the 16x16 MFMA layout:
// lane holds C[m][n..n+3] with m = mw + 16 mb + fr and n = nw + 16 nb + 4 fc
// for MFMA tile T = 8 nb + mb. Expanded by template recursion so every
// accumulator index is a constant and the accumulators never need
// addressable storage.
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
// Used for partial tiles at the matrix edge.
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
    else if constexpr (OUT == kF16) return f2h_of_f32(y);
    else return f2bf(y);
  }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  // s_waitcnt vmcnt(N) with expcnt and lgkmcnt left unconstrained.
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt vmcnt(0) lgkmcnt(0): every vector-memory access of this wave
// (LDS DMA included) completed and every LDS access returned.
__device__ __forceinline__ void wait_vm_lgkm() { __builtin_amdgcn_s_waitcnt(0x7 << 4); }

// s_waitcnt vmcnt(N) lgkmcnt(0).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

// s_waitcnt lgkmcnt(0) alone.
__device__ __forceinline__ void wait_lgkm() { __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4)); }

// Compile-time epilogue options of the persistent kernel (each variant
// carries only the loads it uses).
enum EpilogueFlags { kWithBias = 1, kWithResidual = 2, kWithGate = 4, kWithRope = 8 };

// Layout of the staged epilogue's read-out: a lane owns CPL consecutive
// columns of a 64-column half of the quadrant (8 for 2-byte outputs, 4 for
// 4-byte outputs: one 16-byte store either way) and LPR lanes cover a row.
template <int OUT>
struct Readout {
  static constexpr int ES = (OUT == kF16 || OUT == kBF16) ? 2 : 4;
  static constexpr int CPL = 16 / ES;
  static constexpr int LPR = 64 / CPL;
  static constexpr int RPI = 64 / LPR;  // rows per wave store
  static constexpr int ITERS = 32 / RPI;
};

// Column scales (and biases) of the columns a lane writes in the staged
// epilogue: half h (0, 1) of the quadrant, columns
// nw + 64 h + (lane % LPR) * CPL + [0, CPL).
template <int OUT>
__device__ __forceinline__ int readout_col(int nw, int h, int lane) {
  using R = Readout<OUT>;
  return nw + 64 * h + (lane % R::LPR) * R::CPL;
}

// Staged epilogue of one 128 x 32 NB quadrant (NB = 4, 3 or 2) through an
// 8 KB wave-private LDS slice, in passes of 32 rows x 64 columns (8, or 4
// for NB = 2). Each pass writes the raw int32 accumulators into the slice
// (16-byte chunks XOR-swizzled by row), then
// each lane reads CPL consecutive columns of one row back, dequantizes them
// in the reference's order (ROW (C*a)*w, COLUMN C*(a*w), then + bias, then
// the cast), adds the FP16 residual read with the same coalesced pattern
// and writes 16 bytes. The row scale comes from the lane that holds it in
// the MFMA layout; wsc and bsc hold the column scales and biases of the
// lane's read-out columns (readout_col). Rows past m and columns past n are
// masked, and rows that are not 16-byte aligned (vec16 == 0) or straddle n
// are written element by element. A wave's LDS accesses execute in order,
// so the passes need only compiler ordering between the slice writes and
// reads, and the next pass's writes may issue before this pass's reads
// return.
template <int EPI, int OUT, int FLAGS, bool INTERIOR, int NB = 4>
__device__ __forceinline__ void store_quadrant32_passes(const GemmParams& p, v16i (&acc)[NB][4],
                                                        const float (&wsc)[2][8], const float (&bsc)[2][8],
                                                        const float (&as)[4], const int (&lbl)[4], int mw, int nw,
                                                        int lane, int8_t* stage, int64_t out_off) {
  using R = Readout<OUT>;
  constexpr int RB = 256;  // 64 int32 per staged row
  constexpr bool has_bias = (FLAGS & kWithBias) != 0;
  constexpr bool has_res = (FLAGS & kWithResidual) != 0;
  constexpr bool has_gate = (FLAGS & kWithGate) != 0;
  const int fr = lane & 31, fh = lane >> 5;
  const int orow = lane / R::LPR, ocol = (lane % R::LPR) * R::CPL;
  // The FP16 residual rows of pass `pass` (this lane's read-out columns).
  // Without the gate, pass + 1's rows are loaded while pass is dequantized,
  // so their latency is hidden; the gate variants have no registers to spare
  // for a second set and load each pass's rows at its start.
  auto load_res = [&](int pass, uint4 (&rr)[R::ITERS]) {
    const int mb = pass >> 1, h = pass & 1;
    const int mrow = mw + mb * 32;
    const int ncol = nw + 64 * h + ocol;
    const bool in_quad = NB != 3 || h == 0 || ocol < 32;
    const bool full_cols = INTERIOR || (p.vec16 && ncol + R::CPL <= p.n);
#pragma unroll
    for (int it = 0; it < R::ITERS; ++it) {
      const int m = mrow + it * R::RPI + orow;
      const uint16_t* r = p.residual + (int64_t)m * p.ldr + ncol;
      if (!in_quad) {
        rr[it] = make_uint4(0, 0, 0, 0);
      } else if (INTERIOR || (m < p.m && full_cols)) {
        rr[it] = *reinterpret_cast<const uint4*>(r);
      } else {
        uint32_t w[4] = {0, 0, 0, 0};
        if (m < p.m) {
#pragma unroll
          for (int j = 0; j < R::CPL; ++j)
            if (ncol + j < p.n) w[j >> 1] |= (uint32_t)r[j] << (16 * (j & 1));
        }
        rr[it] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  };
  constexpr bool kResAhead = has_res && !has_gate;
  uint4 rbuf[2][R::ITERS];
  if constexpr (kResAhead) load_res(0, rbuf[0]);
#pragma unroll
  for (int pass = 0; pass < 8; ++pass) {
    const int mb = pass >> 1, h = pass & 1;
    // A quadrant 64 columns wide (NB == 2) has no second half.
    if (NB == 2 && h == 1) continue;
    const int mrow = mw + mb * 32;
    const int ncol = nw + 64 * h + ocol;
    // A quadrant 96 columns wide (NB == 3) has only its first 32 in the
    // second half: the other read-out lanes of those passes store nothing.
    const bool in_quad = NB != 3 || h == 0 || ocol < 32;
    // INTERIOR: every row and column of the quadrant is inside the output
    // and rows are 16-byte aligned, so no store needs a mask.
    const bool full_cols = INTERIOR || (p.vec16 && ncol + R::CPL <= p.n);
    // Buffer of pass q: the parity of its index among the passes that run
    // (NB == 2 runs every other pass).
    auto buf_of = [](int q) { return NB == 2 ? (q >> 1) & 1 : q & 1; };
    if constexpr (kResAhead) {
      const int next = NB == 2 ? pass + 2 : pass + 1;
      if (next < 8) load_res(next, rbuf[buf_of(next)]);
    } else if constexpr (has_res) {
      load_res(pass, rbuf[0]);
    }
    const uint4 (&rres)[R::ITERS] = rbuf[kResAhead ? buf_of(pass) : 0];
    // Gate values of the lane's columns for each of its rows (the row's
    // table row comes from the lane holding its label in the MFMA layout).
    // Gate values of the lane's columns for table row `label`.
    auto load_gate = [&](int label, float (&gv)[R::CPL]) {
      const float* gr = p.gate + (int64_t)label * p.ldg;
      if (!in_quad) {
#pragma unroll
        for (int j = 0; j < R::CPL; ++j) gv[j] = 0.0f;
      } else if (p.gvec && full_cols) {
#pragma unroll
        for (int q = 0; q < R::CPL / 4; ++q) {
          const float4 g4 = *reinterpret_cast<const float4*>(gr + ncol + 4 * q);
          gv[4 * q] = g4.x; gv[4 * q + 1] = g4.y; gv[4 * q + 2] = g4.z; gv[4 * q + 3] = g4.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < R::CPL; ++j) gv[j] = gr[min(ncol + j, p.n - 1)];
      }
    };
    // The 32 rows of a pass almost always share one gate label (the DiT's
    // segments are whole frames), and then one table row serves the whole
    // pass: the lane's CPL values, loaded once. Otherwise each read-out row
    // loads its own (the row's label comes from the lane holding it in the
    // MFMA layout).
    float gv[R::CPL];
    bool gate_one = true;
    if constexpr (has_gate) {
      const int lab0 = __shfl(lbl[mb], 0, 64);
      gate_one = __builtin_amdgcn_ballot_w64(lbl[mb] != lab0) == 0;
      if (gate_one) load_gate(lab0, gv);
    }
    // acc[nb][mb] group g holds columns 32 nb + 8 g + 4 fh + [0, 4) of row fr.
#pragma unroll
    for (int nbl = 0; nbl < 2; ++nbl)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nb = min(2 * h + nbl, NB - 1);
        if (NB == 4 || 2 * h + nbl < NB) {
          const int chunk = nbl * 8 + 2 * g + fh;
          *reinterpret_cast<v4i*>(stage + fr * RB + ((chunk ^ (fr & 15)) << 4)) =
              v4i{acc[nb][mb][4 * g], acc[nb][mb][4 * g + 1], acc[nb][mb][4 * g + 2], acc[nb][mb][4 * g + 3]};
        }
      }
    asm volatile("" ::: "memory");
    // Row scales of the lane's read-out rows (from the lanes holding them in
    // the MFMA layout), issued with the slice reads so one wait covers both.
    float arow[R::ITERS];
#pragma unroll
    for (int it = 0; it < R::ITERS; ++it) arow[it] = EPI != kEpiInt32 ? __shfl(as[mb], it * R::RPI + orow, 64) : 0.0f;
    int c[R::ITERS][R::CPL];
#pragma unroll
    for (int it = 0; it < R::ITERS; ++it) {
      const int row = it * R::RPI + orow;
#pragma unroll
      for (int q = 0; q < R::CPL / 4; ++q) {
        const int chunk = ocol / 4 + q;
        const v4i v = *reinterpret_cast<const v4i*>(stage + row * RB + ((chunk ^ (row & 15)) << 4));
        c[it][4 * q] = v[0]; c[it][4 * q + 1] = v[1]; c[it][4 * q + 2] = v[2]; c[it][4 * q + 3] = v[3];
      }
    }
    asm volatile("" ::: "memory");  // the next pass's writes stay behind these reads
#pragma unroll
    for (int it = 0; it < R::ITERS; ++it) {
      const int row = it * R::RPI + orow;
      const int m = mrow + row;
      const float a = arow[it];
      // words[i]: output elements 2 i, 2 i + 1 (2-byte outputs) or element i.
      uint32_t words[4];
      if constexpr (OUT == kF16) {
        // FP16 pairs convert in packed instructions, the row's eight values
        // behind one opaque step; with a residual the rounded branch is
        // widened again, added and rounded the same way.
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          y[j] = dequant1<EPI>(c[it][j], a, wsc[h][j]);
          if constexpr (has_bias) y[j] = y[j] + bsc[h][j];
        }
        f2h8_of_f32(y, words);
        if constexpr (has_res) {
          if constexpr (has_gate) {
            if (!gate_one) load_gate(__shfl(lbl[mb], row, 64), gv);
          }
          const uint32_t rw[4] = {rres[it].x, rres[it].y, rres[it].z, rres[it].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float r0 = h2f((uint16_t)(rw[i] & 0xffffu)), r1 = h2f((uint16_t)(rw[i] >> 16));
            const float b0 = h2f((uint16_t)(words[i] & 0xffffu)), b1 = h2f((uint16_t)(words[i] >> 16));
            if constexpr (has_gate) {
              y[2 * i] = __builtin_fmaf(b0, gv[2 * i], r0);
              y[2 * i + 1] = __builtin_fmaf(b1, gv[2 * i + 1], r1);
            } else {
              y[2 * i] = r0 + b0;
              y[2 * i + 1] = r1 + b1;
            }
          }
          f2h8_of_f32(y, words);
        }
      } else {
        uint32_t bits[R::CPL];
#pragma unroll
        for (int j = 0; j < R::CPL; ++j)
          bits[j] = out_bits<EPI, OUT>(c[it][j], a, wsc[h][j], bsc[h][j], has_bias);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (R::ES == 2) words[i] = bits[2 * i] | (bits[2 * i + 1] << 16);
          else words[i] = bits[i];
        }
      }
      char* o = reinterpret_cast<char*>(p.out) + (out_off + (int64_t)m * p.ldc + ncol) * R::ES;
      if (!in_quad) {
      } else if (INTERIOR || (m < p.m && full_cols)) {
        // Streaming store: the output is not read again by this kernel, so it
        // should not push the operand lines out of L2.
        __builtin_nontemporal_store(v4i{(int)words[0], (int)words[1], (int)words[2], (int)words[3]},
                                    reinterpret_cast<v4i*>(o));
      } else if (!INTERIOR && m < p.m) {
#pragma unroll
        for (int j = 0; j < R::CPL; ++j) {
          if (ncol + j < p.n) {
            if constexpr (R::ES == 2) reinterpret_cast<uint16_t*>(o)[j] = (uint16_t)(words[j >> 1] >> (16 * (j & 1)));
            else reinterpret_cast<uint32_t*>(o)[j] = words[j];
          }
        }
      }
    }
  }
}

// Column scales (wsc[0]) and RMS gains (wsc[1]) of the columns a lane
// handles in the RMS-RoPE epilogue: nw + 8 (lane % 16) + [0, 8). The gains
// are Q's below heads * 128 columns, K's below 2 * heads * 128, and unused
// in the V columns past them.
template <int EPI>
__device__ __forceinline__ void load_rope_scales(const GemmParams& p, int nw, int lane, float (&wsc)[2][8]) {
  const int d0 = 8 * (lane & 15), width = p.rope_heads * 128;
#pragma unroll
  for (int j = 0; j < 8; ++j) wsc[0][j] = p.col_scale[(int64_t)min(nw + d0 + j, p.n - 1) * p.col_stride];
  if (nw < 2 * width) {
    const float4* g = reinterpret_cast<const float4*>((nw < width ? p.rope_q_gain : p.rope_k_gain) + d0);
    const float4 g0 = g[0], g1 = g[1];
    wsc[1][0] = g0.x; wsc[1][1] = g0.y; wsc[1][2] = g0.z; wsc[1][3] = g0.w;
    wsc[1][4] = g1.x; wsc[1][5] = g1.y; wsc[1][6] = g1.z; wsc[1][7] = g1.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) wsc[1][j] = 0.0f;
  }
}

// Rotation matrix entries of the lane's eight elements d0 .. d0 + 7 of one
// row: element d (pair p = d mod half, side s = d div half) is multiplied by
// F[p][s][s] (diag) and its partner by F[p][s][1 - s] (offd). half % 8 == 0,
// so the eight elements are on one side and use the consecutive pairs
// p0 .. p0 + 7, a 16-byte aligned block of the row's table. (Four 16-byte
// loads and selects beat eight 4-byte loads of just the side's words: the
// epilogue is bound by the number of memory instructions.)
// PAIRS: the table row holds, per side s and pair p, (F[p][s][s],
// F[p][s][1 - s]), so the lane's sixteen values are one contiguous run
// (two 16-byte loads for fp16, no selects).
template <int FQ, bool PAIRS>
__device__ __forceinline__ void load_rope_freqs(const void* frow, int p0, int side, int half, float (&diag)[8],
                                                float (&offd)[8]) {
  if constexpr (PAIRS) {
    const int first = 2 * (side * half + p0);
    if constexpr (FQ == kF32) {
      const float4* f = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(frow) + first);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 v = f[k];
        diag[2 * k] = v.x; offd[2 * k] = v.y; diag[2 * k + 1] = v.z; offd[2 * k + 1] = v.w;
      }
    } else {
      const uint4* f = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(frow) + first);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint4 u = f[k];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          diag[4 * k + q] = h2f((uint16_t)(w[q] & 0xffffu));
          offd[4 * k + q] = h2f((uint16_t)(w[q] >> 16));
        }
      }
    }
  } else if constexpr (FQ == kF32) {
    const float* f = reinterpret_cast<const float*>(frow) + 4 * p0 + 2 * side;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float2 v = *reinterpret_cast<const float2*>(f + 4 * i);   // F[p][s][0], F[p][s][1]
      diag[i] = side ? v.y : v.x;
      offd[i] = side ? v.x : v.y;
    }
  } else {
    const uint4* f = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(frow) + 4 * p0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint4 u = f[k];   // pairs p0 + 2 k, p0 + 2 k + 1
      const uint32_t w[2] = {side ? u.y : u.x, side ? u.w : u.z};
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const float lo = h2f((uint16_t)(w[q] & 0xffffu)), hi = h2f((uint16_t)(w[q] >> 16));
        diag[2 * k + q] = side ? hi : lo;
        offd[2 * k + q] = side ? lo : hi;
      }
    }
  }
}

// RMS-RoPE epilogue of one 128x128 quadrant (FP16 output, no split) that is
// one 128-column head of Q (nw < heads * 128) or of K (nw < 2 * heads *
// 128); V quadrants take the plain staged epilogue. In 8 passes of 16 rows the
// lanes holding those rows in the MFMA layout write their raw accumulators
// to the wave's 8 KB LDS slice (16-byte chunks XOR-swizzled by row); lane
// (rq, t) = (lane / 16, lane % 16) then reads columns 8 t .. 8 t + 7 of rows
// 4 it + rq (it = 0..3), dequantizes and rounds them to FP16 exactly as the
// plain GEMM output, and for a Q or K head continues as the standalone
// RMS-RoPE kernel does on that FP16 output: the sum of squares of the row's
// 128 values (each lane's eight in order, then an xor butterfly over the 16
// lanes of the row, offsets 8, 4, 2, 1), 1 / sqrt(sum * 2^-7 + eps), the
// gain, and the rotation with the partner element, read back from the
// slice after the normalized values replace the accumulators there. Rows
// past m are not stored (their rotation matrices are those of row m - 1).
template <int EPI, int FQ, bool PAIRS>
__device__ __forceinline__ void store_quadrant_rope(const GemmParams& p, v16i (&acc)[4][4], const float (&wsc)[2][8],
                                                    const float (&as)[4], int mw, int nw, int lane, int8_t* stage) {
  constexpr int RB = 512;   // 128 four-byte values per staged row
  constexpr int FES = FQ == kF32 ? 4 : 2;
  const int fr = lane & 31, fh = lane >> 5;
  const int rq = lane >> 4, t = lane & 15;
  const int d0 = 8 * t, half = p.rope_half;
  const bool rotated = d0 < p.rope_rot;
  const int side0 = d0 >= half ? 1 : 0;
  const int p0 = d0 - side0 * half;
  const int other0 = side0 ? d0 - half : d0 + half;
  const int ncol = nw + d0;
  uint16_t* const out = reinterpret_cast<uint16_t*>(p.out);
#pragma unroll
  for (int pass = 0; pass < 8; ++pass) {   // unrolled: acc is indexed by pass
    const int mb = pass >> 1, hh = pass & 1;
    const int mrow = mw + mb * 32 + 16 * hh;
    // acc[nb][mb] group g holds columns 32 nb + 8 g + 4 fh + [0, 4) of row fr.
    if ((fr >> 4) == hh) {
      const int r = fr & 15;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int chunk = 8 * nb + 2 * g + fh;
          *reinterpret_cast<v4i*>(stage + r * RB + ((chunk ^ r) << 4)) =
              v4i{acc[nb][mb][4 * g], acc[nb][mb][4 * g + 1], acc[nb][mb][4 * g + 2], acc[nb][mb][4 * g + 3]};
        }
    }
    asm volatile("" ::: "memory");
    float arow[4];
    int c[4][8];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int r = 4 * it + rq;
      arow[it] = __shfl(as[mb], 16 * hh + r, 64);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const v4i v = *reinterpret_cast<const v4i*>(stage + r * RB + (((2 * t + q) ^ r) << 4));
        c[it][4 * q] = v[0]; c[it][4 * q + 1] = v[1]; c[it][4 * q + 2] = v[2]; c[it][4 * q + 3] = v[3];
      }
    }
    asm volatile("" ::: "memory");  // the slice's next writes stay behind these reads
    // y: the plain GEMM's FP16 outputs, widened. Sum of squares: y * y is
    // exact in fp32, so fma(y, y, ss) rounds once, like ss + y * y.
    float y[4][8], ss[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      ss[it] = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = f2h2_of_f32(dequant1<EPI>(c[it][2 * i], arow[it], wsc[0][2 * i]),
                                       dequant1<EPI>(c[it][2 * i + 1], arow[it], wsc[0][2 * i + 1]));
        y[it][2 * i] = h2f((uint16_t)(w & 0xffffu));
        y[it][2 * i + 1] = h2f((uint16_t)(w >> 16));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss[it] = __builtin_fmaf(y[it][j], y[it][j], ss[it]);
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) ss[it] = ss[it] + __shfl_xor(ss[it], off, 64);
    }
    // Each row's 1 / sqrt once: lane t of group rq takes row 4 (t % 4) + rq,
    // then every lane fetches its four rows' values.
    const int mine = t & 3;
    const float ssm = mine == 0 ? ss[0] : mine == 1 ? ss[1] : mine == 2 ? ss[2] : ss[3];
    const float invm = 1.0f / __builtin_sqrtf(ssm * 0.0078125f + p.rope_eps);
    float nv[4][8];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const float inv = __shfl(invm, (lane & 48) | it, 64);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float s1 = y[it][j] * inv;
        nv[it][j] = s1 * wsc[1][j];
      }
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int r = 4 * it + rq;
#pragma unroll
      for (int q = 0; q < 2; ++q)
        *reinterpret_cast<float4*>(stage + r * RB + (((2 * t + q) ^ r) << 4)) =
            make_float4(nv[it][4 * q], nv[it][4 * q + 1], nv[it][4 * q + 2], nv[it][4 * q + 3]);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int r = 4 * it + rq;
      const int m = mrow + r;
      float o[8];
      if (rotated) {
        float part[8], diag[8], offd[8];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const float4 v = *reinterpret_cast<const float4*>(stage + r * RB + (((other0 / 4 + q) ^ r) << 4));
          part[4 * q] = v.x; part[4 * q + 1] = v.y; part[4 * q + 2] = v.z; part[4 * q + 3] = v.w;
        }
        const char* frow = reinterpret_cast<const char*>(p.rope_freqs) + (int64_t)min(m, p.m - 1) * half * 4 * FES;
        load_rope_freqs<FQ, PAIRS>(frow, p0, side0, half, diag, offd);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float a = nv[it][j] * diag[j];
          o[j] = __builtin_fmaf(part[j], offd[j], a);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = nv[it][j];
      }
      if (m < p.m) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = f2h2_of_f32(o[2 * i], o[2 * i + 1]);
        *reinterpret_cast<uint4*>(out + (int64_t)m * p.ldc + ncol) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
    asm volatile("" ::: "memory");  // the next pass's slice writes stay behind these reads
  }
}

// Register-staged 256x256 tile with v_mfma_i32_16x16x64_i8 and a two-buffer
// LDS pipeline; the fallback for K % 64 != 0 (K tail loads are zero-filled).
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

// Column scales and raw bias bits of the lane's read-out columns
// (readout_col) for both halves of the quadrant at column offset nw:
// clamped loads (columns past n are never written) whose registers stay
// untouched until the epilogue, so no wait for them lands in the K loop.
template <int EPI, int OUT, bool BIAS>
__device__ __forceinline__ void load_readout_scales(const GemmParams& p, int nw, int lane, float (&wsc)[2][8],
                                                    uint32_t (&braw)[2][8]) {
  using R = Readout<OUT>;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      braw[h][j] = 0;
      if constexpr (EPI == kEpiInt32) {
        wsc[h][j] = 0.0f;
      } else {
        const int n = min(readout_col<OUT>(nw, h, lane) + j, p.n - 1);
        wsc[h][j] = j < R::CPL ? p.col_scale[(int64_t)n * p.col_stride] : 0.0f;
      }
    }
  if constexpr (EPI != kEpiInt32 && BIAS) {
    if (p.bias_dtype == kF16) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < R::CPL; ++j)
          braw[h][j] = reinterpret_cast<const uint16_t*>(p.bias)[min(readout_col<OUT>(nw, h, lane) + j, p.n - 1)];
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < R::CPL; ++j)
          braw[h][j] = reinterpret_cast<const uint32_t*>(p.bias)[min(readout_col<OUT>(nw, h, lane) + j, p.n - 1)];
    }
  }
}

// Persistent GEMM (256 x 256, 256 x 192 or 128 x 256 output tiles) fed by
// gfx950 direct global->LDS loads (global_load_lds_dwordx4). One workgroup
// per CU walks its tiles; the operand stream runs across tile boundaries.
//
// A stage holds K = 128 of both operand tiles (up to 256 rows x 128 bytes
// each): every row segment is a whole 128-byte line, which streams from L2
// about 1.6x faster per CU than half lines. The 160 KB of LDS is a ring of five
// 32 KB slots, one operand tile of one stage each: unit h (the A tile of
// stage h / 2 for even h, its B tile for odd h) lives in slot h % 5. While
// stage g computes from units 2g and 2g + 1, units 2g + 2 .. 2g + 4 stream
// in; the barrier at the end of stage g releases two slots for units 2g + 5
// and 2g + 6. An A unit is NA = BM / 32 DMA instructions per wave and a B
// unit JB = BN / 32 (8 rows each): 8 and 8 for 256 x 256 tiles, 8 and 6 for
// 256 x 192, 4 and 8 for 128 x 256. The K = 32 sub-steps spread a stage's
// NA + JB instructions one after each MFMA row, so the address unit never
// queues a burst in front of the MFMAs. A tile's epilogue stages its
// accumulators through the B slot of its last stage, whose next unit is
// issued only during the next stage.
//
// 128 x 256 tiles (a 48 KB stage, whose A tile would fill half a slot) take
// a ring of three whole stages instead: stage g computes from slot g mod 3
// while stage g + 1 lands and stage g + 2 streams into the slot stage g - 1
// released, so two stages are in flight.
//
// The waits count outstanding loads instead of draining them: before each
// stage barrier vmcnt(NA) lgkmcnt(0) (the next stage landed; only the A unit
// issued after it may still be in flight; this wave's fragment reads of the
// stage returned), and before the epilogue vmcnt(NA + JB / 2) (the tile's
// scale and bias loads, issued before its K loop, have landed; only the
// next stage's A unit and half its B unit are younger): 8 / 12 for 256 x 256
// and 8 / 11 for 256 x 192 tiles. The three-stage ring waits vmcnt(NA +
// 3 JB / 4) = 10 at the barrier (stage g + 2's instructions issued so far
// are younger) and vmcnt(NA + JB) = 12 before the epilogue. Loads return in
// order, so a count is exact whenever at least that many younger loads exist.
//
// LDS rows are 128 bytes: 16-byte chunk c of row r sits at physical chunk
// c ^ ((r >> 1) & 7), which keeps both the DMA writes (lane i writes bytes
// [16 i, 16 i + 16) of its instruction's 1 KB) and the fragment reads (32
// rows x one chunk per 16-lane group) free of bank conflicts. A DMA lane
// therefore loads the logical chunk that lands on its physical slot.
constexpr int kSK = 128;                    // K bytes per stage
constexpr int kSTile = 256 * kSK;           // one operand tile of one stage (32 KB): a ring slot
constexpr int kSlots = 5;                   // ring of half stages
constexpr int kPersistentLds = kSlots * kSTile;

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

__device__ __forceinline__ int lds_chunk(int row, int c) { return c ^ ((row >> 1) & 7); }

// f(integral_constant<int, I>) for I = LO .. HI - 1.
template <int LO, int HI, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (LO < HI) {
    f(std::integral_constant<int, LO>{});
    static_for<LO + 1, HI>(f);
  }
}

template <int EPI, int OUT, int FLAGS, int NB>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_i8_persistent(GemmParams p) {
  // NB MFMA column blocks per wave. NB = 4 or 3: tiles are 256 x 64 NB
  // (256 or 192 columns), the waves 2 x 2 quadrants of 128 x 32 NB. NB = 2:
  // tiles are 128 x 256 (for M of a few hundred rows), the waves 1 x 4
  // quadrants of 128 x 64 sharing the A tile, which fills half its slot. An
  // A unit is NA, a B unit JB DMA instructions per wave (8 rows each).
  static_assert(NB == 4 || ((NB == 3 || NB == 2) && (FLAGS & kWithRope) == 0),
                "NB 4, or 3 or 2 without the RoPE epilogue");
  constexpr int BM = NB == 2 ? 128 : 256, BN = NB == 2 ? 256 : 64 * NB, WN = 32 * NB;
  constexpr int NA = BM / 32, JB = BN / 32;
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (p.m + BM - 1) / BM, tiles_n = (p.n + BN - 1) / BN;
  // Tile schedule. Workgroup w runs on XCD w % 8 (round-robin dispatch).
  // With a grid that is a multiple of 8, XCD x owns the contiguous raster
  // range [x*T/8, (x+1)*T/8) and its G/8 workgroups walk it in lockstep, so
  // the tiles resident on one XCD at any time are raster neighbours sharing
  // operand rows in that XCD's L2.
  const int ksplit = max(p.ksplit, 1);
  const int total = tiles_m * tiles_n * ksplit, G = gridDim.x, w = blockIdx.x;
  const bool by_xcd = (G & 7) == 0;
  const int t_start = by_xcd ? (int)(((int64_t)(w & 7) * total) >> 3) : 0;
  const int t_count = by_xcd ? (int)(((int64_t)((w & 7) + 1) * total) >> 3) - t_start : total;
  const int t_stride = by_xcd ? G >> 3 : G;
  const int t_first = by_xcd ? w >> 3 : w;
  const int ntiles = t_first < t_count ? (t_count - t_first + t_stride - 1) / t_stride : 0;
  if (ntiles == 0) return;
  // Work item i of this workgroup: output tile item / ksplit, K split
  // item % ksplit (the splits of one tile are raster neighbours too).
  auto item_of = [&](int i) { return t_start + t_first + i * t_stride; };
  const int kstages = p.k / kSK;
  auto ks_begin = [&](int item) { return (item % ksplit) * kstages / ksplit; };
  auto ks_end = [&](int item) { return (item % ksplit + 1) * kstages / ksplit; };

  // DMA cursor: the (tile, stage) of the next stage to issue. Wave w fills
  // rows 8 NA w .. 8 NA (w + 1) - 1 of the A tile and 8 JB w .. 8 JB (w + 1)
  // - 1 of the B tile, 8 rows per instruction; offsets are 32-bit (the host
  // checks that the operands span < 4 GB).
  uint32_t off_a[NA], off_b[JB];
  auto point = [&](int i) {
    int tm, tn;
    raster(item_of(i) / ksplit, tiles_m, tiles_n, tm, tn);
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int row = (wave * NA + j) * 8 + (lane >> 3);
      off_a[j] = (uint32_t)((int64_t)min(tm * BM + row, p.m - 1) * p.lda + lds_chunk(row, lane & 7) * 16);
    }
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const int row = (wave * JB + j) * 8 + (lane >> 3);
      off_b[j] = (uint32_t)((int64_t)min(tn * BN + row, p.n - 1) * p.ldb + lds_chunk(row, lane & 7) * 16);
    }
  };
  int dma_i = 0, dma_ks = ks_begin(item_of(0)), dma_end = ks_end(item_of(0));
  point(0);
  // The ring: unit h (the A tile of global stage h / 2 for even h, its B
  // tile for odd h) goes to slot h % kSlots. A unit is NA (A) or JB (B) DMA
  // instructions per wave, issued in halves spread between MFMAs (a burst
  // of them would stall the issuing wave behind the address unit). The
  // cursor advances after a B tile's second half; past the last stage of
  // the last tile it stays put and re-reads that stage into slots never
  // consumed.
  // dma_end (the cursor item's last stage + 1) is recomputed only when the
  // cursor moves to the next item, keeping its divisions out of the stages.
  auto advance = [&]() {
    if (dma_ks + 1 < dma_end) {
      ++dma_ks;
    } else if (dma_i + 1 < ntiles) {
      ++dma_i;
      const int it = item_of(dma_i);
      dma_ks = ks_begin(it);
      dma_end = ks_end(it);
      point(dma_i);
    }
  };
  // DMA instruction J (0..NA - 1 of A, 0..JB - 1 of B) of this wave's part
  // of the cursor stage's A or B tile into the ring tile at byte offset base.
  auto dma_one = [&](auto b_tag, auto j_tag, int base) {
    constexpr bool B = decltype(b_tag)::value;
    constexpr int J = decltype(j_tag)::value;
    int8_t* st = smem + base + wave * (B ? JB : NA) * 1024 + J * 1024;
    const uint32_t kof = (uint32_t)(dma_ks * kSK);
    if constexpr (B) dma16(p.b + (off_b[J] + kof), st);
    else dma16(p.a + (off_a[J] + kof), st);
    if constexpr (B && J == JB - 1) advance();
  };
  // Part R (of NB, one per MFMA row) of half H of a unit: instructions
  // [C H + R C / NB, C H + (R + 1) C / NB) with C the half's length.
  auto dma_part = [&](auto b_tag, auto h_tag, auto r_tag, int base) {
    constexpr bool B = decltype(b_tag)::value;
    constexpr int H = decltype(h_tag)::value, R = decltype(r_tag)::value;
    constexpr int C = B ? JB / 2 : NA / 2;
    static_for<C * H + R * C / NB, C * H + (R + 1) * C / NB>([&](auto j) { dma_one(b_tag, j, base); });
  };
  auto issue_half = [&](auto b_tag, auto h_tag, int base) {
    constexpr bool B = decltype(b_tag)::value;
    constexpr int H = decltype(h_tag)::value, C = B ? JB / 2 : NA / 2;
    static_for<C * H, C * H + C>([&](auto j) { dma_one(b_tag, j, base); });
  };
  using A_ = std::false_type;
  using B_ = std::true_type;
  using H0 = std::integral_constant<int, 0>;
  using H1 = std::integral_constant<int, 1>;

  // v_mfma_i32_32x32x32_i8: for sub-step u (K bytes [32 u, 32 u + 32) of the
  // stage), lane (r = lane % 32, h = lane / 32) supplies row r, logical
  // chunk 2 u + h of both operands. Each wave holds a 4x4 grid of 32x32
  // accumulator tiles (its 128x128 quadrant).
  const int wm = NB == 2 ? 0 : wave >> 1, wn = NB == 2 ? wave : wave & 1;
  const int fr = lane & 31, fh = lane >> 5;
  const int a_row = wm * 128 * kSK + fr * kSK, b_row = wn * WN * kSK + fr * kSK;
  auto read_frags = [&](int base_a, int base_b, int u, v4i (&fa)[NB], v4i (&fb)[4]) {
    const int8_t* sa = smem + base_a;
    const int8_t* sb = smem + base_b;
    const int off = lds_chunk(fr, 2 * u + fh) << 4;   // rows 32 i + fr share (row >> 1) & 7
#pragma unroll
    for (int i = 0; i < NB; ++i) fa[i] = *reinterpret_cast<const v4i*>(sb + b_row + i * 32 * kSK + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) fb[i] = *reinterpret_cast<const v4i*>(sa + a_row + i * 32 * kSK + off);
  };
  // Group k (0 .. NB - 2) of the fragment reads of sub-step u, in the order
  // the next sub-step's first MFMA row consumes them (all four A fragments
  // fb, then the B fragments fa). NB = 4: k = 0 reads fb[0..2], k = 1
  // fb[3], fa[0..1], k = 2 fa[2..3]; NB = 3: k = 0 fb[0..3], k = 1
  // fa[0..2]; NB = 2: k = 0 all six. The last MFMA row of a sub-step issues
  // no reads, so the reads have landed when the next sub-step starts.
  auto read_group = [&](int base_a, int base_b, int u, int k, v4i (&fa)[NB], v4i (&fb)[4]) {
    const int off = lds_chunk(fr, 2 * u + fh) << 4;
    const int8_t* sa = smem + base_a + a_row + off;
    const int8_t* sb = smem + base_b + b_row + off;
    auto rd = [](const int8_t* base, int i) { return *reinterpret_cast<const v4i*>(base + i * 32 * kSK); };
    if constexpr (NB == 4) {
      if (k == 0) {
        fb[0] = rd(sa, 0); fb[1] = rd(sa, 1); fb[2] = rd(sa, 2);
      } else if (k == 1) {
        fb[3] = rd(sa, 3); fa[0] = rd(sb, 0); fa[1] = rd(sb, 1);
      } else {
        fa[2] = rd(sb, 2); fa[3] = rd(sb, 3);
      }
    } else if constexpr (NB == 3) {
      if (k == 0) {
        fb[0] = rd(sa, 0); fb[1] = rd(sa, 1); fb[2] = rd(sa, 2); fb[3] = rd(sa, 3);
      } else {
        fa[0] = rd(sb, 0); fa[1] = rd(sb, 1); fa[2] = rd(sb, 2);
      }
    } else {
      fb[0] = rd(sa, 0); fb[1] = rd(sa, 1); fb[2] = rd(sa, 2); fb[3] = rd(sa, 3);
      fa[0] = rd(sb, 0); fa[1] = rd(sb, 1);
    }
  };
  v16i acc[NB][4];
  // Block row nb of the NB x 4 MFMA grid (4 MFMAs).
  auto mfma_row = [&](int nb, const v4i (&fa)[NB], const v4i (&fb)[4]) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
      acc[nb][mb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[nb], fb[mb], acc[nb][mb], 0, 0, 0);
  };

  // Stage g computes from units 2g, 2g + 1 (slots c, c + 1 with
  // c = 2g mod 5). During it the second half of unit 2g + 3 and unit 2g + 4
  // are issued (slots c + 3, c + 4, freed by stage g - 1); its end releases
  // slots c, c + 1, and the first half of unit 2g + 5 goes to slot c.
  //
  // 128 x 256 tiles (NB = 2) take a ring of three whole stages instead
  // (STAGE_RING): stage slot s holds the A tile (16 KB) at 48 KB s and the
  // B tile (32 KB) after it. Stage g computes from slot g mod 3 while stage
  // g + 1 (issued during stage g - 1) lands and stage g + 2 is issued into
  // the slot stage g - 1 released: two stages (96 KB) in flight, where the
  // five half-stage slots keep about one (their A slots half empty).
  constexpr bool STAGE_RING = NB == 2;
  constexpr int kStage2 = (BM + BN) * kSK, kA2 = BM * kSK;
  static_assert(!STAGE_RING || 3 * kStage2 <= kPersistentLds, "three stages fit the LDS");
  auto next_slot = [](int slot) { return slot == (STAGE_RING ? 2 : kSlots - 1) ? 0 : slot + 1; };
  // Byte offsets of the A and B tiles of the stage in slot s (STAGE_RING),
  // or whose A tile is in slot s (its B tile in the next slot).
  auto a_of = [&](int s) { return STAGE_RING ? s * kStage2 : s * kSTile; };
  auto b_of = [&](int s) { return STAGE_RING ? s * kStage2 + kA2 : next_slot(s) * kSTile; };
  if constexpr (STAGE_RING) {
    issue_half(A_{}, H0{}, a_of(0));
    issue_half(A_{}, H1{}, a_of(0));
    issue_half(B_{}, H0{}, b_of(0));
    issue_half(B_{}, H1{}, b_of(0));
    issue_half(A_{}, H0{}, a_of(1));
    issue_half(A_{}, H1{}, a_of(1));
    issue_half(B_{}, H0{}, b_of(1));
    issue_half(B_{}, H1{}, b_of(1));
    wait_vmcnt<NA + JB>();  // stage 0 landed (stage 1 in flight)
  } else {
    issue_half(A_{}, H0{}, 0);
    issue_half(A_{}, H1{}, 0);
    issue_half(B_{}, H0{}, kSTile);
    issue_half(B_{}, H1{}, kSTile);
    issue_half(A_{}, H0{}, 2 * kSTile);
    issue_half(A_{}, H1{}, 2 * kSTile);
    issue_half(B_{}, H0{}, 3 * kSTile);
    wait_vmcnt<NA + JB / 2>();  // stage 0 landed (unit 2 and half of unit 3 in flight)
  }
  block_barrier();
  v4i fa0[NB], fb0[4], fa1[NB], fb1[4];
  read_frags(a_of(0), b_of(0), 0, fa0, fb0);
  int cur_a = 0;   // slot of the current stage (STAGE_RING) or of its A tile
  for (int i = 0; i < ntiles; ++i) {
    const int item = item_of(i);
    int tm, tn;
    raster(item / ksplit, tiles_m, tiles_n, tm, tn);
    const int mw = tm * BM + wm * 128, nw = tn * BN + wn * WN;
    // Row scales in the MFMA layout, the column scales (and biases) of the
    // staged read-out and the gate labels, fetched before the K loop so the
    // epilogue never waits on them.
    float as[4], wsc[2][8];
    uint32_t braw[2][8];
    int lbl[4] = {0, 0, 0, 0};
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      as[mb] = EPI != kEpiInt32 ? p.row_scale[min(mw + mb * 32 + fr, p.m - 1)] : 0.0f;
      if constexpr ((FLAGS & kWithGate) != 0) lbl[mb] = p.labels[min(mw + mb * 32 + fr, p.m - 1)];
    }
    if constexpr ((FLAGS & kWithRope) != 0) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) braw[h][j] = 0;
      if (nw < 2 * p.rope_heads * 128) load_rope_scales<EPI>(p, nw, lane, wsc);
      else load_readout_scales<EPI, OUT, false>(p, nw, lane, wsc, braw);
    } else {
      load_readout_scales<EPI, OUT, (FLAGS & kWithBias) != 0>(p, nw, lane, wsc, braw);
    }
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = v16i{};
    const int nks = ks_end(item) - ks_begin(item);   // >= 1
    // One stage: 16 NB MFMAs, 4 (NB + 4) fragment reads and NA + JB DMA
    // instructions.
    int stg = 0;   // byte offset of the last stage's B tile: the epilogue's staging area
    int ks = 0;
    // A sub-step in fixed order: each MFMA row of the current fragments but
    // the last is followed by one group of the next sub-step's fragment
    // reads, and every row by its part of the half-unit of DMA
    // (sched_barrier keeps the compiler from regrouping them).
    auto substep = [&](const v4i (&ca)[NB], const v4i (&cb)[4], int ra, int rb, int u, v4i (&na)[NB],
                       v4i (&nb)[4], auto b_tag, auto h_tag, int dbase) {
      static_for<0, NB>([&](auto r_tag) {
        constexpr int R = decltype(r_tag)::value;
        mfma_row(R, ca, cb);
        // (The last row's DMA may rise among its MFMAs.)
        if constexpr (R + 1 < NB) {
          __builtin_amdgcn_sched_barrier(0);
          read_group(ra, rb, u, R, na, nb);
        }
        dma_part(b_tag, h_tag, r_tag, dbase);
        __builtin_amdgcn_sched_barrier(0);
      });
    };
    do {  // nks >= 1
      // At a tile's last stage the next tile's first fragments are read
      // after the epilogue, so they do not hold registers through it.
      const bool last = ks + 1 == nks;
      if constexpr (STAGE_RING) {
        // Stage g + 2 goes to the slot stage g - 1 released: its A tile
        // during sub-steps 0 and 1, its B tile during 2 and 3.
        using R0 = std::integral_constant<int, 0>;
        using R1 = std::integral_constant<int, 1>;
        const int nxt = next_slot(cur_a), fill = next_slot(nxt);
        const int ca = a_of(cur_a), cb = b_of(cur_a);
        substep(fa0, fb0, ca, cb, 1, fa1, fb1, A_{}, H0{}, a_of(fill));
        substep(fa1, fb1, ca, cb, 2, fa0, fb0, A_{}, H1{}, a_of(fill));
        substep(fa0, fb0, ca, cb, 3, fa1, fb1, B_{}, H0{}, b_of(fill));
        mfma_row(0, fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
        dma_part(B_{}, H1{}, R0{}, b_of(fill));
        __builtin_amdgcn_sched_barrier(0);
        // Stage g + 1 landed - only the NA + 3 JB / 4 instructions of stage
        // g + 2 issued so far are younger - and this wave's reads of stage g
        // returned; the barrier releases slot g mod 3 for stage g + 3.
        wait_vm_lgkm<NA + 3 * JB / 4>();
        block_barrier();
        if (!last) read_group(a_of(nxt), b_of(nxt), 0, 0, fa0, fb0);
        dma_part(B_{}, H1{}, R1{}, b_of(fill));
        __builtin_amdgcn_sched_barrier(0);
        mfma_row(1, fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
        stg = cb;
        cur_a = nxt;
      } else {
        const int cur_b = next_slot(cur_a);
        const int nxt_a = next_slot(cur_b), nxt_b = next_slot(nxt_a), fill = next_slot(nxt_b);
        substep(fa0, fb0, a_of(cur_a), a_of(cur_b), 1, fa1, fb1, B_{}, H1{}, a_of(nxt_b));
        substep(fa1, fb1, a_of(cur_a), a_of(cur_b), 2, fa0, fb0, A_{}, H0{}, a_of(fill));
        substep(fa0, fb0, a_of(cur_a), a_of(cur_b), 3, fa1, fb1, A_{}, H1{}, a_of(fill));
        // The first MFMA row of the last sub-step consumes its fragments, so
        // past it this wave is done reading the stage's slots.
        mfma_row(0, fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
        // The next stage (units 2g + 2, 2g + 3) landed - only unit 2g + 4,
        // issued after them, may still be in flight - and this wave's reads of
        // this stage returned;
        wait_vm_lgkm<NA>();
        block_barrier();   // ... for every wave: both slots are released.
        static_for<0, NB>([&](auto r_tag) {
          constexpr int R = decltype(r_tag)::value;
          if constexpr (R > 0) {
            mfma_row(R, fa1, fb1);
            __builtin_amdgcn_sched_barrier(0);
          }
          if constexpr (R + 1 < NB) {
            if (!last) read_group(a_of(nxt_a), a_of(nxt_b), 0, R, fa0, fb0);
          }
          dma_part(B_{}, H0{}, r_tag, a_of(cur_a));
          __builtin_amdgcn_sched_barrier(0);
        });
        stg = a_of(cur_b);
        cur_a = nxt_a;
      }
    } while (++ks < nks);
    // The tile's scale and bias loads have landed: they are older than the
    // DMA still in flight (half-stage slots: at most unit 2g + 4 and the
    // first half of unit 2g + 5; STAGE_RING: stage g + 2). (The epilogue's
    // residual loads queue behind those instructions.)
    wait_vmcnt<STAGE_RING ? NA + JB : NA + JB / 2>();
    float bsc[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        bsc[h][j] = (FLAGS & kWithBias) == 0       ? 0.0f
                    : p.bias_dtype == kF16 ? h2f((uint16_t)braw[h][j])
                                           : __builtin_bit_cast(float, braw[h][j]);
    int8_t* const stage_w = smem + stg + wave * 8192;
    const int64_t out_off = (item % ksplit) * p.split_stride;
    // Interior quadrants take a copy without store masks (not for the gate
    // variants, whose registers a second copy would push into spills).
    if constexpr ((FLAGS & kWithRope) != 0) {
      if (nw >= 2 * p.rope_heads * 128) {   // V columns
        if (p.vec16 && mw + 128 <= p.m && nw + 128 <= p.n)
          store_quadrant32_passes<EPI, OUT, 0, true>(p, acc, wsc, bsc, as, lbl, mw, nw, lane, stage_w, out_off);
        else
          store_quadrant32_passes<EPI, OUT, 0, false>(p, acc, wsc, bsc, as, lbl, mw, nw, lane, stage_w, out_off);
      } else if (p.rope_pairs) {
        if (p.rope_f32) store_quadrant_rope<EPI, kF32, true>(p, acc, wsc, as, mw, nw, lane, stage_w);
        else store_quadrant_rope<EPI, kF16, true>(p, acc, wsc, as, mw, nw, lane, stage_w);
      } else if (p.rope_f32) {
        store_quadrant_rope<EPI, kF32, false>(p, acc, wsc, as, mw, nw, lane, stage_w);
      } else {
        store_quadrant_rope<EPI, kF16, false>(p, acc, wsc, as, mw, nw, lane, stage_w);
      }
    } else if ((FLAGS & kWithGate) == 0 && p.vec16 && mw + 128 <= p.m && nw + WN <= p.n)
      store_quadrant32_passes<EPI, OUT, FLAGS, (FLAGS & kWithGate) == 0, NB>(p, acc, wsc, bsc, as, lbl, mw, nw,
                                                                            lane, stage_w, out_off);
    else
      store_quadrant32_passes<EPI, OUT, FLAGS, false, NB>(p, acc, wsc, bsc, as, lbl, mw, nw, lane, stage_w,
                                                          out_off);
    // The staging slot's next unit (2g + 6; STAGE_RING: the B tile of stage
    // g + 3) is issued during the next stage; a wave's DMA into a slot
    // writes the same 8 KB it used for staging, so its own staging reads
    // returning is all that unit waits for.
    wait_lgkm();
    // The next tile's first fragments (its stage 0 landed before the last
    // barrier).
    static_for<0, NB - 1>([&](auto k) { read_group(a_of(cur_a), b_of(cur_a), 0, decltype(k)::value, fa0, fb0); });
  }
  wait_vmcnt<0>();  // no DMA may still target this workgroup's LDS at exit
}

// Skinny GEMM for 2 <= M <= 64 where K is not a multiple of 128, and for
// 2 <= M <= 8 where its 16-row grid fills the GPU in one wave (the streaming
// kernel below takes the rest): weight streaming. A workgroup of W
// wavefronts owns NR weight rows (NR = 16 with W = 8, or NR = 32 with W = 4
// when N / 32 still fills the GPU); the waves
// split K into contiguous ranges and multiply with v_mfma_i32_16x16x64_i8
// (weight rows as the MFMA A operand, MB 16-row activation blocks as B),
// loading both operands straight from memory into registers in batches of U
// K steps, double buffered so the next batch is in flight while the current
// one multiplies. The W partial sums meet in LDS; the shared epilogue writes
// the outputs. The activation rows (<= 64 x K) stay cache-resident across
// workgroups.
constexpr int kSkinnyMaxM = 64;

template <int EPI, int OUT, int NR, int MB>
__global__ __launch_bounds__(NR == 16 ? 512 : 256) void gemm_i8_skinny(GemmParams p) {
  constexpr int NB = NR / 16;
  constexpr int W = NR == 16 ? 8 : 4;
  constexpr int U = MB == 1 ? 4 : 2;
  __shared__ int red[W][NR][MB * 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * NR;
  const int ksteps = p.k >> 6;
  const int per = (ksteps + W - 1) / W;
  const int s0 = min(wave * per, ksteps), s1 = min(s0 + per, ksteps);
  const int fr = lane & 15, fc = lane >> 4;

  const int8_t* wrow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) wrow[nb] = p.b + (int64_t)min(n0 + nb * 16 + fr, p.n - 1) * p.ldb + fc * 16;
  const int8_t* arow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) arow[mb] = p.a + (int64_t)min(mb * 16 + fr, p.m - 1) * p.lda + fc * 16;

  v4i acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = v4i{0, 0, 0, 0};

  // Batch at K step s: U steps (past s1 the last step is re-read and not used).
  auto load = [&](int s, v4i (&wf)[U][NB], v4i (&af)[U][MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kof = min(s + u, s1 - 1) * 64;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) wf[u][nb] = *reinterpret_cast<const v4i*>(wrow[nb] + kof);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) af[u][mb] = *reinterpret_cast<const v4i*>(arow[mb] + kof);
    }
  };
  auto mma = [&](int s, const v4i (&wf)[U][NB], const v4i (&af)[U][MB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s + u < s1) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[nb][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[u][nb], af[u][mb], acc[nb][mb], 0, 0, 0);
      }
    }
  };
  v4i wa[U][NB], aa[U][MB], wb[U][NB], ab[U][MB];
  if (s0 < s1) load(s0, wa, aa);
  for (int s = s0; s < s1; s += 2 * U) {
    if (s + U < s1) load(s + U, wb, ab);
    mma(s, wa, aa);
    if (s + 2 * U < s1) load(s + 2 * U, wa, aa);
    if (s + U < s1) mma(s + U, wb, ab);
  }
  // Lane holds C[m][n..n+3] for m = 16 mb + fr, n = 16 nb + 4 fc (local).
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][nb * 16 + 4 * fc + v][mb * 16 + fr] = acc[nb][mb][v];
  __syncthreads();
  // Thread -> (m, 4 consecutive n): sum the W partials, then the epilogue.
  for (int idx = tid; idx < p.m * (NR / 4); idx += W * 64) {
    const int m = idx / (NR / 4);
    const int nl = (idx % (NR / 4)) * 4;
    const int n = n0 + nl;
    const int valid = min(4, p.n - n);
    if (valid <= 0) continue;
    int c[4] = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < W; ++w)
#pragma unroll
      for (int v = 0; v < 4; ++v) c[v] += red[w][nl + v][m];
    const float a = EPI != kEpiInt32 ? p.row_scale[m] : 0.0f;
    epilogue4<EPI, OUT>(p, m, n, valid, c, a);
  }
}

// GEMV (M == 1, decode): wave w owns R consecutive weight rows; lane l
// reads the 16-byte K chunks l, l + 64, ... of each, so every load
// instruction covers 1 KB of one row, and multiplies them with the matching
// activation chunk by v_dot4_i32_i8 (exact int32 sums in any order). A batch
// is C = 16 / R chunks of each row: 16 KB per wave in flight. Each row's
// partial sums meet by a cross-lane reduction; lane 0 stores the R outputs
// through the shared epilogue.
template <int EPI, int OUT, int R>
__global__ __launch_bounds__(256) void gemv_i8(GemmParams p) {
  constexpr int C = R == 4 ? 4 : 8;
  const int lane = threadIdx.x & 63;
  const int n0 = (int)(((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * R);
  if (n0 >= p.n) return;
  const int chunks = p.k >> 4;
  const int8_t* wr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wr[r] = p.b + (int64_t)min(n0 + r, p.n - 1) * p.ldb;
  int acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0;
  for (int c0 = 0; c0 < chunks; c0 += 64 * C) {
    v4i w[R][C], x[C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const int c = c0 + 64 * i + lane;
      const bool ok = c < chunks;
      x[i] = ok ? *reinterpret_cast<const v4i*>(p.a + (int64_t)c * 16) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < R; ++r)
        w[r][i] = ok ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wr[r] + (int64_t)c * 16))
                     : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < C; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[r] = __builtin_amdgcn_sdot4(w[r][i][e], x[i][e], acc[r], false);
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc[r] += __shfl_xor(acc[r], off, 64);
  if (lane != 0) return;
  const float a = EPI != kEpiInt32 ? p.row_scale[0] : 0.0f;
#pragma unroll
  for (int g = 0; g < R; g += 4) {
    const int n = n0 + g;
    const int valid = min(min(4, R - g), p.n - n);
    if (valid <= 0) break;
    int c[4] = {0, 0, 0, 0};
#pragma unroll
    for (int v = 0; v < 4 && g + v < R; ++v) c[v] = acc[g + v];
    epilogue4<EPI, OUT>(p, 0, n, valid, c, a);
  }
}

// Rows per wave of the GEMV: the most (4, 2, 1) that still give every SIMD
// of the GPU four waves.
template <int EPI, int OUT>
void launch_gemv(const GemmParams& p, int cus, hipStream_t s) {
  const int64_t want = (int64_t)cus * 16;   // 4 SIMDs x 4 waves
  auto grid = [&](int r) { return dim3((unsigned)(((p.n + r - 1) / r + 3) / 4)); };
  if ((p.n + 3) / 4 >= want) hipLaunchKernelGGL((gemv_i8<EPI, OUT, 4>), grid(4), dim3(256), 0, s, p);
  else if ((p.n + 1) / 2 >= want) hipLaunchKernelGGL((gemv_i8<EPI, OUT, 2>), grid(2), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((gemv_i8<EPI, OUT, 1>), grid(1), dim3(256), 0, s, p);
}

template <int EPI, int OUT, int MB>
void launch_skinny(const GemmParams& p, hipStream_t s) {
  // 32 weight rows per workgroup while that still fills 256 workgroups.
  if (p.n / 32 >= 256) {
    hipLaunchKernelGGL((gemm_i8_skinny<EPI, OUT, 32, MB>), dim3((unsigned)((p.n + 31) / 32)), dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL((gemm_i8_skinny<EPI, OUT, 16, MB>), dim3((unsigned)((p.n + 15) / 16)), dim3(512), 0, s, p);
  }
}

// Weight streaming for 2 <= M <= 64 with K a multiple of 128 (text-encoder
// decode and short prefill). A workgroup of 4 waves owns 64 weight rows and
// one of ksplit contiguous K ranges. A step is 128 bytes of K: the 64
// weight rows and the MB 16-row blocks of activation rows (8 rows per
// global_load_lds_dwordx4). The workgroup streams its range through one LDS
// ring of S steps with S - 1 steps in flight. Each wave issues a quarter of every
// step's DMA; one barrier per step makes the step visible to all waves and
// frees the slot read in the step before for the next refill. In each
// 128-byte row, 16-byte chunk c lands at c ^ ((r >> 1) & 7), so the DMA
// writes and the fragment reads are free of bank conflicts. Every load of
// the loop is an LDS DMA, and every iteration issues the same number of them
// (past the range's end the walk's last step is loaded again into the freed slot,
// which is never read), so the counted waits are exact. With four
// activation blocks (M 49..64) wave w multiplies a 32 x 32 block, weight rows
// 32 (w >> 1) .. + 31 with activation rows 32 (w & 1) .. + 31: four fragment
// reads per four MFMAs instead of five, which the LDS read rate rewards
// (64 x 14336 x 4096 16.0 -> 14.1 us). With fewer blocks wave w multiplies
// weight rows 16 w .. 16 w + 15 with every activation block. The MFMA is
// v_mfma_i32_16x16x64_i8, two 64-byte sub-steps per step. Each wave finishes
// its own outputs: with ksplit == 1 the shared epilogue writes them, otherwise
// plane ks of the caller's workspace receives the int32 sums and
// splitk_reduce_kernel finishes.
constexpr int kStreamRows = 64;      // weight rows per workgroup
constexpr int kStreamStep = 128;     // K bytes per step
constexpr int kStreamWaves = 4;

// 48 KB per workgroup, up to three workgroups per CU: 3 slots for MB 3, 4
// (16 KB slots), 4 for MB 1, 2 (12 KB). Two or three steps in flight per
// workgroup stream as fast as deeper rings at every measured shape (a sweep
// of 48 to 120 KB rings at M = 17..64), and the shallow
// ring lets CUs hold more than one workgroup when the grid exceeds the CUs.
constexpr int kStreamRingBytes = 48 * 1024;

template <int MB>
struct StreamRing {
  static constexpr int kRows = kStreamRows + 16 * MB;             // weight + activation rows of a step
  static constexpr int kDpw = (kRows / 8 + kStreamWaves - 1) / kStreamWaves;   // DMA per wave and step
  static constexpr int kSlot = 8 * kStreamWaves * kDpw * kStreamStep;          // padded to whole DMA groups
  static constexpr int kSlots = kStreamRingBytes / kSlot;
  static constexpr int kLds = kSlots * kSlot;
};

template <int EPI, int OUT, int MB, bool PARTIAL>
__global__ __launch_bounds__(kStreamWaves * 64) void gemm_i8_stream(GemmParams p, int nblocks, int ksplit) {
  using R = StreamRing<MB>;
  static_assert(R::kLds <= kStreamRingBytes && R::kSlots >= 3 && (R::kSlots - 2) * R::kDpw < 64,
                "LDS and vmcnt range");
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nblk = blockIdx.x % nblocks, ks = blockIdx.x / nblocks;
  const int n0 = nblk * kStreamRows;
  const int steps = p.k / kStreamStep;
  const int g0 = (int)((int64_t)ks * steps / ksplit), g1 = (int)((int64_t)(ks + 1) * steps / ksplit);
  const int nsteps = g1 - g0;

  // This wave's DMA instruction i of a step: slot rows 8 d .. 8 d + 7 with
  // d = kDpw * wave + i; lane -> row 8 d + lane / 8 and the logical chunk
  // that lands on physical chunk lane % 8. Rows 0..63 are weight rows n0 +
  // r (clamped to the last weight row), the next 16 MB activation rows
  // (clamped to the last of the m rows; clamped rows are never stored), the
  // padding rows past them load a weight row that is never read.
  const int8_t* src[R::kDpw];
#pragma unroll
  for (int i = 0; i < R::kDpw; ++i) {
    const int r = 8 * (R::kDpw * wave + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    src[i] = r >= kStreamRows && r < R::kRows
                 ? p.a + (int64_t)min(r - kStreamRows, p.m - 1) * p.lda + c * 16
                 : p.b + (int64_t)min(n0 + (r < kStreamRows ? r : 0), p.n - 1) * p.ldb + c * 16;
  }
  const int fr = lane & 15, fc = lane >> 4;
  // MB == 4: wave w takes weight rows 32 (w >> 1) .. + 31 against activation
  // rows 32 (w & 1) .. + 31 (2 x 2 blocks); otherwise weight rows 16 w .. +15
  // against every activation block.
  constexpr bool kQuad = MB == 4;
  const int wi = wave >> 1, wj = wave & 1;
  v4i acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = v4i{0, 0, 0, 0};

  if (nsteps > 0) {
    // Workgroup nblk walks its K range starting at step nblk % nsteps and
    // wraps around (integer sums do not depend on the order), so the
    // workgroups of one K range read different columns of their rows at any
    // moment instead of all the same one: 64 x 4096 x 14336 15.8 -> 14.5 us.
    const int rot = nblk % nsteps;
    auto dma_step = [&](int t, int slot) {
      int u = min(t, nsteps - 1) + rot;
      u = u >= nsteps ? u - nsteps : u;
      const int64_t kof = (int64_t)(g0 + u) * kStreamStep;
#pragma unroll
      for (int i = 0; i < R::kDpw; ++i)
        dma16(src[i] + kof, lds + slot * R::kSlot + (R::kDpw * wave + i) * 1024);
    };
    // Fragment (slot rows row0 + fr, K bytes 64 j + 16 fc .. + 16).
    auto frag = [&](int slot, int row0, int j) {
      const int r = row0 + fr;
      const int c = (4 * j + fc) ^ ((r >> 1) & 7);
      return *reinterpret_cast<const v4i*>(lds + slot * R::kSlot + r * kStreamStep + c * 16);
    };
#pragma unroll
    for (int i = 0; i < R::kSlots - 1; ++i) dma_step(i, i);
    int slot = 0;                      // slot of step t
    int refill = R::kSlots - 1;        // slot of step t + S - 1 (read in step t - 1)
    for (int t = 0; t < nsteps; ++t) {
      // This wave's loads of step t landed (only the S - 2 younger steps'
      // may be in flight); after the barrier every wave's have, and every
      // wave is done reading the slot of step t - 1.
      wait_vmcnt<(R::kSlots - 2) * R::kDpw>();
      block_barrier();
      dma_step(t + R::kSlots - 1, refill);
      if constexpr (kQuad) {
        v4i w[2][2], x[2][2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            w[j][h] = frag(slot, 32 * wi + 16 * h, j);
            x[j][h] = frag(slot, kStreamRows + 32 * wj + 16 * h, j);
          }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
              acc[2 * a + b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j][a], x[j][b], acc[2 * a + b], 0, 0, 0);
      } else {
        v4i w[2], x[2][MB];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          w[j] = frag(slot, 16 * wave, j);
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) x[j][mb] = frag(slot, kStreamRows + mb * 16, j);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j], x[j][mb], acc[mb], 0, 0, 0);
      }
      refill = slot;
      slot = slot + 1 == R::kSlots ? 0 : slot + 1;
    }
  }
  wait_vmcnt<0>();   // no DMA may still target the ring at exit
  // Lane holds C[m][n .. n + 3] for m = 16 mb + fr, n = n0 + 16 wave + 4 fc
  // (MB == 4: block 2 a + b holds m = 32 wj + 16 b + fr, n = n0 + 32 wi +
  // 16 a + 4 fc).
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int n = kQuad ? n0 + 32 * wi + 16 * (mb >> 1) + 4 * fc : n0 + 16 * wave + 4 * fc;
    const int valid = min(4, p.n - n);
    if (valid <= 0) continue;
    const int m = kQuad ? 32 * wj + 16 * (mb & 1) + fr : 16 * mb + fr;
    if (m >= p.m) continue;
    const int c[4] = {acc[mb][0], acc[mb][1], acc[mb][2], acc[mb][3]};
    if constexpr (PARTIAL) {
      int* o = reinterpret_cast<int*>(p.ws) + (int64_t)ks * p.m * p.n + (int64_t)m * p.n + n;
      if (valid == 4 && (p.n & 3) == 0) *reinterpret_cast<int4*>(o) = make_int4(c[0], c[1], c[2], c[3]);
      else for (int v = 0; v < valid; ++v) o[v] = c[v];
    } else {
      epilogue4<EPI, OUT>(p, m, n, valid, c, EPI != kEpiInt32 ? p.row_scale[m] : 0.0f);
    }
  }
}

// Shapes the streaming kernel takes: 2..64 rows and whole 128-byte K steps,
// except up to 8 rows where the register-batched kernel's grid of 16-row
// workgroups fills more than half of the CUs in a single wave (N = 3072 and
// 4096 on 256 CUs): there it finishes first, with no split-K partials.
inline bool stream_applies(int64_t m, int64_t n, int64_t k, int cus) {
  if (m < 2 || m > kSkinnyMaxM || k < kStreamStep || k % kStreamStep != 0) return false;
  const int64_t skinny_wgs = (n + 15) / 16;
  return !(m <= 8 && 2 * skinny_wgs > cus && skinny_wgs <= cus);
}

// K split of the streaming kernel: the largest power of two up to 8 that
// keeps at most 4/3 workgroups per CU and at least four steps per
// workgroup. Measured at M = 2..64: more workgroups than that lose more to
// the split-K finish than they gain, fewer leave CUs idle.
inline int stream_ksplit(int64_t n, int64_t k, int cus) {
  const int64_t nblocks = (n + kStreamRows - 1) / kStreamRows, steps = k / kStreamStep;
  int ks = 1;
  while (ks < 8 && nblocks * ks * 2 * 3 <= 4 * (int64_t)cus && steps / (ks * 2) >= 4) ks *= 2;
  return ks;
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

// Split-K finish: thread -> 4 consecutive columns of one row; adds the
// ksplit int32 partial tiles (exact), then the shared epilogue. Every plan
// splits K at most kMaxSplit ways; the planes' loads are all issued before
// the first add, so their latencies overlap instead of adding up.
constexpr int kMaxSplit = 8;

template <int EPI, int OUT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams p, const int32_t* __restrict__ ws,
                                                            int ksplit, int64_t stride) {
  const int quads = (p.n + 3) >> 2;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.m * quads) return;
  const int m = (int)(idx / quads);
  const int n = (int)(idx - (int64_t)m * quads) * 4;
  const int valid = min(4, p.n - n);
  const int32_t* src = ws + (int64_t)m * p.n + n;
  int c[4] = {0, 0, 0, 0};
  if (valid == 4 && (p.n & 3) == 0 && ksplit <= kMaxSplit) {
    int4 v[kMaxSplit];
#pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp)
      v[sp] = sp < ksplit ? *reinterpret_cast<const int4*>(src + sp * stride) : make_int4(0, 0, 0, 0);
#pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp) {
      c[0] += v[sp].x; c[1] += v[sp].y; c[2] += v[sp].z; c[3] += v[sp].w;
    }
  } else if (valid == 4 && (p.n & 3) == 0) {
    for (int sp = 0; sp < ksplit; ++sp) {
      const int4 v = *reinterpret_cast<const int4*>(src + sp * stride);
      c[0] += v.x; c[1] += v.y; c[2] += v.z; c[3] += v.w;
    }
  } else {
    for (int sp = 0; sp < ksplit; ++sp)
      for (int v = 0; v < valid; ++v) c[v] += src[sp * stride + v];
  }
  epilogue4<EPI, OUT>(p, m, n, valid, c, EPI != kEpiInt32 ? p.row_scale[m] : 0.0f);
}

// ------------------------------------------------------------------ launch

// Per-device one-time records (bit d = device d done).
struct DeviceOnce {
  std::atomic<uint64_t> done{0};
};

inline int current_device(int& dev) {
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("w8a8_gemm: hipGetDevice failed");
    return W8A8_ERR_LAUNCH;
  }
  return W8A8_OK;
}

template <int EPI, int OUT, int FLAGS, int NB>
int launch_persistent(const GemmParams& p, int64_t tiles, int dev, hipStream_t s) {
  // The LDS ring and staging area exceed the 64 KB default: raise the
  // kernel's dynamic LDS limit once per device.
  static DeviceOnce lds_enabled;
  const uint64_t bit = 1ull << dev;
  if (!(lds_enabled.done.load(std::memory_order_acquire) & bit)) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_i8_persistent<EPI, OUT, FLAGS, NB>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, kPersistentLds);
    if (e != hipSuccess) {
      set_error("w8a8_gemm: cannot enable %d bytes of LDS: %s", kPersistentLds, hipGetErrorString(e));
      return W8A8_ERR_LAUNCH;
    }
    lds_enabled.done.fetch_or(bit, std::memory_order_acq_rel);
  }
  // One workgroup per CU (the ring takes the whole LDS); a multiple of 8 so
  // every XCD holds the same number of them, unless that would take one
  // more round of work items (150 items on 144 workgroups).
  const int64_t items = tiles * (p.ksplit > 1 ? p.ksplit : 1);
  int64_t grid = items < device_cus(dev) ? items : device_cus(dev);
  const int64_t grid8 = grid & ~7ll;
  if (grid8 >= 8 && (items + grid8 - 1) / grid8 == (items + grid - 1) / grid) grid = grid8;
  hipLaunchKernelGGL((gemm_i8_persistent<EPI, OUT, FLAGS, NB>), dim3((unsigned)grid), dim3(256), kPersistentLds, s,
                     p);
  return W8A8_OK;
}

// The persistent kernel with 256 x 64 nb tiles.
template <int EPI, int OUT, int FLAGS>
int launch_persistent_nb(const GemmParams& p, const GemmPlan& plan, int dev, hipStream_t s) {
  const int64_t tiles = plan_tiles(p.m, p.n, plan);
  if constexpr ((FLAGS & kWithRope) == 0) {
    if (plan.nb == 3) return launch_persistent<EPI, OUT, FLAGS, 3>(p, tiles, dev, s);
    if (plan.nb == 2) return launch_persistent<EPI, OUT, FLAGS, 2>(p, tiles, dev, s);
  }
  return launch_persistent<EPI, OUT, FLAGS, 4>(p, tiles, dev, s);
}

template <int EPI, int OUT, int MB>
int launch_stream(const GemmParams& p, int ksplit, hipStream_t s) {
  using R = StreamRing<MB>;
  static_assert(R::kLds <= 64 * 1024, "the ring fits the default dynamic LDS limit");
  const int nblocks = (p.n + kStreamRows - 1) / kStreamRows;
  const dim3 grid((unsigned)(nblocks * ksplit)), block(kStreamWaves * 64);
  if (ksplit == 1) {
    hipLaunchKernelGGL((gemm_i8_stream<EPI, OUT, MB, false>), grid, block, R::kLds, s, p, nblocks, 1);
    return W8A8_OK;
  }
  hipLaunchKernelGGL((gemm_i8_stream<EPI, OUT, MB, true>), grid, block, R::kLds, s, p, nblocks, ksplit);
  const int64_t threads = (int64_t)p.m * ((p.n + 3) / 4);
  hipLaunchKernelGGL((splitk_reduce_kernel<EPI, OUT>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, p,
                     reinterpret_cast<const int32_t*>(p.ws), ksplit, (int64_t)p.m * p.n);
  return W8A8_OK;
}

template <int EPI, int OUT>
int launch_gemm(const GemmParams& p, hipStream_t s) {
  if (p.m == 1 && p.k % 16 == 0) {
    int dev = 0;
    const int rc = current_device(dev);
    if (rc != W8A8_OK) return rc;
    launch_gemv<EPI, OUT>(p, device_cus(dev), s);
    return W8A8_OK;
  }
  if (p.m <= kSkinnyMaxM) {
    int dev = 0;
    const int rc = current_device(dev);
    if (rc != W8A8_OK) return rc;
    const int cus = device_cus(dev);
    if (stream_applies(p.m, p.n, p.k, cus)) {
      int ks = stream_ksplit(p.n, p.k, cus);
      if (ks > 1 && (p.ws == nullptr || p.ws_bytes < (int64_t)ks * p.m * p.n * 4)) ks = 1;
      switch ((p.m + 15) / 16) {
        case 1: return launch_stream<EPI, OUT, 1>(p, ks, s);
        case 2: return launch_stream<EPI, OUT, 2>(p, ks, s);
        case 3: return launch_stream<EPI, OUT, 3>(p, ks, s);
        default: return launch_stream<EPI, OUT, 4>(p, ks, s);
      }
    }
  }
  if (p.m <= kSkinnyMaxM && p.k % 64 == 0) {
    if (p.m <= 16) launch_skinny<EPI, OUT, 1>(p, s);
    else launch_skinny<EPI, OUT, 4>(p, s);
    return W8A8_OK;
  }
  // The persistent kernel streams whole K = 128 stages and addresses the
  // operands with 32-bit offsets; anything else takes the register-staged
  // kernel.
  const bool offsets32 = (int64_t)(p.m - 1) * p.lda + p.k < (1ll << 32) && (int64_t)(p.n - 1) * p.ldb + p.k < (1ll << 32);
  if (p.k % kSK != 0 || !offsets32) {
    const int64_t tiles = (int64_t)((p.m + kBM - 1) / kBM) * ((p.n + kBN - 1) / kBN);
    hipLaunchKernelGGL((gemm_i8_256x256<EPI, OUT>), dim3((unsigned)tiles), dim3(256), 0, s, p);
    return W8A8_OK;
  }
  int dev = 0;
  int rc = current_device(dev);
  if (rc != W8A8_OK) return rc;
  // Tile width and K split (the RoPE epilogue takes neither: one head per
  // 128-column quadrant, whole K).
  GemmPlan plan = p.rope_heads ? GemmPlan{4, 1} : gemm_plan(p.m, p.n, p.k, device_cus(dev));
  const int64_t ws_need = split_partials_bytes(p.m, p.n, plan.ksplit);
  if (plan.ksplit > 1 && (p.ws == nullptr || p.ws_bytes < ws_need)) plan = gemm_plan(p.m, p.n, p.k, device_cus(dev), 1);
  const int ksplit = plan.ksplit;
  if (ksplit > 1) {
    GemmParams q = p;
    q.out = p.ws;
    q.ldc = p.n;
    q.vec16 = (p.n & 3) == 0;
    q.residual = nullptr;
    q.gate = nullptr;
    q.bias_dtype = 0;
    q.ksplit = ksplit;
    q.split_stride = (int64_t)p.m * p.n;
    rc = launch_gemm_partials(q, plan, dev, s);
    if (rc != W8A8_OK) return rc;
    const int64_t threads = (int64_t)p.m * ((p.n + 3) / 4);
    hipLaunchKernelGGL((splitk_reduce_kernel<EPI, OUT>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       p, reinterpret_cast<const int32_t*>(p.ws), ksplit, q.split_stride);
    return W8A8_OK;
  }
  if constexpr (EPI == kEpiInt32) {
    return launch_persistent_nb<EPI, OUT, 0>(p, plan, dev, s);
  } else if constexpr (OUT != kF16) {  // a residual requires FP16 output
    return p.bias_dtype ? launch_persistent_nb<EPI, OUT, kWithBias>(p, plan, dev, s)
                        : launch_persistent_nb<EPI, OUT, 0>(p, plan, dev, s);
  } else {
    // The host admits the RMS-RoPE epilogue only without bias, residual or gate.
    if (p.rope_heads) return launch_persistent_nb<EPI, OUT, kWithRope>(p, plan, dev, s);
    switch ((p.bias_dtype ? kWithBias : 0) | (p.residual ? kWithResidual : 0) | (p.gate ? kWithGate : 0)) {
      case 0: return launch_persistent_nb<EPI, OUT, 0>(p, plan, dev, s);
      case kWithBias: return launch_persistent_nb<EPI, OUT, kWithBias>(p, plan, dev, s);
      case kWithResidual: return launch_persistent_nb<EPI, OUT, kWithResidual>(p, plan, dev, s);
      case kWithBias | kWithResidual: return launch_persistent_nb<EPI, OUT, kWithBias | kWithResidual>(p, plan, dev, s);
      case kWithResidual | kWithGate: return launch_persistent_nb<EPI, OUT, kWithResidual | kWithGate>(p, plan, dev, s);
      default: return launch_persistent_nb<EPI, OUT, kWithBias | kWithResidual | kWithGate>(p, plan, dev, s);
    }
  }
}

template <int EPI, int OUT>
void launch_dequant(const GemmParams& p, const int32_t* acc, int64_t ldacc, hipStream_t s) {
  const int64_t threads = (int64_t)p.m * ((p.n + 3) / 4);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipLaunchKernelGGL((dequant_kernel<EPI, OUT>), grid, dim3(256), 0, s, p, acc, ldacc);
}

}  // namespace w8a8
