// INT8 attention for 128-wide heads: the preparation of the INT8 operands
// (key centering, per-token Q scales, per-64-key K scales, per-channel V
// scales, V transposed) and the attention kernel (S = Q.K^T on INT8 MFMA;
// a first pass finds each query's largest logit, the second quantizes the
// exp2-domain probabilities against it to integers P in 0..255 and feeds
// P - 128 to the signed INT8 MFMA P.V product; the 128 * sum over keys of V
// it leaves out is one per-channel integer that the preparation sums. The denominator is the sum of the same integers P, so the whole
// accumulation is exact. The exponentials use the hardware exp2
// (v_exp_f32).
//
// Layout of the attention kernel: a workgroup of eight wavefronts (two per
// SIMD) takes 256 queries of one (batch, head); a wavefront owns 32. Keys come in
// blocks of 64 through a four-stage LDS ring (K tile 64 x 128 bytes, V^T
// tile 128 x 64 bytes). The score tile is computed transposed, S^T = K.Q^T, so a
// lane holds one query (lane % 32) and 16 of every 32 keys: the softmax
// statistics of a query need one exchange with the lane 32 away, and the
// quantized probabilities are already the B operand of O^T = V^T.P^T. Its K
// positions follow the order in which the score layout hands out the keys,
// so the preparation writes V^T with the same order inside each 32-key
// group (position 16 h + 4 g + i holds key 8 g + 4 h + i).
#include "w8a8_device.h"
#include "w8a8_host.h"

#include <type_traits>
#include <utility>

namespace w8a8 {

constexpr int kAttnD = 128;       // head dimension
constexpr int kAttnBK = 64;       // keys per block
constexpr int kAttnChunk = 256;   // tokens per partial of the key statistics
constexpr int kAttnWaveQ = 32;    // queries per wavefront
constexpr int kAttnWaves = 8;     // wavefronts per workgroup
constexpr int kAttnBQ = kAttnWaves * kAttnWaveQ;   // queries per workgroup
constexpr int kAttnDma = 8 / kAttnWaves;           // 1 KB DMA instructions per wave and tile
constexpr float kLog2e = 0x1.715476p+0f;    // fp32(log2(e))
constexpr float kLog2_255 = 0x1.ffa37cp+2f; // fp32(log2(255))

// Element strides of a [batch, head, token, channel] tensor whose channels
// are contiguous; at(bh, t) is the offset of token t's row of the flat
// (batch, head) index bh.
struct Strides3 {
  int64_t b, h, t;
  int heads;
  __device__ __forceinline__ int64_t at(int64_t bh, int64_t tok) const {
    return (bh / heads) * b + (bh % heads) * h + tok * t;
  }
};

struct AttnPrepParams {
  const void* q;
  const void* k;
  const void* v;
  Strides3 qst, kst, vst;
  int nq, nk, nkp, nblk, chunks;
  float c0;   // fp32(sm_scale * log2(e))
  int8_t* q8;
  float* qs;
  int8_t* k8;
  float* ks;
  int8_t* vt8;
  float* vs;
  int32_t* vsum;   // sum over the keys of vt8 per channel (int32 atomics)
  float* part_sum;
  float* part_max;
  float* kmean;
  float* vrcp;   // 1 / vs per channel (IEEE), so tokens do not divide
};

// 8 consecutive channels of one token row (16-byte loads).
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t off, float (&x)[8]) {
  if constexpr (DT == kF32) {
    const float4* q = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
    const float4 a = q[0], b = q[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + off);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = h2f((uint16_t)(u[i] & 0xffffu));
      x[2 * i + 1] = h2f((uint16_t)(u[i] >> 16));
    }
  }
}

// Partial statistics of 256 keys of one (batch, head): the fp32 sum of k
// (sequential from +0) and the absmax of v, per channel. Thread (chunk
// tid / 16, channels 8 (tid % 16) + [0, 8)) walks its chunk's tokens in
// order; a workgroup covers 16 chunks.
template <int DT>
__global__ __launch_bounds__(256) void attn_stats_kernel(AttnPrepParams p) {
  const int cg = threadIdx.x & 15, chunk = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int64_t bh = blockIdx.y;
  if (chunk >= p.chunks) return;
  const int t0 = chunk * kAttnChunk, t1 = min(t0 + kAttnChunk, p.nk);
  const int64_t kb = p.kst.at(bh, 0) + 8 * cg, vb = p.vst.at(bh, 0) + 8 * cg;
  float s[8], m[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) s[i] = m[i] = 0.0f;
  // Eight tokens' loads are issued before their adds, in token order.
  int t = t0;
  for (; t + 8 <= t1; t += 8) {
    float k[8][8], v[8][8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      load8<DT>(p.k, kb + (t + u) * p.kst.t, k[u]);
      load8<DT>(p.v, vb + (t + u) * p.vst.t, v[u]);
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the sixteen loads ahead of the adds
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        s[i] = s[i] + k[u][i];
        m[i] = fmaxf(m[i], fabsf(v[u][i]));
      }
  }
  for (; t < t1; ++t) {
    float k[8], v[8];
    load8<DT>(p.k, kb + t * p.kst.t, k);
    load8<DT>(p.v, vb + t * p.vst.t, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s[i] = s[i] + k[i];
      m[i] = fmaxf(m[i], fabsf(v[i]));
    }
  }
  const int64_t o = (bh * p.chunks + chunk) * kAttnD + 8 * cg;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    p.part_sum[o + i] = s[i];
    p.part_max[o + i] = m[i];
  }
}

// Key mean (the partials added in chunk order, then one division by Nk) and
// the per-channel V scale. The partials are loaded 16 chunks at a time.
__global__ __launch_bounds__(128) void attn_finalize_kernel(AttnPrepParams p) {
  const int d = threadIdx.x;
  const int64_t bh = blockIdx.x;
  const float* ps = p.part_sum + bh * p.chunks * kAttnD + d;
  const float* pm = p.part_max + bh * p.chunks * kAttnD + d;
  float s = 0.0f, m = 0.0f;
  int c = 0;
  for (; c + 16 <= p.chunks; c += 16) {
    float a[16], b[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      a[u] = ps[(int64_t)(c + u) * kAttnD];
      b[u] = pm[(int64_t)(c + u) * kAttnD];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      s = s + a[u];
      m = fmaxf(m, b[u]);
    }
  }
  for (; c < p.chunks; ++c) {
    s = s + ps[(int64_t)c * kAttnD];
    m = fmaxf(m, pm[(int64_t)c * kAttnD]);
  }
  p.kmean[bh * kAttnD + d] = s / (float)p.nk;
  const float sv = row_scale_of(m);
  p.vs[bh * kAttnD + d] = sv;
  p.vrcp[bh * kAttnD + d] = 1.0f / sv;
  p.vsum[bh * kAttnD + d] = 0;   // the quant kernel adds each block's codes
}

// 32 consecutive channels [32 part, 32 part + 32) of token t (16-byte loads).
template <int DT>
__device__ __forceinline__ void load32(const void* base, int64_t off, float (&x)[32]) {
  float a[16], b[16];
  if constexpr (DT == kF32) {
    load16<kF32>(reinterpret_cast<const float*>(base) + off, a);
    load16<kF32>(reinterpret_cast<const float*>(base) + off + 16, b);
  } else {
    load16<kF16>(reinterpret_cast<const uint16_t*>(base) + off, a);
    load16<kF16>(reinterpret_cast<const uint16_t*>(base) + off + 16, b);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    x[i] = a[i];
    x[16 + i] = b[i];
  }
}

__device__ __forceinline__ void store32_i8(int8_t* dst, const int (&q)[32]) {
  uint4 w[2];
  uint32_t* u = reinterpret_cast<uint32_t*>(w);
#pragma unroll
  for (int i = 0; i < 8; ++i) u[i] = pack4(q[4 * i], q[4 * i + 1], q[4 * i + 2], q[4 * i + 3]);
  reinterpret_cast<uint4*>(dst)[0] = w[0];
  reinterpret_cast<uint4*>(dst)[1] = w[1];
}

// 32 consecutive channels of one token row kept as raw 16-byte words, so
// the loads of several rows can be in flight before any is converted.
template <int DT>
struct Raw32 {
  uint4 w[DT == kF32 ? 8 : 4];
};

template <int DT>
__device__ __forceinline__ void load_raw32(const void* base, int64_t off, Raw32<DT>& r) {
  const uint4* q = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + off * (DT == kF32 ? 4 : 2));
#pragma unroll
  for (int i = 0; i < (DT == kF32 ? 8 : 4); ++i) r.w[i] = q[i];
}

template <int DT>
__device__ __forceinline__ void unpack32(const Raw32<DT>& r, float (&x)[32]) {
#pragma unroll
  for (int i = 0; i < (DT == kF32 ? 8 : 4); ++i) {
    const uint32_t u[4] = {r.w[i].x, r.w[i].y, r.w[i].z, r.w[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == kF32) {
        x[4 * i + j] = __uint_as_float(u[j]);
      } else {
        x[8 * i + 2 * j] = h2f((uint16_t)(u[j] & 0xffffu));
        x[8 * i + 2 * j + 1] = h2f((uint16_t)(u[j] >> 16));
      }
    }
  }
}

// Block blk of 64 tokens of one (batch, head): thread (token tid / 4, part
// tid % 4) handles 32 channels. Q rows get their own scale; K rows are
// centred and share one scale per block; V is quantized with the channel
// scales and written transposed (through LDS) in the permuted key order.
template <int DT>
__global__ __launch_bounds__(256) void attn_quant_kernel(AttnPrepParams p) {
  __shared__ __attribute__((aligned(16))) int8_t vtile[kAttnBK * kAttnD];
  __shared__ float wmax[4];
  const int tid = threadIdx.x, tl = tid >> 2, part = tid & 3;
  const int blk = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int t = blk * kAttnBK + tl;
  const int c0 = 32 * part;
  // The Q, K and V rows are loaded up front, in the order they are used
  // (rows past the end re-read the last row and are then ignored).
  Raw32<DT> rq, rk, rv;
  load_raw32<DT>(p.q, p.qst.at(bh, min(t, p.nq - 1)) + c0, rq);
  load_raw32<DT>(p.k, p.kst.at(bh, min(t, p.nk - 1)) + c0, rk);
  load_raw32<DT>(p.v, p.vst.at(bh, min(t, p.nk - 1)) + c0, rv);
  // Both phases run in every workgroup (one basic block keeps the three
  // loads ahead); the stores are masked to the rows that exist.
  const bool q_blk = blk * kAttnBK < p.nq, k_blk = blk < p.nblk;   // workgroup-uniform
  {
    const bool valid = q_blk && t < p.nq;
    float x[32];
    unpack32<DT>(rq, x);
#pragma unroll
    for (int i = 0; i < 32; ++i) x[i] = valid ? x[i] : 0.0f;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    const float s = row_scale_of(amax), rcp = 1.0f / s;
    int q[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = quant1(x[i], s, rcp);
    if (valid) {
      store32_i8(p.q8 + (bh * p.nq + t) * kAttnD + c0, q);
      if (part == 0) p.qs[bh * p.nq + t] = s * p.c0;
    }
  }
  {
    const bool valid = k_blk && t < p.nk;
    const float* mean = p.kmean + bh * kAttnD + c0;
    float x[32];
    unpack32<DT>(rk, x);
#pragma unroll
    for (int i = 0; i < 32; ++i) x[i] = valid ? x[i] - mean[i] : 0.0f;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    amax = wave_max(amax);
    if ((tid & 63) == 0) wmax[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float s = row_scale_of(amax), rcp = 1.0f / s;
    int q[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = quant1(x[i], s, rcp);
    if (k_blk) {
      store32_i8(p.k8 + (bh * p.nkp + t) * kAttnD + c0, q);
      if (tid == 0) p.ks[bh * p.nblk + blk] = s;
    }
    // V: channel scales, then the tile goes through LDS to be transposed.
    const float* vsc = p.vs + bh * kAttnD + c0;
    const float* vrc = p.vrcp + bh * kAttnD + c0;
    unpack32<DT>(rv, x);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float sv = vsc[i];
      q[i] = valid ? quant1(x[i], sv, vrc[i]) : 0;
    }
    store32_i8(vtile + tl * kAttnD + c0, q);
    __syncthreads();
    // Thread (channel ch, 32-key group gq) writes 32 bytes of V^T row ch.
    const int ch = tid >> 1, gq = tid & 1;
    int vb[32];
#pragma unroll
    for (int pos = 0; pos < 32; ++pos) {
      const int key = 8 * ((pos >> 2) & 3) + 4 * (pos >> 4) + (pos & 3);
      vb[pos] = vtile[(32 * gq + key) * kAttnD + ch];
    }
    if (k_blk) {
      store32_i8(p.vt8 + (bh * kAttnD + ch) * (int64_t)p.nkp + blk * kAttnBK + 32 * gq, vb);
      // The block's codes of channel ch, added to its sum over the keys
      // (integer atomics: exact in any order).
      int sum = 0;
#pragma unroll
      for (int pos = 0; pos < 32; ++pos) sum += vb[pos];
      sum += __shfl_xor(sum, 1, 64);
      if (gq == 0) atomicAdd(p.vsum + bh * kAttnD + ch, sum);
    }
  }
}

// Direct global -> LDS load (global_load_lds_dwordx4): lane i's 16 bytes
// land at l + 16 i (l wave-uniform).
__device__ __forceinline__ void lds_dma16(const int8_t* g, int8_t* l) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}

// s_waitcnt vmcnt(0) (loads, including the LDS DMA, have landed).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt vmcnt(N): all but this wave's N most recent vector-memory
// operations (LDS DMA included) done; LDS and export counters unconstrained.
// Workgroup barrier without a memory fence (__syncthreads() would also wait
// for every outstanding DMA): callers wait for the DMA they need with
// wait_vm first, and every LDS read before it has been consumed.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(N | (0x7 << 4) | (0xF << 8));
}

struct AttnParams {
  const int8_t* q8;
  const float* qs;
  const int8_t* k8;
  const float* ks;
  const int8_t* vt8;
  const float* vs;
  const int32_t* vsum;
  void* out;
  Strides3 ost;
  int nq, nk, nkp, nblk;
};

template <int OUT>
__global__ __launch_bounds__(64 * kAttnWaves) void attention_kernel(AttnParams p) {
  // A ring of LDS stages, each [0: K tile, 64 keys x 128 bytes; 1: V^T
  // tile, 128 channels x 64 bytes]. Two passes over the keys: the first
  // finds each query's largest logit (K tiles only, two blocks per stage,
  // three stages), the second quantizes the probabilities against it and
  // accumulates P.V and sum(P) in int32 (one block per stage, four stages).
  // In both, a step computes the next block's scores before working on the
  // current one (the MFMAs run under the VALU work), and every DMA has two
  // steps to land. The stages are separate arrays named by compile-time
  // index, so the compiler sees that reads of one stage do not alias a DMA
  // still landing in another and does not wait for that DMA before them.
  __shared__ __attribute__((aligned(16))) int8_t stage0[2][kAttnBK * kAttnD];
  __shared__ __attribute__((aligned(16))) int8_t stage1[2][kAttnBK * kAttnD];
  __shared__ __attribute__((aligned(16))) int8_t stage2[2][kAttnBK * kAttnD];
  __shared__ __attribute__((aligned(16))) int8_t stage3[2][kAttnBK * kAttnD];
  using Stage = int8_t (*)[kAttnBK * kAttnD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, hh = lane >> 5;
  const int64_t bh = blockIdx.y;
  const int q0 = blockIdx.x * kAttnBQ + wave * kAttnWaveQ;
  const int qrow = min(q0 + fr, p.nq - 1);
  const int8_t* k8 = p.k8 + bh * (int64_t)p.nkp * kAttnD;
  const int8_t* vt8 = p.vt8 + bh * (int64_t)kAttnD * p.nkp;
  // Q fragments (B operand of S^T = K.Q^T): query fr, channels 32 ds + 16 hh + [0, 16).
  v4i qf[4];
  {
    const int8_t* qp = p.q8 + (bh * p.nq + qrow) * kAttnD + 16 * hh;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = *reinterpret_cast<const v4i*>(qp + 32 * ds);
  }
  const float qscale = p.qs[bh * p.nq + qrow];
  // The per-block K scales of the head, staged in LDS (read before the
  // first DMA) so the block loops issue no vector-memory loads besides the
  // DMA and their waits can count it exactly.
  __shared__ float ksc[2048];   // nblk <= 131072 / 64
  for (int i = tid; i < p.nblk; i += 64 * kAttnWaves) ksc[i] = p.ks[bh * p.nblk + i];
  // Tiles are DMA'd global -> LDS, each wave filling 2 KB of each: K rows
  // are 128 bytes with 16-byte chunk c stored at chunk c ^ ((r >> 1) & 7),
  // V^T rows 64 bytes with chunk c at c ^ ((row >> 2) & 3) (the fragment
  // reads, 32 rows of one chunk column, are then free of bank conflicts). A
  // DMA lane writes the next 16 bytes of its instruction's kilobyte, so it
  // loads the chunk that lands on its physical position.
  auto dma_tiles = [&](int j, Stage stg) {
#pragma unroll
    for (int u = 0; u < kAttnDma; ++u) {
      const int kb = kAttnDma * wave + u;
      const int r = 8 * kb + (lane >> 3), kc = (lane & 7) ^ ((r >> 1) & 7);
      lds_dma16(k8 + (int64_t)(kAttnBK * j + r) * kAttnD + 16 * kc, stg[0] + kb * 1024);
      const int ch = 16 * kb + (lane >> 2), vc = (lane & 3) ^ ((ch >> 2) & 3);
      lds_dma16(vt8 + (int64_t)ch * p.nkp + kAttnBK * j + 16 * vc, stg[1] + kb * 1024);
    }
  };
  // S^T of the K tile at kt: sacc[t][4 g + i] is the score of key
  // 32 t + 8 g + 4 hh + i of the block for query fr.
  auto scores_at = [&](const int8_t* kt, v16i (&sacc)[2]) {
    sacc[0] = v16i{};
    sacc[1] = v16i{};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const int r = 32 * t + fr, ck = 2 * ds + hh;
        const v4i kf = *reinterpret_cast<const v4i*>(kt + r * kAttnD + ((ck ^ ((r >> 1) & 7)) << 4));
        sacc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[ds], sacc[t], 0, 0, 0);
      }
  };
  // K tile of block j DMA'd to dst (the layout of dma_tiles).
  auto dma_k = [&](int j, int8_t* dst) {
#pragma unroll
    for (int u = 0; u < kAttnDma; ++u) {
      const int kb = kAttnDma * wave + u;
      const int r = 8 * kb + (lane >> 3), kc = (lane & 7) ^ ((r >> 1) & 7);
      lds_dma16(k8 + (int64_t)(kAttnBK * j + r) * kAttnD + 16 * kc, dst + kb * 1024);
    }
  };
  // Keys of the last block past nk.
  auto masked = [&](int j, int t, int x) { return kAttnBK * j + 32 * t + 8 * (x >> 2) + 4 * hh + (x & 3) >= p.nk; };
  // Pass 1: the largest logit of the query, max over blocks of
  // fp32(max(S) * c_j) (the lane's half of the keys, then the other half).
  // It takes two key blocks per step (K only: block 2u in the K half of a
  // stage, block 2u + 1 in its V half), halving the barriers.
  float ml = -__builtin_inff();
  {
    // A full block (every key below nk): no masks, no checks.
    auto block_max_full = [&](int j, const v16i (&s)[2]) {
      int mx = INT32_MIN;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int x = 0; x < 16; ++x) mx = max(mx, s[t][x]);
      ml = fmaxf(ml, (float)mx * (qscale * ksc[j]));
    };
    auto block_max = [&](int j, const v16i (&s)[2]) {
      int mx = INT32_MIN;
      if (kAttnBK * (j + 1) > p.nk) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int x = 0; x < 16; ++x) mx = masked(j, t, x) ? mx : max(mx, s[t][x]);
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int x = 0; x < 16; ++x) mx = max(mx, s[t][x]);
      }
      if (mx != INT32_MIN) ml = fmaxf(ml, (float)mx * (qscale * ksc[j]));
    };
    const int npairs = (p.nblk + 1) / 2;
    // Every pair issues exactly two DMA instructions per wave, so the waits
    // below count them exactly (the compiler's own wait placement then sees
    // the same counts): past the last block it re-loads in-range blocks
    // into a stage whose scores are never computed.
    auto dma_pair = [&](int u, int8_t (*stg)[kAttnBK * kAttnD]) {
      const int b0 = 2 * min(u, npairs - 1);
      dma_k(b0, stg[0]);
      dma_k(min(b0 + 1, p.nblk - 1), stg[1]);
    };
    auto pair_scores = [&](int u, int8_t (*stg)[kAttnBK * kAttnD], v16i (&s0)[2], v16i (&s1)[2]) {
      scores_at(stg[0], s0);
      if (2 * u + 1 < p.nblk) scores_at(stg[1], s1);
    };
    // Pair u lives in stage u % 3. Step u computes the scores of pair u + 1,
    // refills stage u % 3 (whose scores step u - 1 computed) with pair
    // u + 3, works on pair u, then waits for pair u + 2 only: each DMA has
    // two steps of lead.
    dma_pair(0, stage0);
    dma_pair(1, stage1);
    dma_pair(2, stage2);
    wait_vm<2>();   // pairs 0 and 1 landed
    __syncthreads();
    v16i a0[2], a1[2], b0[2], b1[2];
    pair_scores(0, stage0, a0, a1);
    // Step u with pair u in stage s0 and pair u + 1 in stage s1.
    auto step = [&](int u, int8_t (*s0)[kAttnBK * kAttnD], int8_t (*s1)[kAttnBK * kAttnD],
                    const v16i (&c0)[2], const v16i (&c1)[2], v16i (&n0)[2], v16i (&n1)[2]) {
      if (u + 1 < npairs) pair_scores(u + 1, s1, n0, n1);
      dma_pair(u + 3, s0);
      block_max(2 * u, c0);
      if (2 * u + 1 < p.nblk) block_max(2 * u + 1, c1);
      wait_vm<2>();   // pair u + 2 landed; pair u + 3 may still be in flight
      lds_barrier();
    };
    // The same step for u <= npairs - 3: pairs u and u + 1 are whole and
    // hold no key past nk (only the last block can), so nothing is checked.
    auto step_full = [&](int u, int8_t (*s0)[kAttnBK * kAttnD], int8_t (*s1)[kAttnBK * kAttnD],
                         const v16i (&c0)[2], const v16i (&c1)[2], v16i (&n0)[2], v16i (&n1)[2]) {
      scores_at(s1[0], n0);
      scores_at(s1[1], n1);
      dma_pair(u + 3, s0);
      block_max_full(2 * u, c0);
      block_max_full(2 * u + 1, c1);
      wait_vm<2>();
      lds_barrier();
    };
    // Six steps return to stage 0 and to the first score buffers.
    int u = 0;
    for (; u + 8 <= npairs; u += 6) {
      step_full(u, stage0, stage1, a0, a1, b0, b1);
      step_full(u + 1, stage1, stage2, b0, b1, a0, a1);
      step_full(u + 2, stage2, stage0, a0, a1, b0, b1);
      step_full(u + 3, stage0, stage1, b0, b1, a0, a1);
      step_full(u + 4, stage1, stage2, a0, a1, b0, b1);
      step_full(u + 5, stage2, stage0, b0, b1, a0, a1);
    }
    // At most seven steps remain.
    if (u < npairs) step(u, stage0, stage1, a0, a1, b0, b1);
    if (u + 1 < npairs) step(u + 1, stage1, stage2, b0, b1, a0, a1);
    if (u + 2 < npairs) step(u + 2, stage2, stage0, a0, a1, b0, b1);
    if (u + 3 < npairs) step(u + 3, stage0, stage1, b0, b1, a0, a1);
    if (u + 4 < npairs) step(u + 4, stage1, stage2, a0, a1, b0, b1);
    if (u + 5 < npairs) step(u + 5, stage2, stage0, b0, b1, a0, a1);
    if (u + 6 < npairs) step(u + 6, stage0, stage1, a0, a1, b0, b1);
  }
  const float m = fmaxf(ml, __shfl_xor(ml, 32, 64));
  const float nm = kLog2_255 - m;

  // Pass 2: P = min(255, rne(exp2(fma(S, c_j, nm)))) (v_cvt_pk_u8_f32
  // rounds to nearest even and saturates), O^T += V^T.(P - 128)^T and
  // sum(P - 128), exact in int32.
  v16i oi[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) oi[ct] = v16i{};
  int li = 0;
  auto work = [&](int j, Stage stg, const v16i (&s)[2]) {
    const float c = qscale * ksc[j];
    uint32_t pw[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float qv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf((float)s[t][4 * g + i], c, nm));
        uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(qv[0], 0, 0u);
        w = __builtin_amdgcn_cvt_pk_u8_f32(qv[1], 1, w);
        w = __builtin_amdgcn_cvt_pk_u8_f32(qv[2], 2, w);
        w = __builtin_amdgcn_cvt_pk_u8_f32(qv[3], 3, w);
        pw[t][g] = w ^ 0x80808080u;   // P - 128 as signed bytes
        li = __builtin_amdgcn_sdot4((int)pw[t][g], 0x01010101, li, false);
      }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const v4i pf = {(int)pw[t][0], (int)pw[t][1], (int)pw[t][2], (int)pw[t][3]};
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int r = 32 * ct + fr, ck = 2 * t + hh;
        const v4i vf = *reinterpret_cast<const v4i*>(stg[1] + r * kAttnBK + ((ck ^ ((r >> 2) & 3)) << 4));
        oi[ct] = __builtin_amdgcn_mfma_i32_32x32x32_i8(vf, pf, oi[ct], 0, 0, 0);
      }
    }
  };
  {
    // Block j lives in stage j % 4. Step j computes the scores of block
    // j + 1, refills stage (j + 3) % 4 (read by steps j - 2 and j - 1) with
    // block j + 3, works on block j, then waits for block j + 2 only. Every
    // block issues exactly two DMA instructions per wave (past the last
    // block an in-range block is re-loaded into a stage never read), so the
    // waits count exactly.
    auto dma_blk = [&](int j, Stage stg) { dma_tiles(min(j, p.nblk - 1), stg); };
    dma_blk(0, stage0);
    dma_blk(1, stage1);
    dma_blk(2, stage2);
    wait_vm<2>();   // blocks 0 and 1 landed
    __syncthreads();
    v16i sa[2], sb[2];
    scores_at(stage0[0], sa);
    auto step = [&](int j, Stage s0, Stage s1, Stage s3, const v16i (&cur)[2], v16i (&nxt)[2]) {
      if (j + 1 < p.nblk) scores_at(s1[0], nxt);
      dma_blk(j + 3, s3);
      work(j, s0, cur);
      wait_vm<2>();   // block j + 2 landed; block j + 3 may still be in flight
      lds_barrier();
    };
    // The same step when block j + 1 exists (no check).
    auto step_full = [&](int j, Stage s0, Stage s1, Stage s3, const v16i (&cur)[2], v16i (&nxt)[2]) {
      scores_at(s1[0], nxt);
      dma_blk(j + 3, s3);
      work(j, s0, cur);
      wait_vm<2>();
      lds_barrier();
    };
    int j = 0;
    for (; j + 5 <= p.nblk; j += 4) {
      step_full(j, stage0, stage1, stage3, sa, sb);
      step_full(j + 1, stage1, stage2, stage0, sb, sa);
      step_full(j + 2, stage2, stage3, stage1, sa, sb);
      step_full(j + 3, stage3, stage0, stage2, sb, sa);
    }
    // At most four steps remain.
    if (j < p.nblk) step(j, stage0, stage1, stage3, sa, sb);
    if (j + 1 < p.nblk) step(j + 1, stage1, stage2, stage0, sb, sa);
    if (j + 2 < p.nblk) step(j + 2, stage2, stage3, stage1, sa, sb);
    if (j + 3 < p.nblk) step(j + 3, stage3, stage0, stage2, sb, sa);
  }
  // Each lane summed P - 128 over its 32 keys of every block: sum(P) puts
  // the 128s back. Keys past nk in the last block have all-zero K and V^T
  // codes: each scored 0, added nothing to P.V and the same P =
  // cvt_pk_u8(exp2(fma(0, c, nm))) to this lane's sum; take them out exactly.
  li += 128 * 32 * p.nblk;
  {
    const int jl = p.nblk - 1, kl = p.nk - kAttnBK * jl;
    int npad = 0;
#pragma unroll
    for (int x = 0; x < 32; ++x) npad += (32 * (x >> 4) + 8 * ((x >> 2) & 3) + 4 * hh + (x & 3)) >= kl;
    if (npad) {
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(0.0f, qscale * ksc[jl], nm));
      li -= npad * (int)(__builtin_amdgcn_cvt_pk_u8_f32(e, 0, 0u) & 0xffu);
    }
  }
  const float l = (float)(li + __shfl_xor(li, 32, 64));
  if (q0 + fr >= p.nq) return;
  const int64_t orow = p.ost.at(bh, q0 + fr);
  const float* vsc = p.vs + bh * kAttnD;
  const int* vsm = p.vsum + bh * kAttnD;   // O = O' + 128 * vsum, exact in int64
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = 32 * ct + 8 * g + 4 * hh;
      const float4 s4 = *reinterpret_cast<const float4*>(vsc + c0);
      const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
      const int4 m4 = *reinterpret_cast<const int4*>(vsm + c0);
      const int vm[4] = {m4.x, m4.y, m4.z, m4.w};
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = ((float)((int64_t)oi[ct][4 * g + i] + 128 * (int64_t)vm[i]) * sv[i]) / l;
      if constexpr (OUT == kF32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + orow + c0) = make_float4(y[0], y[1], y[2], y[3]);
      } else {
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + orow + c0) =
            make_uint2(f2h2_of_f32(y[0], y[1]), f2h2_of_f32(y[2], y[3]));
      }
    }
}

static int64_t attn_chunks(int64_t nk) { return (nk + kAttnChunk - 1) / kAttnChunk; }

// Non-negative element strides whose byte sizes are multiples of 16 (the
// kernels move rows in 16-byte pieces).
static bool strides_aligned(const int64_t (&st)[3], int elem) {
  for (int i = 0; i < 3; ++i)
    if (st[i] < 0 || (st[i] * elem) % 16 != 0) return false;
  return true;
}

// True when no two (batch, head, token) rows of 128 contiguous elements
// overlap: taken in increasing stride order, each dimension of size > 1
// steps past everything the smaller ones span.
static bool strides_disjoint(const int64_t (&st)[3], const int64_t (&n)[3]) {
  int order[3] = {0, 1, 2};
  for (int i = 0; i < 3; ++i)
    for (int j = i + 1; j < 3; ++j)
      if (st[order[j]] < st[order[i]]) std::swap(order[i], order[j]);
  int64_t extent = kAttnD;
  for (int i = 0; i < 3; ++i) {
    const int dim = order[i];
    if (n[dim] <= 1) continue;
    if (st[dim] < extent) return false;
    extent += st[dim] * (n[dim] - 1);
  }
  return true;
}

static Strides3 strides3(const int64_t (&st)[3], int64_t heads) { return {st[0], st[1], st[2], (int)heads}; }

}  // namespace w8a8

extern "C" int64_t w8a8_attention_workspace_size(int64_t b, int64_t h, int64_t nk) {
  using namespace w8a8;
  if (b <= 0 || h <= 0 || nk <= 0) return 0;
  return b * h * (2 * attn_chunks(nk) + 2) * kAttnD * (int64_t)sizeof(float);
}

extern "C" int w8a8_attention_prepare(const W8A8AttnPrepareArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_attention_prepare: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8AttnPrepareArgs), "w8a8_attention_prepare: struct_size %u != %zu",
               a->struct_size, sizeof(W8A8AttnPrepareArgs));
  W8A8_REQUIRE(a->in_dtype == W8A8_F16 || a->in_dtype == W8A8_F32, "w8a8_attention_prepare: in_dtype not F16/F32");
  W8A8_REQUIRE(a->d == kAttnD, "w8a8_attention_prepare: head dimension %d != 128", a->d);
  W8A8_REQUIRE(a->b > 0 && a->h > 0 && a->nq > 0 && a->nk > 0, "w8a8_attention_prepare: empty problem");
  W8A8_REQUIRE(a->nq < (1 << 24) && a->nk < (1 << 24) && a->b * a->h < 65536,
               "w8a8_attention_prepare: sizes out of range");
  W8A8_REQUIRE(a->q && a->k && a->v && a->q8 && a->qs && a->k8 && a->ks && a->vt8 && a->vs && a->vsum &&
                   a->workspace,
               "w8a8_attention_prepare: null buffer");
  W8A8_REQUIRE(aligned16(a->q) && aligned16(a->k) && aligned16(a->v) && aligned16(a->q8) && aligned16(a->k8) &&
                   aligned16(a->vt8) && aligned16(a->vs) && aligned16(a->vsum) && aligned16(a->workspace),
               "w8a8_attention_prepare: tensors must be 16-byte aligned");
  W8A8_REQUIRE(a->workspace_bytes >= w8a8_attention_workspace_size(a->b, a->h, a->nk),
               "w8a8_attention_prepare: workspace below w8a8_attention_workspace_size()");
  W8A8_REQUIRE(a->sm_scale > 0.0f, "w8a8_attention_prepare: sm_scale must be positive");
  const int elem = a->in_dtype == W8A8_F16 ? 2 : 4;
  W8A8_REQUIRE(strides_aligned(a->q_strides, elem) && strides_aligned(a->k_strides, elem) &&
                   strides_aligned(a->v_strides, elem),
               "w8a8_attention_prepare: strides must be non-negative multiples of 16 bytes");
  AttnPrepParams p;
  p.q = a->q; p.k = a->k; p.v = a->v;
  p.qst = strides3(a->q_strides, a->h);
  p.kst = strides3(a->k_strides, a->h);
  p.vst = strides3(a->v_strides, a->h);
  p.nq = (int)a->nq; p.nk = (int)a->nk;
  p.nblk = (int)((a->nk + kAttnBK - 1) / kAttnBK);
  p.nkp = p.nblk * kAttnBK;
  p.chunks = (int)attn_chunks(a->nk);
  p.c0 = a->sm_scale * kLog2e;
  p.q8 = a->q8; p.qs = a->qs; p.k8 = a->k8; p.ks = a->ks; p.vt8 = a->vt8; p.vs = a->vs; p.vsum = a->vsum;
  const int64_t bh = a->b * a->h;
  float* ws = reinterpret_cast<float*>(a->workspace);
  p.part_sum = ws;
  p.part_max = ws + bh * p.chunks * kAttnD;
  p.kmean = ws + 2 * bh * p.chunks * kAttnD;
  p.vrcp = p.kmean + bh * kAttnD;
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  const int qblocks = (p.nq + kAttnBK - 1) / kAttnBK;
  const dim3 gstat((unsigned)((p.chunks + 15) / 16), (unsigned)bh), gq((unsigned)max(qblocks, p.nblk), (unsigned)bh);
  if (a->in_dtype == W8A8_F16) {
    hipLaunchKernelGGL(attn_stats_kernel<kF16>, gstat, dim3(256), 0, s, p);
    hipLaunchKernelGGL(attn_finalize_kernel, dim3((unsigned)bh), dim3(128), 0, s, p);
    hipLaunchKernelGGL(attn_quant_kernel<kF16>, gq, dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL(attn_stats_kernel<kF32>, gstat, dim3(256), 0, s, p);
    hipLaunchKernelGGL(attn_finalize_kernel, dim3((unsigned)bh), dim3(128), 0, s, p);
    hipLaunchKernelGGL(attn_quant_kernel<kF32>, gq, dim3(256), 0, s, p);
  }
  return launch_status("w8a8_attention_prepare");
}

extern "C" int w8a8_attention(const W8A8AttentionArgs* a) {
  using namespace w8a8;
  W8A8_REQUIRE(a != nullptr, "w8a8_attention: null args");
  W8A8_REQUIRE(a->struct_size == sizeof(W8A8AttentionArgs), "w8a8_attention: struct_size %u != %zu",
               a->struct_size, sizeof(W8A8AttentionArgs));
  W8A8_REQUIRE(a->out_dtype == W8A8_F16 || a->out_dtype == W8A8_F32, "w8a8_attention: out_dtype not F16/F32");
  W8A8_REQUIRE(a->d == kAttnD, "w8a8_attention: head dimension %d != 128", a->d);
  W8A8_REQUIRE(a->b > 0 && a->h > 0 && a->nq > 0 && a->nk > 0, "w8a8_attention: empty problem");
  W8A8_REQUIRE(a->nq < (1 << 24) && a->nk < (1 << 24) && a->b * a->h < 65536, "w8a8_attention: sizes out of range");
  if (a->nk > (1 << 17)) {   // the int32 sums of (P - 128).V hold nk * 128 * 127
    set_error("w8a8_attention: at most 131072 keys (exact int32 accumulation)");
    return W8A8_ERR_UNSUPPORTED;
  }
  W8A8_REQUIRE(a->q8 && a->qs && a->k8 && a->ks && a->vt8 && a->vs && a->vsum && a->out,
               "w8a8_attention: null buffer");
  W8A8_REQUIRE(aligned16(a->q8) && aligned16(a->k8) && aligned16(a->vt8) && aligned16(a->vs) && aligned16(a->vsum) &&
                   aligned16(a->out),
               "w8a8_attention: tensors must be 16-byte aligned");
  const int64_t extents[3] = {a->b, a->h, a->nq};
  W8A8_REQUIRE(strides_aligned(a->out_strides, a->out_dtype == W8A8_F16 ? 2 : 4),
               "w8a8_attention: out strides must be non-negative multiples of 16 bytes");
  W8A8_REQUIRE(strides_disjoint(a->out_strides, extents), "w8a8_attention: out strides make rows overlap");
  AttnParams p;
  p.q8 = a->q8; p.qs = a->qs; p.k8 = a->k8; p.ks = a->ks; p.vt8 = a->vt8; p.vs = a->vs; p.vsum = a->vsum;
  p.out = a->out;
  p.ost = strides3(a->out_strides, a->h);
  p.nq = (int)a->nq; p.nk = (int)a->nk;
  p.nblk = (int)((a->nk + kAttnBK - 1) / kAttnBK);
  p.nkp = p.nblk * kAttnBK;
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  const dim3 grid((unsigned)((p.nq + kAttnBQ - 1) / kAttnBQ), (unsigned)(a->b * a->h));
  if (a->out_dtype == W8A8_F32) hipLaunchKernelGGL(attention_kernel<kF32>, grid, dim3(64 * kAttnWaves), 0, s, p);
  else hipLaunchKernelGGL(attention_kernel<kF16>, grid, dim3(64 * kAttnWaves), 0, s, p);
  return launch_status("w8a8_attention");
}
