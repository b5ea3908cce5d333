// INT8 attention for 128-wide heads on the reference kernel's scheme
// (SageAttention's qk_int_sv_i8 as vendored by the reference: per-thread-group
// Q and K scales, a one-pass online softmax in the exp2 domain, u8
// probabilities relative to each key block's own maximum, FP32 rescaling of
// the running output and denominators, the per-channel V scale applied at
// the end), for key blocks of 128.
//
// Preparation: key statistics (fp32 chunk sums of K, absmax of V per
// channel), then per 128-token block the Q codes (one scale per 32-row group
// and row mod 8), the centred K codes (four scales per block, one per
// (key mod 8) / 2), the V codes with the channel scales, V^T in the order the
// score tile hands a lane its keys, and 128 times each block's sum of the V
// codes per channel. Codes are sat(round half away(x / s)), s = amax / 127 +
// 1e-7.
//
// Attention: a workgroup of four wavefronts (one per SIMD, two workgroups
// per CU) takes 128 queries of one (batch, head); a wavefront owns 32. Key
// blocks of 128 are DMA'd global -> LDS into two K tiles and two V^T tiles
// (with each wave's copy of the block's V sums): step j reads K of block
// j + 1 and V of block j, then refills the tiles step j - 1 read. Scores are
// computed transposed, S^T = K.Q^T on v_mfma_i32_32x32x32_i8, so a lane
// holds one query (lane % 32) and 64 of the block's keys: exactly the keys of
// two of the four K-scale groups, whose maxima it takes alone. The u8
// probabilities are then already the B operand of O^T = V^T.P^T; the signed
// MFMA takes P - 128, and its accumulator starts from the block's 128 * sum
// of V codes, so it ends with the exact P.V.
#include "w8a8_device.h"
#include "w8a8_host.h"

#include <type_traits>
#include <utility>

namespace w8a8 {

constexpr int kAttnD = 128;        // head dimension
constexpr int kAttnBK = 128;       // keys per block (the reference launcher's CTA_K = 128)
constexpr int kAttnChunk = 256;    // tokens per partial of the key statistics
constexpr int kAttnWaveQ = 32;     // queries per wavefront
constexpr int kAttnWaves = 4;      // wavefronts per workgroup (one per SIMD; two workgroups per CU)
constexpr int kAttnBQ = kAttnWaves * kAttnWaveQ;   // queries per workgroup
constexpr int kAttnTile = kAttnBK * kAttnD;        // bytes of one K or V^T tile
constexpr int kAttnDmaTile = kAttnTile / 1024 / kAttnWaves;   // 1 KB DMA instructions per wave and tile
constexpr int kAttnMaxBlk = 1024;  // nk <= 131072 (32-bit DMA offsets within a head)
constexpr float kLog2e = 0x1.715476p+0f;     // fp32(log2(e))
// The reference's constants (kitchen_attention_native/vendor/attn_utils.cuh:
// S_U8_OFFSET, :40; the running maximum's start and the out-of-bounds score
// of its last-block path).
constexpr float kSU8Offset = 7.9943534f;
constexpr float kMInit = -50000.0f;
constexpr float kMaskScore = -1e30f;
// SageAttention's per-thread quantizers: scale = amax / 127 + 1e-7 (no scale
// is zero, so the out-of-bounds score masks every padded key).
constexpr float kScaleEps = 1e-7f;

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
  int8_t* q8;
  float* qs;
  int8_t* k8;
  float* ks;
  int8_t* vt8;
  float* vs;
  int32_t* vsum;   // [bh, nblk, 128]: 128 * the block's sum of V codes per channel
  float* part_sum;
  float* part_max;
  float* kmean;
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
// the per-channel V scale amax / 127 + 1e-7 (IEEE division). The partials are
// loaded 16 chunks at a time.
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
  p.vs[bh * kAttnD + d] = m / 127.0f + kScaleEps;
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

// The reference quantizer's code of x / s: round half away from zero as
// floor(q + 0.5) for q >= 0 and ceil(q - 0.5) below (each addition rounded
// in fp32), saturated to [-128, 127].
__device__ __forceinline__ int rha_code(float q) {
  const float r = q >= 0.0f ? floorf(q + 0.5f) : ceilf(q - 0.5f);
  return (int)fminf(fmaxf(r, -128.0f), 127.0f);
}

// Block blk of 128 tokens of one (batch, head): thread (token tid / 4, part
// tid % 4) handles 32 channels. Q row 32 G + 8 i + j shares its scale with
// the rows of the same 32-row group G and the same j; centred K key
// 8 t + 2 c + e with the keys of the block of the same c; V takes the channel
// scales, goes through LDS to be written transposed in the permuted key
// order, and each channel's block sum of codes (times 128) is stored.
// Group maxima meet in LDS (integer max of the non-negative fp32 bits).
template <int DT>
__global__ __launch_bounds__(512) void attn_quant_kernel(AttnPrepParams p) {
  __shared__ __attribute__((aligned(16))) int8_t vtile[kAttnBK * kAttnD];
  __shared__ unsigned qmax[32], kmax[4];
  const int tid = threadIdx.x, tl = tid >> 2, part = tid & 3;
  const int blk = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int t = blk * kAttnBK + tl;
  const int c0 = 32 * part;
  // The Q, K and V rows are loaded up front (rows past the end re-read the
  // last row and are then ignored).
  Raw32<DT> rq, rk, rv;
  load_raw32<DT>(p.q, p.qst.at(bh, min(t, p.nq - 1)) + c0, rq);
  load_raw32<DT>(p.k, p.kst.at(bh, min(t, p.nk - 1)) + c0, rk);
  load_raw32<DT>(p.v, p.vst.at(bh, min(t, p.nk - 1)) + c0, rv);
  if (tid < 32) qmax[tid] = 0u;
  if (tid < 4) kmax[tid] = 0u;
  __syncthreads();
  const bool q_blk = blk * kAttnBK < p.nq, k_blk = blk < p.nblk;   // workgroup-uniform
  const bool qvalid = q_blk && t < p.nq, kvalid = k_blk && t < p.nk;
  const int qg = (tl >> 5) * 8 + (tl & 7);   // row 32 G + 8 i + j of the block: group (G, j)
  const int kg = (tl & 7) >> 1;              // key 8 t + 2 c + e of the block: group c
  float xq[32], xk[32];
  unpack32<DT>(rq, xq);
  unpack32<DT>(rk, xk);
  const float* mean = p.kmean + bh * kAttnD + c0;
  float aq = 0.0f, ak = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    xq[i] = qvalid ? xq[i] : 0.0f;
    xk[i] = kvalid ? xk[i] - mean[i] : 0.0f;
    aq = fmaxf(aq, fabsf(xq[i]));
    ak = fmaxf(ak, fabsf(xk[i]));
  }
  atomicMax(&qmax[qg], __float_as_uint(aq));
  atomicMax(&kmax[kg], __float_as_uint(ak));
  __syncthreads();
  if (q_blk) {
    const float s = __uint_as_float(qmax[qg]) / 127.0f + kScaleEps;
    int q[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = rha_code(xq[i] / s);
    if (qvalid) {
      store32_i8(p.q8 + (bh * p.nq + t) * kAttnD + c0, q);
      if (part == 0) p.qs[bh * p.nq + t] = s;
    }
  }
  if (k_blk) {
    const float s = __uint_as_float(kmax[kg]) / 127.0f + kScaleEps;
    int q[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = rha_code(xk[i] / s);
    store32_i8(p.k8 + (bh * p.nkp + t) * kAttnD + c0, q);
    if (tl < 8 && (tl & 1) == 0 && part == 0) p.ks[(bh * p.nblk + blk) * 4 + kg] = s;
    // V: channel scales, then the tile goes through LDS to be transposed.
    const float* vsf = p.vs + bh * kAttnD + c0;
    float xv[32];
    unpack32<DT>(rv, xv);
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = kvalid ? rha_code(xv[i] / vsf[i]) : 0;
    store32_i8(vtile + tl * kAttnD + c0, q);
    __syncthreads();
    // Thread (channel ch, 32-key slice u) writes 32 bytes of V^T row ch:
    // position p of the slice holds key 8 ((p >> 2) & 3) + 4 (p >> 4) + (p & 3).
    const int ch = tid >> 2, u = tid & 3;
    int vb[32];
#pragma unroll
    for (int pos = 0; pos < 32; ++pos) {
      const int key = 32 * u + 8 * ((pos >> 2) & 3) + 4 * (pos >> 4) + (pos & 3);
      vb[pos] = vtile[key * kAttnD + ch];
    }
    store32_i8(p.vt8 + (bh * kAttnD + ch) * (int64_t)p.nkp + blk * kAttnBK + 32 * u, vb);
    int sum = 0;
#pragma unroll
    for (int pos = 0; pos < 32; ++pos) sum += vb[pos];
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    if (u == 0) p.vsum[(bh * p.nblk + blk) * kAttnD + ch] = 128 * sum;
  }
}

// Direct global -> LDS load (global_load_lds_dwordx4): lane i's 16 bytes
// land at l + 16 i (l wave-uniform).
__device__ __forceinline__ void lds_dma16(const int8_t* g, int8_t* l) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}

// Direct global -> LDS load (global_load_lds_dword): lane i's 4 bytes land
// at l + 4 i.
__device__ __forceinline__ void lds_dma4(const int8_t* g, int8_t* l) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)l, 4, 0, 0);
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
  static_assert(N >= 0 && N < 64, "vmcnt range");   // six bits: [3:0] and [15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
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
  float c0;   // fp32(sm_scale * log2(e))
};

// LDS tiles: a block's K (128 keys x 128 bytes), or its V^T (128 channels x
// 128 bytes) with each wave's copy of the block's 128 * V code sums (every
// lane of every wave takes part in every DMA, so no DMA sits behind a lane
// branch). Rows of both tiles are 128 bytes with 16-byte chunk c stored at
// chunk c ^ ((r >> 1) & 7), so the fragment reads (32 rows of one chunk
// column) are free of bank conflicts.
struct AttnKTile {
  int8_t k[kAttnTile];
};
struct AttnVTile {
  int8_t v[kAttnTile];
  int32_t vsum[kAttnWaves][kAttnD];
};

// The reference's online softmax, per query row (the lane's query fr; the
// two half-waves hold the two halves of each 32-key slice):
//   group maxima mt_c over the block's keys of K-scale group c (the last
//     block: keys past nk excluded and a floor of -50000);
//   tile_m = max_c fma(mt_c, ts_c, -S_U8_OFFSET) with ts_c = fp32(c0 *
//     fp32(qs * ks_c)); m' = max(m, tile_m); smaller = exp2(-|m - tile_m|);
//     the state (output and denominators) is scaled by smaller when the tile
//     raises the maximum, the tile's contribution otherwise;
//   P = sat_u8(rne(exp2(fma(S, ts_c, -tile_m))));
//   the denominators add the block's P (u8 codes; the last block: the FP32
//     probabilities) times the tile scale;
//   O += f32(P.V) * tile scale (one FMA), P.V exact in int32;
// finally O * (1 / denominator) * vs. The reference keeps four denominators
// (one per K-scale group, each starting at 1) and adds a group's codes per
// 16-key tile; here a lane keeps one for its two groups, starting at 2, and
// adds the block's code sum (exact in int32) with one FMA, which changes
// only the FP32 rounding of the sum. The exponentials use the hardware
// exp2 (v_exp_f32).
//
// A workgroup is four wavefronts, one per SIMD, and two workgroups share a
// CU (the LDS holds two of everything below), so the two wavefronts on a
// SIMD belong to different workgroups, wait at different barriers and drift
// out of phase: one forms probabilities on the VALU while the other's MFMAs
// run. Step j is software-pipelined: the VALU turns block j's scores into
// probabilities while the MFMAs score block j + 1 into the registers just
// freed, then O^T += V^T.P^T runs while block j + 1's statistics are taken.
// Step j reads K of block j + 1 and V of block j; after its barrier it DMAs
// K of block j + 2 and V of block j + 1 into the tiles that steps j - 1
// read, so two K tiles and two V tiles suffice.
template <int OUT>
__global__ __launch_bounds__(64 * kAttnWaves, 2) void attention_kernel(AttnParams p) {
  // Named by compile-time index so the compiler sees that reads of one tile
  // do not alias a DMA still landing in another.
  __shared__ __attribute__((aligned(16))) AttnKTile ka, kb;
  __shared__ __attribute__((aligned(16))) AttnVTile va, vb;
  extern __shared__ __attribute__((aligned(16))) float ksc[];   // the head's K scales, four per block (16 nblk bytes)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, hh = lane >> 5;
  const int64_t bh = blockIdx.y;
  const int q0 = blockIdx.x * kAttnBQ + wave * kAttnWaveQ;
  const int qrow = min(q0 + fr, p.nq - 1);
  const int8_t* k8 = p.k8 + bh * (int64_t)p.nkp * kAttnD;
  const int8_t* vt8 = p.vt8 + bh * (int64_t)kAttnD * p.nkp;
  const int32_t* vsumh = p.vsum + bh * (int64_t)p.nblk * kAttnD;
  // Q fragments (B operand of S^T = K.Q^T): query fr, channels 32 ds + 16 hh + [0, 16).
  v4i qf[4];
  {
    const int8_t* qp = p.q8 + (bh * p.nq + qrow) * kAttnD + 16 * hh;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = *reinterpret_cast<const v4i*>(qp + 32 * ds);
  }
  const float qsr = p.qs[bh * p.nq + qrow];
  for (int i = tid; i < 4 * p.nblk; i += 64 * kAttnWaves) ksc[i] = p.ks[bh * 4 * p.nblk + i];
  // Each wave DMAs kAttnDmaTile kilobytes of a tile (8 rows per
  // instruction; a lane loads the chunk that lands on its position) and its
  // own copy of the 512 bytes of V sums (two 4-byte DMAs). Blocks past the
  // last are not loaded. The lanes' byte offsets within a block are
  // loop-invariant (32-bit: a head's V^T is at most 128 x 131072 bytes);
  // each block adds a wave-uniform base.
  uint32_t koff[kAttnDmaTile], voff[kAttnDmaTile];
#pragma unroll
  for (int u = 0; u < kAttnDmaTile; ++u) {
    const int r = 8 * (kAttnDmaTile * wave + u) + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
    koff[u] = (uint32_t)(r * kAttnD + 16 * c);
    voff[u] = (uint32_t)(r * p.nkp + 16 * c);
  }
  const uint32_t soff = (uint32_t)(4 * lane);
  auto dma_k = [&](int j, AttnKTile& t) {
    if (j >= p.nblk) return;
    const uint32_t jk = (uint32_t)(j * kAttnBK * kAttnD);
#pragma unroll
    for (int u = 0; u < kAttnDmaTile; ++u) lds_dma16(k8 + (koff[u] + jk), t.k + (kAttnDmaTile * wave + u) * 1024);
  };
  auto dma_v = [&](int j, AttnVTile& t) {
    if (j >= p.nblk) return;
    const uint32_t jv = (uint32_t)(j * kAttnBK), js = (uint32_t)(j * kAttnD * 4);
#pragma unroll
    for (int u = 0; u < kAttnDmaTile; ++u) lds_dma16(vt8 + (voff[u] + jv), t.v + (kAttnDmaTile * wave + u) * 1024);
    const int8_t* vs8 = reinterpret_cast<const int8_t*>(vsumh);
    lds_dma4(vs8 + (soff + js), reinterpret_cast<int8_t*>(t.vsum[wave]));
    lds_dma4(vs8 + (soff + js + 256), reinterpret_cast<int8_t*>(t.vsum[wave]) + 256);
  };
  // Rows of 128 bytes, 16-byte chunk ck of row r at chunk ck ^ ((r >> 1) & 7).
  auto frag = [&](const int8_t* tile, int r, int ck) {
    return *reinterpret_cast<const v4i*>(tile + r * kAttnD + ((ck ^ ((r >> 1) & 7)) << 4));
  };
  // Scores of the block's 32-key slice t: s[4 g + i] is the score of key
  // 32 t + 8 g + 4 hh + i for query fr.
  auto score_slice = [&](const AttnKTile& kt, int t) {
    v16i acc = v16i{};
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(frag(kt.k, 32 * t + fr, 2 * ds + hh), qf[ds], acc, 0, 0, 0);
    return acc;
  };
  // Each lane's value and the other half-wave's (first: lane & 31's,
  // second: lane | 32's).
  auto halves = [](float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return std::make_pair(__uint_as_float(r[0]), __uint_as_float(r[1]));
  };
  // O^T: o[ct][4 g + i] is channel 32 ct + 8 g + 4 hh + i of query fr.
  float o[4][16];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int x = 0; x < 16; ++x) o[ct][x] = 0.0f;
  float m = kMInit, den = 2.0f;
  v16i s[4];                  // the current block's scores
  float tm, ts0, ts1, tsc;    // its tile maximum, the lane's two scales and its tile scale

  // Block j's statistics from s (LAST: keys past nk masked): the group
  // maxima, the tile maximum, the running maximum and the scales. Returns
  // the factor the running state is to be scaled by.
  auto stats = [&](int j, auto last_tag) {
    constexpr bool LAST = decltype(last_tag)::value;
    const int kl = p.nk - kAttnBK * j;
    int mx0 = INT32_MIN, mx1 = INT32_MIN;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = (LAST && 32 * t + 8 * g + 4 * hh + i >= kl) ? INT32_MIN : s[t][4 * g + i];
          if (i < 2) mx0 = max(mx0, v);
          else mx1 = max(mx1, v);
        }
    float mt0 = (float)mx0, mt1 = (float)mx1;
    if constexpr (LAST) {
      mt0 = fmaxf(kMInit, mt0);
      mt1 = fmaxf(kMInit, mt1);
    }
    ts0 = p.c0 * (qsr * ksc[4 * j + 2 * hh]);
    ts1 = p.c0 * (qsr * ksc[4 * j + 2 * hh + 1]);
    tm = fmaxf(__builtin_fmaf(mt0, ts0, -kSU8Offset), __builtin_fmaf(mt1, ts1, -kSU8Offset));
    const auto hv = halves(tm);
    tm = fmaxf(hv.first, hv.second);
    const float mprev = m;
    m = fmaxf(mprev, tm);
    const float smaller = __builtin_amdgcn_exp2f(-fabsf(mprev - tm));
    tsc = tm < mprev ? smaller : 1.0f;
    return mprev < tm ? smaller : 1.0f;
  };
  auto rescale = [&](float osc) {
    if (__builtin_amdgcn_ballot_w64(osc != 1.0f) != 0) {
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int x = 0; x < 16; ++x) o[ct][x] = o[ct][x] * osc;
      den = den * osc;
    }
  };

  // Step j: s holds block j's scores, (tm, ts0, ts1, tsc) its statistics and
  // the running state is already scaled for it. kn holds K of block j + 1,
  // vc V of block j; kr and vr take K of block j + 2 and V of block j + 1.
  // LAST: j is the last block; otherwise block j + 1 (the last when
  // NEXT_LAST) is scored into s on the way and its statistics are taken
  // while block j's P.V runs.
  auto step = [&](int j, const AttnKTile& kn, AttnKTile& kr, const AttnVTile& vc, AttnVTile& vr, auto last_tag,
                  auto next_last_tag) {
    constexpr bool LAST = decltype(last_tag)::value;
    const int kl = p.nk - kAttnBK * j;   // keys of the block below nk (LAST)
    auto masked = [&](int t, int g, int i) { return LAST && 32 * t + 8 * g + 4 * hh + i >= kl; };
    // Every DMA of step j - 1 (K of block j + 1, V of block j) landed and
    // every wave is past step j - 1: refill the tiles it read.
    wait_vm<0>();
    lds_barrier();
    if constexpr (!LAST) {
      dma_k(j + 2, kr);
      dma_v(j + 1, vr);
    }
    // Probabilities as u8 words (w[t][g] byte i: key 32 t + 8 g + 4 hh + i),
    // slice by slice, each slice's registers then taking block j + 1's.
    uint32_t w[4][4];
    uint32_t csum = 0;
    float plast = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float pf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float sf = masked(t, g, i) ? kMaskScore : (float)s[t][4 * g + i];
          pf[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sf, i < 2 ? ts0 : ts1, -tm));
        }
        uint32_t u = __builtin_amdgcn_cvt_pk_u8_f32(pf[0], 0, 0u);
        u = __builtin_amdgcn_cvt_pk_u8_f32(pf[1], 1, u);
        u = __builtin_amdgcn_cvt_pk_u8_f32(pf[2], 2, u);
        w[t][g] = __builtin_amdgcn_cvt_pk_u8_f32(pf[3], 3, u);
        if constexpr (LAST) {
          plast += (pf[0] + pf[1]) + (pf[2] + pf[3]);
        } else {
          csum = __builtin_amdgcn_udot4(w[t][g], 0x01010101u, csum, false);
        }
      }
      if constexpr (!LAST) s[t] = score_slice(kn, t);
    }
    const float tsj = tsc;
    den = __builtin_fmaf(LAST ? plast : (float)csum, tsj, den);
    float osc = 1.0f;
    if constexpr (!LAST) osc = stats(j + 1, next_last_tag);
    // O^T += V^T.P^T per 32-channel tile: the signed MFMA takes P - 128 and
    // starts from 128 * the block's code sums, so acc is P.V exactly.
    v4i pfr[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      pfr[t] = v4i{(int)(w[t][0] ^ 0x80808080u), (int)(w[t][1] ^ 0x80808080u), (int)(w[t][2] ^ 0x80808080u),
                   (int)(w[t][3] ^ 0x80808080u)};
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      v16i acc;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int4 c4 = *reinterpret_cast<const int4*>(vc.vsum[wave] + 32 * ct + 8 * g + 4 * hh);
        acc[4 * g] = c4.x; acc[4 * g + 1] = c4.y; acc[4 * g + 2] = c4.z; acc[4 * g + 3] = c4.w;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(frag(vc.v, 32 * ct + fr, 2 * t + hh), pfr[t], acc, 0, 0, 0);
#pragma unroll
      for (int x = 0; x < 16; ++x) o[ct][x] = __builtin_fmaf((float)acc[x], tsj, o[ct][x]);
    }
    if constexpr (!LAST) rescale(osc);
  };
  using NotLast = std::false_type;
  using Last = std::true_type;
  dma_k(0, ka);
  dma_k(1, kb);
  dma_v(0, va);
  wait_vm<0>();
  __syncthreads();   // the K scales, K of blocks 0 and 1 and V of block 0 are in LDS
#pragma unroll
  for (int t = 0; t < 4; ++t) s[t] = score_slice(ka, t);
  const int nb = p.nblk;
  rescale(nb == 1 ? stats(0, Last{}) : stats(0, NotLast{}));
  // Step j reads K tile (j + 1) % 2 and V tile j % 2. Steps 0 .. nb - 3
  // (neither the block nor the next the last) two at a time; then nb - 2
  // (the next the last) and nb - 1.
  int j = 0;
  for (; j + 2 <= nb - 2; j += 2) {
    step(j, kb, ka, va, vb, NotLast{}, NotLast{});
    step(j + 1, ka, kb, vb, va, NotLast{}, NotLast{});
  }
  if (j < nb - 2) step(j, kb, ka, va, vb, NotLast{}, NotLast{});
  if (nb >= 2) {
    if ((nb - 2) & 1) step(nb - 2, ka, kb, vb, va, NotLast{}, Last{});
    else step(nb - 2, kb, ka, va, vb, NotLast{}, Last{});
  }
  if ((nb - 1) & 1) step(nb - 1, ka, kb, vb, va, Last{}, Last{});
  else step(nb - 1, kb, ka, va, vb, Last{}, Last{});
  // (The last step issued no DMA: nothing targets this workgroup's LDS.)
  const auto dh = halves(den);
  const float rcp = 1.0f / (dh.first + dh.second);
  if (q0 + fr >= p.nq) return;
  const int64_t orow = p.ost.at(bh, q0 + fr);
  const float* vsc = p.vs + bh * kAttnD;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = 32 * ct + 8 * g + 4 * hh;
      const float4 s4 = *reinterpret_cast<const float4*>(vsc + c0);
      const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = (o[ct][4 * g + i] * rcp) * sv[i];
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
  W8A8_REQUIRE(a->nq < (1 << 24) && a->nk <= kAttnMaxBlk * kAttnBK && a->b * a->h < 65536,
               "w8a8_attention_prepare: sizes out of range (at most 131072 keys)");
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
  p.q8 = a->q8; p.qs = a->qs; p.k8 = a->k8; p.ks = a->ks; p.vt8 = a->vt8; p.vs = a->vs; p.vsum = a->vsum;
  const int64_t bh = a->b * a->h;
  float* ws = reinterpret_cast<float*>(a->workspace);
  p.part_sum = ws;
  p.part_max = ws + bh * p.chunks * kAttnD;
  p.kmean = ws + 2 * bh * p.chunks * kAttnD;
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  const int qblocks = (p.nq + kAttnBK - 1) / kAttnBK;
  const dim3 gstat((unsigned)((p.chunks + 15) / 16), (unsigned)bh), gq((unsigned)max(qblocks, p.nblk), (unsigned)bh);
  if (a->in_dtype == W8A8_F16) {
    hipLaunchKernelGGL(attn_stats_kernel<kF16>, gstat, dim3(256), 0, s, p);
    hipLaunchKernelGGL(attn_finalize_kernel, dim3((unsigned)bh), dim3(128), 0, s, p);
    hipLaunchKernelGGL(attn_quant_kernel<kF16>, gq, dim3(512), 0, s, p);
  } else {
    hipLaunchKernelGGL(attn_stats_kernel<kF32>, gstat, dim3(256), 0, s, p);
    hipLaunchKernelGGL(attn_finalize_kernel, dim3((unsigned)bh), dim3(128), 0, s, p);
    hipLaunchKernelGGL(attn_quant_kernel<kF32>, gq, dim3(512), 0, s, p);
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
  W8A8_REQUIRE(a->nq < (1 << 24) && a->b * a->h < 65536, "w8a8_attention: sizes out of range");
  if (a->nk > kAttnMaxBlk * kAttnBK) {   // the limit w8a8_attention_prepare enforces
    set_error("w8a8_attention: at most %d keys", kAttnMaxBlk * kAttnBK);
    return W8A8_ERR_UNSUPPORTED;
  }
  W8A8_REQUIRE(a->sm_scale > 0.0f, "w8a8_attention: sm_scale must be positive");
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
  p.c0 = a->sm_scale * kLog2e;
  hipStream_t s = reinterpret_cast<hipStream_t>(a->stream);
  const dim3 grid((unsigned)((p.nq + kAttnBQ - 1) / kAttnBQ), (unsigned)(a->b * a->h));
  const size_t ksc_bytes = (size_t)16 * p.nblk;   // two workgroups per CU up to 53504 keys or so, one beyond
  if (a->out_dtype == W8A8_F32) hipLaunchKernelGGL(attention_kernel<kF32>, grid, dim3(64 * kAttnWaves), ksc_bytes, s, p);
  else hipLaunchKernelGGL(attention_kernel<kF16>, grid, dim3(64 * kAttnWaves), ksc_bytes, s, p);
  return launch_status("w8a8_attention");
}
