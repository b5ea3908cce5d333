"""CPU oracle of the INT8 attention - TEST INFRASTRUCTURE ONLY.

The reference routes DiT attention through comfy-kitchen 0.2.37's INT8
attention (patches/h3_operator_policy.py:153-209: ``prequantize_int8_attention``
then ``int8_attention_from_prequantized``; patches/kitchen_attention.py:227-238
and the launcher patches/kitchen_attention_native/attention.cu:20-38, which
instantiates the vendored SageAttention kernel ``qk_int_sv_i8_attn_kernel`` of
kitchen_attention_native/vendor/qk_int_sv_i8_cuda.cuh and attn_utils.cuh).
That kernel's arithmetic is restated at the end of this module
(``kitchen_prepare`` / ``kitchen_attention``); Kitchen's quantizer is not in
the reference (comfy-kitchen is not installed), so the restatement assumes
the SageAttention quantizer and is **parity unpinned** for those bits and for
CUDA's approximate exp2 / reciprocal. This build's GPU kernel implements a
different scheme, restated first (``prepare`` / ``attention``): two passes
instead of one online pass, u8 probabilities relative to the row's largest
logit instead of relative to each 64-key tile's largest logit, per-token Q
and per-64-key K scales instead of the kernel's per-thread groups. The GPU
feeds P - 128 to its signed INT8 MFMA and adds 128 * (sum over keys of v8)
per channel afterwards, which gives the same integer P . v8. Its error
against exact attention grows with the key count (max-abs error over max
|output| in tests/test_oracle.py, against the restated reference scheme):

prepare (exact, checked bit for bit):
  * K is centred per channel: mean[d] = (sum over tokens of k[t][d], fp32,
    sequential inside 256-token chunks, then over the chunks) / Nk; kc =
    fp32(k - mean). Centering shifts every logit of a query by the same
    amount, so the softmax is unchanged.
  * Q: per-token scale s = max(amax * fp32(1/127), 1e-30), q8 = sat(rne(q / s))
    (the framework's row quantizer); the stored scale is fp32(s * c0) with
    c0 = fp32(sm_scale * log2(e)), so logits come out in the exp2 domain.
  * K: one scale per 64-key block (amax over the block's 64 x 128 centred
    values), k8 = sat(rne(kc / s)); keys past Nk are zero.
  * V: one scale per channel (amax over all tokens), v8 = sat(rne(v / s)),
    and vsum = sum over the keys of v8 per channel (the GPU's P - 128
    correction).

attention (checked within a tolerance: the GPU's exp2 is the hardware
approximation), per query:
    S = q8 . k8 (int32, exact) and c_j = fp32(qs * ks[j]) for key block j;
    m = max over blocks of fp32(max(S_j) * c_j), the largest logit;
    nm = fp32(log2(255) - m);
    P = min(255, rne(exp2(fma(S, c_j, nm)))), integers 0..255, 0 past Nk;
    acc = P . v8 and l = sum(P), exact integers;
    out = fp32(fp32(f32(acc) * vs) / f32(l)).
"""
import numpy as np

from .w8a8_oracle import R127, SCALE_FLOOR, quantize_rows

F32 = np.float32
LOG2E = F32(1.4426950408889634)
L255 = F32(np.log2(255.0))
BLOCK_K = 64
CHUNK = 256


def _f32(x):
    return np.asarray(x, dtype=np.float32)


def default_scale(d):
    return F32(1.0 / np.sqrt(float(d)))


def perm32():
    """Key of each position of a 32-key group in the transposed V layout.

    Position p = 16 h + 4 g + i holds key 8 g + 4 h + i: the order in which
    the MFMA layout of the score tile hands a lane its keys, so the
    probabilities feed the P.V product without moving between lanes.
    """
    p = np.arange(32)
    return 8 * ((p >> 2) & 3) + 4 * (p >> 4) + (p & 3)


def key_mean(k):
    """Per-channel mean of k [..., N, D] in the prepare kernel's order."""
    k = _f32(k)
    n = k.shape[-2]
    total = np.zeros(k.shape[:-2] + k.shape[-1:], F32)
    for c0 in range(0, n, CHUNK):
        part = np.zeros_like(total)
        for t in range(c0, min(c0 + CHUNK, n)):
            part = part + k[..., t, :]
        total = total + part
    return (total / F32(n)).astype(F32)


def prepare(q, k, v, sm_scale=None):
    """INT8 operands of the attention: dict of q8, qs, k8, ks, vt8, vs, vsum
    (and kmean), for q [B, H, Nq, D], k, v [B, H, Nk, D] (any float dtype)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, h, nq, d = q.shape
    nk = k.shape[2]
    nkp = -(-nk // BLOCK_K) * BLOCK_K
    scale = default_scale(d) if sm_scale is None else F32(sm_scale)
    c0 = F32(scale * LOG2E)
    q8, qsc = quantize_rows(q.reshape(-1, d))
    qs = (qsc * c0).astype(F32).reshape(b, h, nq)
    q8 = q8.reshape(b, h, nq, d)
    mean = key_mean(k)
    kc = np.zeros((b, h, nkp, d), F32)
    kc[:, :, :nk] = (k - mean[:, :, None, :]).astype(F32)
    blocks = kc.reshape(b, h, nkp // BLOCK_K, BLOCK_K * d)
    amax = np.abs(blocks).max(-1)
    ks = np.maximum(amax * R127, SCALE_FLOOR).astype(F32)
    with np.errstate(over='ignore', invalid='ignore', divide='ignore'):
        k8 = np.clip(np.rint(blocks / ks[..., None]), -128, 127).astype(np.int8).reshape(b, h, nkp, d)
    vmax = np.abs(v).max(2)
    vs = np.maximum(vmax * R127, SCALE_FLOOR).astype(F32)
    v8 = np.zeros((b, h, nkp, d), np.int8)
    with np.errstate(over='ignore', invalid='ignore', divide='ignore'):
        v8[:, :, :nk] = np.clip(np.rint(v / vs[:, :, None, :]), -128, 127).astype(np.int8)
    perm = perm32()
    vt8 = v8.reshape(b, h, nkp // 32, 32, d)[:, :, :, perm, :].reshape(b, h, nkp, d).transpose(0, 1, 3, 2).copy()
    vsum = v8.astype(np.int64).sum(2).astype(np.int32)     # per channel, exact (|sum| < 2^31)
    return dict(q8=q8, qs=qs, k8=k8, ks=ks, vt8=vt8, vs=vs, vsum=vsum, kmean=mean, v8=v8, nk=nk)


def attention(prep, out_dtype='f32'):
    """INT8 attention from prepared operands (module docstring).
    Returns [B, H, Nq, D] in out_dtype ('f32' or 'f16')."""
    q8 = prep['q8'].astype(np.int64)
    k8 = prep['k8'].astype(np.int64)
    v8 = prep['v8'].astype(np.int64)
    qs, ks, vs, nk = prep['qs'], prep['ks'], prep['vs'], prep['nk']
    b, h, nq, d = q8.shape
    nkp = k8.shape[2]
    nblk = nkp // BLOCK_K
    valid = np.arange(nkp) < nk
    out = np.zeros((b, h, nq, d), F32)
    for bi in range(b):
        for hi in range(h):
            s = q8[bi, hi] @ k8[bi, hi].T                                  # [nq, nkp] exact
            c = (qs[bi, hi][:, None] * ks[bi, hi][None, :]).astype(F32)   # [nq, nblk]
            cfull = np.repeat(c, BLOCK_K, axis=1)
            smask = np.where(valid[None, :], s, np.iinfo(np.int64).min)
            mblk = smask.reshape(nq, nblk, BLOCK_K).max(-1)
            with np.errstate(over='ignore', invalid='ignore'):
                mj = np.where(mblk > np.iinfo(np.int64).min, (mblk.astype(F32) * c).astype(F32), -np.inf)
                m = mj.max(1).astype(F32)
                nm = (L255 - m).astype(F32)
                e = (s.astype(np.float64) * cfull.astype(np.float64) + nm[:, None]).astype(F32)
                p = np.exp2(e).astype(F32)
            pi = np.where(valid[None, :], np.minimum(np.rint(p), 255), 0).astype(np.int64)
            acc = pi @ v8[bi, hi]
            l = pi.sum(1).astype(F32)
            out[bi, hi] = ((acc.astype(F32) * vs[bi, hi][None, :]).astype(F32) / l[:, None]).astype(F32)
    if out_dtype == 'f16':
        return out.astype(np.float16)
    return out


def reference_attention(q, k, v, sm_scale=None):
    """Exact softmax attention in float64 (the unquantized target)."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    scale = float(default_scale(q.shape[-1]) if sm_scale is None else sm_scale)
    s = np.einsum('bhqd,bhkd->bhqk', q, k) * scale
    s = s - s.max(-1, keepdims=True)
    w = np.exp(s)
    w = w / w.sum(-1, keepdims=True)
    return np.einsum('bhqk,bhkd->bhqd', w, v)


# --------------------------------------------------------------------------
# The reference's vendored kernel, restated.
#
# patches/kitchen_attention_native/attention.cu:20-38 instantiates
# qk_int_sv_i8_attn_kernel (vendor/qk_int_sv_i8_cuda.cuh, comfy-kitchen
# 0.2.37) for 128-wide heads with per-thread Q and K scale granularity, INT8
# V with a fused per-channel V scale, no V mean, FP32 output. Its arithmetic
# per query row, following the vendored source:
#   * scores S = q8 . k8 (int32) for key blocks of CTA_K keys (64, or 128 when
#     Kitchen's packer chooses it: attention.cu:43-66);
#   * the score scale of a (row, key) pair is fp32(c0 * fp32(qs * ks)) with
#     c0 = fp32(sm_scale * log2 e) (qk_int_sv_i8_cuda.cuh:170,546-549); the
#     Q scale is shared by the rows of a 32-row group with the same row mod 8,
#     the K scale by the keys of a block with the same (key mod 8) // 2 - the
#     key set of one thread of the MMA quad (:174-227);
#   * one pass of online softmax in the exp2 domain
#     (attn_utils.cuh:716-790 update_mdo_i32_u8): the tile maximum
#     tile_m = max fma(f32(S), scale, -S_U8_OFFSET) with S_U8_OFFSET = log2 255
#     (attn_utils.cuh:40), the running max m (initially -50000),
#     smaller = exp2(-|m_prev - tile_m|), the old state (output and
#     denominator, initially 0 and 1) scaled by smaller when the tile raises
#     the maximum, the tile's contribution by smaller otherwise;
#   * probabilities P = sat_u8(rne(exp2(fma(f32(S), scale, -tile_m)))) in
#     0..255 relative to the tile's own maximum (mma.cuh:769-781 pack_u8x4);
#   * each thread's denominator adds fp32(sum of four P bytes) * tile_scale;
#     P . V is exact in int32 (m16n8k32 u8 x s8) and the output accumulates
#     fma(f32(P . V), tile_scale, O) (attn_utils.cuh:1148-1186);
#   * the last key block takes the generic path instead
#     (qk_int_sv_i8_cuda.cuh:900-1000, attn_utils.cuh:569-650,918-934): keys
#     past Nk get the raw score -1e30, the tile max starts at -50000 in the
#     raw score domain, and the denominator adds the FP32 probabilities
#     (((p0 + p1) + (p4 + p5)) per 16-key tile) rather than their u8 codes;
#   * finally the quad's four denominators are summed ((d0 + d1) + (d2 + d3)),
#     O is multiplied by 1/d and then by the channel's V scale
#     (attn_utils.cuh:1103-1130, qk_int_sv_i8_cuda.cuh:1054-1071).
#
# Parity unpinned: (1) Kitchen's quantizer (prequantize_int8_attention) is
# absent from the reference; kitchen_prepare assumes the SageAttention
# per-thread quantizer (amax / 127 per group, round half away from zero, K
# centred by its per-channel mean, V per channel). (2) ex2.approx.ftz and
# rcp.approx are CUDA hardware approximations; exact exp2 and 1/d stand in.
# (3) The fp32 updates d += den * ts and O *= o_scale are taken as nvcc
# emits them by default (d += den * ts contracted to one fma).
# --------------------------------------------------------------------------
S_U8_OFFSET = F32(7.9943534)


def _round_half_away(x):
    return np.where(x >= 0, np.floor(x + 0.5), np.ceil(x - 0.5))


def kitchen_prepare(q, k, v, cta_k=64):
    """INT8 operands in the layout qk_int_sv_i8_attn_kernel reads, with one
    effective scale per query row (qs) and per key (ks); see the section
    comment for what is assumed of Kitchen's quantizer."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, h, nq, d = q.shape
    nk = k.shape[2]
    nq32 = -(-nq // 32) * 32
    qp = np.zeros((b, h, nq32, d), F32)
    qp[:, :, :nq] = q
    g = qp.reshape(b, h, nq32 // 32, 4, 8, d)                  # row = 32 G + 8 i + j
    qgs = (np.abs(g).max(axis=(3, 5)) / F32(127)).astype(F32)  # [b, h, G, 8]
    safe = np.where(qgs > 0, qgs, F32(1))
    q8 = np.clip(_round_half_away(g / safe[:, :, :, None, :, None]), -128, 127).astype(np.int8)
    q8 = q8.reshape(b, h, nq32, d)[:, :, :nq]
    qs = np.broadcast_to(qgs[:, :, :, None, :], (b, h, nq32 // 32, 4, 8)).reshape(b, h, nq32)[:, :, :nq]
    mean = (k.astype(np.float64).sum(2) / nk).astype(F32)
    nkp = -(-nk // cta_k) * cta_k
    kc = np.zeros((b, h, nkp, d), F32)
    kc[:, :, :nk] = (k - mean[:, :, None, :]).astype(F32)
    kb = kc.reshape(b, h, nkp // cta_k, cta_k // 8, 4, 2, d)    # key = cta_k B + 8 t + 2 c + e
    kgs = (np.abs(kb).max(axis=(3, 5, 6)) / F32(127)).astype(F32)   # [b, h, B, 4]
    safe = np.where(kgs > 0, kgs, F32(1))
    k8 = np.clip(_round_half_away(kb / safe[:, :, :, None, :, None, None]), -128, 127).astype(np.int8)
    k8 = k8.reshape(b, h, nkp, d)
    ks = np.broadcast_to(kgs[:, :, :, None, :, None], kb.shape[:-1]).reshape(b, h, nkp)
    vs = (np.abs(v).max(2) / F32(127)).astype(F32)
    safe = np.where(vs > 0, vs, F32(1))
    v8 = np.zeros((b, h, nkp, d), np.int8)
    v8[:, :, :nk] = np.clip(_round_half_away(v / safe[:, :, None, :]), -128, 127).astype(np.int8)
    return dict(q8=q8, qs=np.ascontiguousarray(qs), k8=k8, ks=np.ascontiguousarray(ks), v8=v8, vs=vs, nk=nk,
                cta_k=cta_k)


def _exp2(x):
    with np.errstate(over='ignore', under='ignore'):
        return np.exp2(_f32(x).astype(np.float64)).astype(F32)


def kitchen_attention(prep, sm_scale=None):
    """qk_int_sv_i8_attn_kernel's arithmetic (section comment) on
    kitchen_prepare's operands: [B, H, Nq, D] fp32."""
    from .w8a8_oracle import fma_f32
    q8 = prep['q8'].astype(np.int64)
    k8 = prep['k8'].astype(np.int64)
    v8 = prep['v8'].astype(np.int64)
    qs, ks, vs, nk, ck = prep['qs'], prep['ks'], prep['vs'], prep['nk'], prep['cta_k']
    b, h, nq, d = q8.shape
    nkp = k8.shape[2]
    nblk = nkp // ck
    c0 = F32(F32(default_scale(d) if sm_scale is None else sm_scale) * LOG2E)
    key = np.arange(ck)
    thread = (key % 8) // 2                      # the quad thread holding each key of a block
    tile = key // 16
    in_tile = key % 16
    out = np.zeros((b, h, nq, d), F32)
    for bi in range(b):
        for hi in range(h):
            s_all = q8[bi, hi] @ k8[bi, hi].T                       # exact
            m = np.full(nq, F32(-50000.0), F32)
            dsum = np.ones((nq, 4), F32)
            o = np.zeros((nq, d), F32)
            for bj in range(nblk):
                keys = bj * ck + key
                s = s_all[:, keys]
                kscale = ks[bi, hi][keys]                            # per key (constant per thread)
                sc = (c0 * (qs[bi, hi][:, None] * kscale[None, :]).astype(F32)).astype(F32)   # [nq, ck]
                last = bj == nblk - 1
                if last:
                    sf = np.where(keys[None, :] < nk, s.astype(F32), F32(-1e30))
                    mt = np.stack([np.maximum(F32(-50000.0), sf[:, thread == c].max(1)) for c in range(4)], 1)
                else:
                    sf = s.astype(F32)
                    mt = np.stack([sf[:, thread == c].max(1) for c in range(4)], 1)
                tsc = np.stack([sc[:, np.argmax(thread == c)] for c in range(4)], 1)   # the thread's scale
                tile_m = fma_f32(mt, tsc, -S_U8_OFFSET).max(1)
                m_prev = m
                m = np.maximum(m_prev, tile_m)
                smaller = _exp2(-np.abs(m_prev - tile_m))
                o_scale = np.where(m_prev < tile_m, smaller, F32(1))
                t_scale = np.where(tile_m < m_prev, smaller, F32(1))
                dsum = (dsum * o_scale[:, None]).astype(F32)
                o = (o * o_scale[:, None]).astype(F32)
                p = _exp2(fma_f32(sf, sc, -tile_m[:, None]))
                u8 = np.clip(np.rint(p), 0, 255).astype(np.int64)
                for c in range(4):
                    for t in range(ck // 16):
                        sel = [16 * t + 2 * c, 16 * t + 2 * c + 1, 16 * t + 8 + 2 * c, 16 * t + 9 + 2 * c]
                        if last:
                            part = ((p[:, sel[0]] + p[:, sel[1]]).astype(F32)
                                    + (p[:, sel[2]] + p[:, sel[3]]).astype(F32)).astype(F32)
                        else:
                            part = u8[:, sel].sum(1).astype(F32)
                        dsum[:, c] = fma_f32(part, t_scale, dsum[:, c])
                pv = u8 @ v8[bi, hi][keys]                          # exact int32
                o = fma_f32(pv.astype(F32), t_scale[:, None], o)
            dt = ((dsum[:, 0] + dsum[:, 1]).astype(F32) + (dsum[:, 2] + dsum[:, 3]).astype(F32)).astype(F32)
            rcp = (F32(1) / dt).astype(F32)
            out[bi, hi] = ((o * rcp[:, None]).astype(F32) * vs[bi, hi][None, :]).astype(F32)
    return out
