"""CPU oracle of the INT8 attention - TEST INFRASTRUCTURE ONLY.

The reference routes DiT attention through comfy-kitchen 0.2.37's INT8
attention (patches/h3_operator_policy.py:153-209: ``prequantize_int8_attention``
then ``int8_attention_from_prequantized``; patches/kitchen_attention.py:227-238
and the launcher patches/kitchen_attention_native/attention.cu:20-66, which
instantiates the vendored SageAttention kernel ``qk_int_sv_i8_attn_kernel`` of
kitchen_attention_native/vendor/qk_int_sv_i8_cuda.cuh and attn_utils.cuh for
key blocks of CTA_K = 64 or 128, as Kitchen's packer chooses). That kernel's
arithmetic is restated here (``kitchen_prepare`` / ``kitchen_attention``),
and the GPU kernel implements it for CTA_K = 128. Kitchen's quantizer is not
in the reference (comfy-kitchen is not installed), so the restatement assumes
the SageAttention quantizer, with the key mean in a fixed fp32 order
(``key_mean``), and is **parity unpinned** for those bits and for CUDA's
approximate exp2 / reciprocal. ``reference_attention`` is exact softmax
attention in float64, the unquantized target both are measured against.
"""
import numpy as np

from .w8a8_oracle import R127, SCALE_FLOOR, quantize_rows

F32 = np.float32
LOG2E = F32(1.4426950408889634)
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
# centred by its per-channel mean, V per channel; scale = amax / 127 + 1e-7). (2) ex2.approx.ftz and
# rcp.approx are CUDA hardware approximations; exact exp2 and 1/d stand in.
# (3) The fp32 updates d += den * ts and O *= o_scale are taken as nvcc
# emits them by default (d += den * ts contracted to one fma).
# --------------------------------------------------------------------------
S_U8_OFFSET = F32(7.9943534)
# SageAttention's per-thread quantizers take scale = amax / 127 + 1e-7, so no
# scale is zero (an all-padding K group of the last block would otherwise
# zero the score scale that masks its keys).
SCALE_EPS = F32(1e-7)


def _round_half_away(x):
    return np.where(x >= 0, np.floor(x + 0.5), np.ceil(x - 0.5))


def kitchen_prepare(q, k, v, cta_k=64, sm_scale=None):
    """INT8 operands in the layout qk_int_sv_i8_attn_kernel reads, with one
    effective scale per query row (qs) and per key (ks); see the section
    comment for what is assumed of Kitchen's quantizer. Also the layouts the
    GPU kernel reads: ksg [B, H, Nkp / CTA_K, 4] (the four K scales of each
    block, group c = (key mod 8) // 2), vt8 [B, H, D, Nkp] (V^T with key
    perm32()[p] of each 32-key group at position p) and vsum128
    [B, H, Nkp / CTA_K, D] (128 times each block's sum of V codes per
    channel: the GPU's signed MFMA takes P - 128)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, h, nq, d = q.shape
    nk = k.shape[2]
    nq32 = -(-nq // 32) * 32
    qp = np.zeros((b, h, nq32, d), F32)
    qp[:, :, :nq] = q
    g = qp.reshape(b, h, nq32 // 32, 4, 8, d)                  # row = 32 G + 8 i + j
    qgs = (np.abs(g).max(axis=(3, 5)) / F32(127) + SCALE_EPS).astype(F32)  # [b, h, G, 8]
    q8 = np.clip(_round_half_away(g / qgs[:, :, :, None, :, None]), -128, 127).astype(np.int8)
    q8 = q8.reshape(b, h, nq32, d)[:, :, :nq]
    qs = np.broadcast_to(qgs[:, :, :, None, :], (b, h, nq32 // 32, 4, 8)).reshape(b, h, nq32)[:, :, :nq]
    mean = key_mean(k)
    nkp = -(-nk // cta_k) * cta_k
    kc = np.zeros((b, h, nkp, d), F32)
    kc[:, :, :nk] = (k - mean[:, :, None, :]).astype(F32)
    kb = kc.reshape(b, h, nkp // cta_k, cta_k // 8, 4, 2, d)    # key = cta_k B + 8 t + 2 c + e
    kgs = (np.abs(kb).max(axis=(3, 5, 6)) / F32(127) + SCALE_EPS).astype(F32)   # [b, h, B, 4]
    k8 = np.clip(_round_half_away(kb / kgs[:, :, :, None, :, None, None]), -128, 127).astype(np.int8)
    k8 = k8.reshape(b, h, nkp, d)
    ks = np.broadcast_to(kgs[:, :, :, None, :, None], kb.shape[:-1]).reshape(b, h, nkp)
    vs = (np.abs(v).max(2) / F32(127) + SCALE_EPS).astype(F32)
    v8 = np.zeros((b, h, nkp, d), np.int8)
    v8[:, :, :nk] = np.clip(_round_half_away(v / vs[:, :, None, :]), -128, 127).astype(np.int8)
    perm = perm32()
    vt8 = v8.reshape(b, h, nkp // 32, 32, d)[:, :, :, perm, :].reshape(b, h, nkp, d).transpose(0, 1, 3, 2).copy()
    vsum128 = (v8.astype(np.int32).reshape(b, h, nkp // cta_k, cta_k, d).sum(3) * 128).astype(np.int32)
    scale = default_scale(d) if sm_scale is None else F32(sm_scale)
    return dict(q8=q8, qs=np.ascontiguousarray(qs), k8=k8, ks=np.ascontiguousarray(ks), v8=v8, vs=vs, nk=nk,
                cta_k=cta_k, ksg=np.ascontiguousarray(kgs), vt8=vt8, vsum128=vsum128, kmean=mean,
                sm_scale=scale)


# The key block of the GPU kernel (the reference launcher's CTA_K = 128) and
# the prepared tensors it reads.
GPU_CTA_K = 128
GPU_OPERANDS = ('q8', 'qs', 'k8', 'ks', 'vt8', 'vs', 'vsum')


def gpu_operands(prep):
    """kitchen_prepare's tensors under the GPU preparation's names and layouts."""
    return dict(q8=prep['q8'], qs=prep['qs'], k8=prep['k8'], ks=prep['ksg'], vt8=prep['vt8'], vs=prep['vs'],
                vsum=prep['vsum128'])


def _exp2(x):
    with np.errstate(over='ignore', under='ignore'):
        return np.exp2(_f32(x).astype(np.float64)).astype(F32)


def kitchen_attention(prep, sm_scale=None):
    """qk_int_sv_i8_attn_kernel's arithmetic (section comment) on
    kitchen_prepare's operands: [B, H, Nq, D] fp32 (sm_scale defaults to the
    one kitchen_prepare recorded)."""
    from .w8a8_oracle import fma_f32
    q8 = prep['q8'].astype(np.int64)
    k8 = prep['k8'].astype(np.int64)
    v8 = prep['v8'].astype(np.int64)
    qs, ks, vs, nk, ck = prep['qs'], prep['ks'], prep['vs'], prep['nk'], prep['cta_k']
    b, h, nq, d = q8.shape
    nkp = k8.shape[2]
    nblk = nkp // ck
    c0 = F32(F32(prep.get('sm_scale', default_scale(d)) if sm_scale is None else sm_scale) * LOG2E)
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
