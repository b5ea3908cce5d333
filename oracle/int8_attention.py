"""CPU oracle of the INT8 attention - TEST INFRASTRUCTURE ONLY.

The reference routes DiT attention through comfy-kitchen 0.2.37's INT8
attention (patches/h3_operator_policy.py:153-209: ``prequantize_int8_attention``
then ``int8_attention_from_prequantized``; patches/kitchen_attention.py:227-238
and the launcher patches/kitchen_attention_native/attention.cu:20-38, which
instantiates the vendored SageAttention kernel ``qk_int_sv_i8_attn_kernel``).
The kernel header and Kitchen's quantizers are not in the reference
(kitchen_attention_native/vendor is empty; comfy-kitchen is not installed), so
their bits cannot be reproduced: **parity with the reference is unpinned**.
This module restates the algorithm this build implements, which follows the
published SageAttention scheme and the properties the reference's design
notes record (docs/design/TP2_GROUP32_KITCHEN_DESIGN.md:35-45: INT8 Q/K with
scales covering the channel reduction, key centering, signed INT8 V,
quantized probabilities for an integer P.V, FP32 softmax and output state,
exp2-domain online softmax):

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
  * V: one scale per channel (amax over all tokens), v8 = sat(rne(v / s)).

attention (checked within a tolerance: the GPU's exp2 is the hardware
approximation), per query:
    S = q8 . k8 (int32, exact) and c_j = fp32(qs * ks[j]) for key block j;
    m = max over blocks of fp32(max(S_j) * c_j), the largest logit;
    nm = fp32(fp32(log2(127) - m) - fp32(|m| * 2^-22));
    P = rne(exp2(fma(S, c_j, nm))), integers 0..127 (the 2^-22 margin keeps
    the largest exponent within a few ulps of log2(127)), 0 past Nk;
    acc = P . v8 and l = sum(P), exact integers;
    out = fp32(fp32(f32(acc) * vs) / f32(l)).
"""
import numpy as np

from .w8a8_oracle import R127, SCALE_FLOOR, quantize_rows

F32 = np.float32
LOG2E = F32(1.4426950408889634)
L127 = F32(np.log2(127.0))
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
    """INT8 operands of the attention: dict of q8, qs, k8, ks, vt8, vs (and
    kmean), for q [B, H, Nq, D], k, v [B, H, Nk, D] (any float dtype)."""
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
    return dict(q8=q8, qs=qs, k8=k8, ks=ks, vt8=vt8, vs=vs, kmean=mean, v8=v8, nk=nk)


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
                nm = ((L127 - m).astype(F32) - (np.abs(m) * F32(2.0 ** -22)).astype(F32)).astype(F32)
                e = (s.astype(np.float64) * cfull.astype(np.float64) + nm[:, None]).astype(F32)
                p = np.exp2(e).astype(F32)
            pi = np.where(valid[None, :], np.rint(p), 0).astype(np.int64)
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
