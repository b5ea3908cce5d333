"""INT8 attention (the reference's Kitchen INT8 attention API).

Same names as the reference's calls into comfy-kitchen 0.2.37
(patches/h3_operator_policy.py:153-209: ``prequantize_int8_attention`` and
``int8_attention_from_prequantized``; patches/kitchen_attention.py:227-238:
``int8_attention(q, k, v, *, scale=None, attn_mask=None)``), for 128-wide
heads without masks. q, k, v are [batch, heads, tokens, 128] fp16 or fp32; the
output has q's dtype. Two libw8a8 calls with the numerics of the reference's
vendored kernel (kitchen_attention_native/vendor/qk_int_sv_i8_cuda.cuh) for
128-key blocks: the preparation (per-thread-group Q and K scales, K centred,
per-channel V scales, INT8 codes, V transposed, per-block V code sums) and the
attention kernel (INT8 MFMA for Q.K^T and P.V, one online-softmax pass with u8
probabilities relative to each key block's maximum and FP32 rescaling).
"""
from dataclasses import dataclass

import torch

from . import kernels


@dataclass
class PreparedAttention:
    """INT8 operands of one attention call (device tensors) and the output dtype."""
    operands: dict
    out_dtype: torch.dtype

    def release(self):
        self.operands = None


def prequantize_int8_attention(q, k, v, *, scale=None, attn_mask=None):
    """patches/h3_operator_policy.py:190 (ck.prequantize_int8_attention)."""
    if attn_mask is not None:
        raise ValueError('attention masks are not supported by the INT8 attention')
    return PreparedAttention(kernels.attention_prepare(q, k, v, sm_scale=scale), q.dtype)


def int8_attention_from_prequantized(prepared):
    """patches/h3_operator_policy.py:209 (ck.int8_attention_from_prequantized)."""
    if prepared.operands is None:
        raise ValueError('prepared attention was released')
    return kernels.attention(prepared.operands, out_dtype=prepared.out_dtype)


def int8_attention(q, k, v, *, scale=None, attn_mask=None):
    """patches/kitchen_attention.py:227-238: attention of [B, H, N, 128] q, k, v."""
    return int8_attention_from_prequantized(prequantize_int8_attention(q, k, v, scale=scale, attn_mask=attn_mask))
