"""Operator selection for the INT8 projections (subset of the reference policy).

Mirrors the linear-path fields and dispatch of patches/h3_operator_policy.py
(H3OperatorPolicy :9-41, row_linear :213-237, row_linear_parts :240-255).
Attention, RMS-RoPE and lifetime switches of the reference are not part of
this path and are not represented.
"""
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class H3OperatorPolicy:
    row_linear_backend: str = 'tilelang_scaled_fp16'
    fc2_quantizer: str = 'fused_stored'
    column_linear_backend: str = 'cuda_int8_tilelang'

    def __post_init__(self):
        if self.row_linear_backend not in ('tilelang_packed', 'tilelang_scaled_fp16', 'native'):
            raise ValueError('Unknown row-linear backend')
        if self.fc2_quantizer not in ('native', 'owned_fp32', 'fused_stored', 'fused_recompute'):
            raise ValueError('Unknown FC2 quantizer')
        if self.column_linear_backend not in ('preallocated', 'cuda_int8_tilelang'):
            raise ValueError('Unknown column linear backend')


def configure_block(block, kind, policy):
    """Attach the policy to a block's projections (h3_operator_policy.py:56-75, linear part)."""
    block.operator_policy = policy
    names = ('o_proj', 'down_proj', 'q_proj', 'k_proj', 'v_proj', 'gate_proj', 'up_proj') if kind == 'te' \
        else ('out_proj', 'fc2', 'qkv_proj', 'fc1')
    for name in names:
        module = getattr(block, name, None)
        if module is not None:
            module.operator_policy = policy
    return block


def row_linear(module, x, fallback, comm, input_act=None, residual=None, gate=None, segments=None):
    """Dispatch a row projection; the fused SwiGLU route when the policy selects it.

    ``residual`` (FP16, optional) is fused into the GEMM epilogue on the fused
    route; on the fallback it is added after the storage cast. With ``gate``
    (fp32 [R, N] DiT modulation table) and ``segments`` [(a, b, row)] the
    update is the gated one (tp_dit.py:160-162 -> h3_tensor_flow.gated_add);
    the fused route needs segments that tile the rows.
    """
    from . import swiglu_quant as quant
    policy = getattr(module, 'operator_policy', None)
    fused = (policy is not None and policy.fc2_quantizer in ('fused_stored', 'fused_recompute')
             and input_act == 'swiglu' and policy.row_linear_backend != 'native')
    labels = None
    if gate is not None:
        if residual is None:
            raise ValueError('the gate scales the residual update: residual required')
        rows = x.reshape(-1, x.shape[-1]).shape[0]
        from .h3_tensor_flow import labels_for
        labels = labels_for(rows, segments, gate.shape[0], device=x.device)
    if fused and (gate is None or labels is not None) and quant.supported(
            x, module.weight, module.weight_scale, module.world_size, module.convrot_groupsize):
        return quant.row_linear(x, module.weight, module.weight_scale, comm, mode=policy.fc2_quantizer,
                                scaled_transport=policy.row_linear_backend == 'tilelang_scaled_fp16',
                                residual=residual, gate=gate, gate_labels=labels)
    if (input_act is None and residual is not None and (gate is None or labels is not None)
            and policy is not None and policy.row_linear_backend != 'native' and module.world_size == 1
            and module.convrot and module.convrot_groupsize == 256
            and x.dtype in (torch.float16, torch.float32) and residual.dtype == torch.float16):
        # The O projection with the (gated) residual update in the GEMM
        # epilogue: patches/tilelang_dit_fusion.py:153-199 (row_gated ->
        # tilelang_transport_p2.row_linear on value.float(), finish_row):
        # ConvRot256 in FP32, row-order dequant, fp16(fma(branch, gate, X)).
        from . import kernels
        flat = x.reshape(-1, x.shape[-1])
        q, scale = kernels.quantize_rows(flat, convrot=True, round_rotated=False)
        n = module.weight.shape[0]
        out = kernels.gemm(q, module.weight, epilogue=kernels.EPI_ROW, row_scale=scale,
                           col_scale=module.weight_scale, out_dtype=torch.float16,
                           residual=residual.reshape(-1, n), gate=gate, gate_labels=labels)
        return out.reshape(*x.shape[:-1], n)
    if input_act == 'swiglu' or (policy is not None and policy.row_linear_backend == 'tilelang_scaled_fp16'):
        # FP32 preparation island, as the reference keeps on fallback geometry.
        x = x.float()
    out = fallback(x, module.weight, module.weight_scale, comm, module.world_size, module.convrot_groupsize,
                   input_act)
    if residual is not None:
        from .h3_tensor_flow import gated_add, residual_add
        if gate is not None:
            return gated_add(residual, gate, out.to(residual.dtype), segments)
        out = residual_add(residual, out.to(residual.dtype))
    return out


def adjacent_cat(gate, up):
    """cat((gate, up), -1), without a copy when up directly follows gate in
    the columns of one buffer (project_columns' packed output)."""
    g2 = gate.reshape(-1, gate.shape[-1])
    u2 = up.reshape(-1, up.shape[-1])
    w = g2.shape[1]
    if (g2.stride(1) == 1 and u2.stride(1) == 1 and g2.stride(0) == u2.stride(0)
            and u2.data_ptr() == g2.data_ptr() + w * g2.element_size()
            and g2.untyped_storage().data_ptr() == u2.untyped_storage().data_ptr()):
        return g2.as_strided((g2.shape[0], 2 * w), (g2.stride(0), 1)).view(*gate.shape[:-1], 2 * w)
    return torch.cat((gate, up), -1)


def row_linear_parts(module, gate, up, fallback, comm):
    """TE down projection from separate gate/up halves (h3_operator_policy.py:240-255).

    With a fused FC2 quantizer (and a non-native row backend) the halves are
    concatenated and run through the fused FP32 SwiGLU route; only that route
    requires matching halves. Otherwise the product silu(gate) * up is formed
    in the halves' own dtype (torch's elementwise ops, with their storage
    rounding and FP16 overflow, as the reference's eager fallback) and the
    row projection runs with no input activation.
    """
    policy = getattr(module, 'operator_policy', None)
    if (policy is not None and policy.row_linear_backend != 'native'
            and policy.fc2_quantizer in ('fused_stored', 'fused_recompute')):
        if gate.shape != up.shape or gate.dtype != up.dtype or gate.device != up.device:
            raise ValueError('Matching gate/up required')
        return row_linear(module, adjacent_cat(gate, up), fallback, comm, 'swiglu')
    return row_linear(module, torch.nn.functional.silu(gate) * up, fallback, comm)
