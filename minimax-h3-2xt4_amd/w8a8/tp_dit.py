"""INT8 projection modules (the reference's tp_dit API) on one GPU.

ColumnParallelLinearINT8 / RowParallelLinearINT8 keep the attribute names of
patches/tp_dit.py:25-162 (weight int8 [N, K], weight_scale fp32 [N, 1],
convrot, convrot_groupsize, world_size, in/out features) so shards load the
same way. At world_size 1 there is no exchange. A module holding one rank's
shard (world_size 2, e.g. checkpoint.load_block(rank=r, world_size=2)) runs
that shard at its real shape: a column shard is complete by itself; a row
shard exposes the two points where the reference exchanges data
(local_maximum before the MAX, partial before the SUM) and its forward
returns the FP32 partial. DiTAttentionINT8 is the attention sublayer of
TPDiTBlockINT8.forward (patches/tp_dit.py:277-345: modulated norm -> QKV ->
RMS-RoPE -> INT8 attention -> O + gated residual), DiTFeedForwardINT8 the
FC1 -> SwiGLU/ConvRot256 -> FC2 (+ residual) part (patches/tp_dit.py:347-362),
and chunked_rows runs any of them over M in fixed row chunks with the
weights resident.
"""
import torch
from torch import nn

from . import kernels, parallel_int8
from .dit_column_linear import column_linear, column_linear_quantized
from .h3_tensor_flow import modulated_norm_quantize
from .h3_operator_policy import H3OperatorPolicy, row_linear as dispatch_row
from .rms_rope import fused_qkv


class ColumnParallelLinearINT8(nn.Module):
    """Output-feature split INT8 projection (patches/tp_dit.py:25-96)."""

    def __init__(self, in_features, out_features, rank=0, world_size=1, convrot=True, convrot_groupsize=256,
                 device=None, components=1):
        super().__init__()
        if out_features % world_size:
            raise ValueError('out_features must divide across ranks')
        self.components = components
        self.in_features = in_features
        self.out_features_per_rank = out_features // world_size
        self.rank = rank
        self.world_size = world_size
        self.convrot = convrot
        self.convrot_groupsize = convrot_groupsize
        self.device = torch.device(device) if device is not None else torch.device('cuda', 0)
        self.weight = nn.Parameter(torch.empty(self.out_features_per_rank, in_features, dtype=torch.int8,
                                               device=self.device), requires_grad=False)
        self.weight_scale = nn.Parameter(torch.empty(self.out_features_per_rank, 1, dtype=torch.float32,
                                                     device=self.device), requires_grad=False)

    def load_shard_from_full(self, full_weight, full_scale):
        w, scale = parallel_int8.packed_rows(full_weight, full_scale, self.rank, self.world_size, self.components)
        self.weight.data.copy_(w)
        self.weight_scale.data.copy_(scale)

    def forward(self, x, *, prepared=None):
        """``prepared`` = (codes, row_scale) of x already rotated and quantized
        (modulated_norm_quantize); x then only supplies the shape and dtype."""
        if prepared is not None:
            out = column_linear_quantized(prepared[0], prepared[1], self.weight, self.weight_scale,
                                          out_dtype=x.dtype)
            return out.view(*x.shape[:-1], self.out_features_per_rank)
        policy = getattr(self, 'operator_policy', None)
        backend = 'preallocated' if policy is None else policy.column_linear_backend
        out = column_linear(x.reshape(-1, self.in_features), self.weight, self.weight_scale,
                            convrot=self.convrot, convrot_groupsize=self.convrot_groupsize,
                            out_dtype=x.dtype, backend=backend)
        return out.view(*x.shape[:-1], self.out_features_per_rank)


class RowParallelLinearINT8(nn.Module):
    """Input-feature split INT8 projection (patches/tp_dit.py:98-162)."""

    def __init__(self, in_features, out_features, rank=0, world_size=1, convrot=True, convrot_groupsize=256,
                 device=None):
        super().__init__()
        if in_features % world_size:
            raise ValueError('in_features must divide across ranks')
        self.in_features_per_rank = in_features // world_size
        self.out_features = out_features
        self.rank = rank
        self.world_size = world_size
        self.convrot = convrot
        self.convrot_groupsize = convrot_groupsize
        self.device = torch.device(device) if device is not None else torch.device('cuda', 0)
        self.weight = nn.Parameter(torch.empty(out_features, self.in_features_per_rank, dtype=torch.int8,
                                               device=self.device), requires_grad=False)
        self.weight_scale = nn.Parameter(torch.empty(out_features, 1, dtype=torch.float32, device=self.device),
                                         requires_grad=False)

    def load_shard_from_full(self, full_weight, full_scale):
        start = self.rank * self.in_features_per_rank
        self.weight.data.copy_(full_weight[:, start:start + self.in_features_per_rank])
        self.weight_scale.data.copy_(full_scale)

    def forward(self, x, reduce_sum=True, input_act=None, *, residual=None, gate=None, segments=None,
                out_dtype=None, row_max=None, out=None):
        """Row projection. With ``residual`` (FP16) the result is the updated
        residual fp16(residual + fp16(branch)), or with the DiT modulation
        ``gate`` table and ``segments`` the gated update (tp_dit.py:141-162);
        otherwise the branch in ``out_dtype`` (default x's dtype).

        A rank's shard (world_size > 1) has no partner on one GPU: it returns
        its FP32 partial (f32(C_rank) * a) * w before the SUM exchange (see
        ``partial``), quantized with ``row_max`` (the MAX exchange's global
        row maximum) or, when None, with its own row maximum. The residual and
        gate apply after the SUM, so a shard takes neither.
        """
        if not reduce_sum and self.world_size > 1:
            raise ValueError('Quantization-preserving projection requires reduction')
        if self.world_size > 1:
            if residual is not None or gate is not None:
                raise ValueError('the residual update follows the SUM exchange: a rank shard returns its partial')
            return self.partial(x, input_act, row_max=row_max, out=out)
        if row_max is not None:
            raise ValueError('row_max is the MAX exchange of a rank shard (world_size > 1)')
        if out is not None:
            if input_act != 'swiglu' or residual is None:
                raise ValueError('out= is supported on the fused FC2 route with a residual')
            from . import swiglu_quant
            return swiglu_quant.row_linear(x, self.weight, self.weight_scale, None, residual=residual, gate=gate,
                                           gate_labels=_labels(x, gate, segments), out=out)
        out = dispatch_row(self, x, parallel_int8.row_linear, None, input_act, residual=residual, gate=gate,
                           segments=segments)
        if residual is not None:
            return out
        return out.to(out_dtype or x.dtype)

    def _local_rows(self, x, input_act):
        width = self.in_features_per_rank * (2 if input_act == 'swiglu' else 1)
        if input_act not in (None, 'swiglu'):
            raise ValueError(f'unsupported input_act {input_act!r}')
        if x.shape[-1] != width:
            raise ValueError(f'a rank shard takes [.., {width}] inputs (its K slice'
                             + (', gate then up)' if input_act == 'swiglu' else ')'))
        if self.convrot_groupsize != 256 or not self.convrot:
            raise ValueError('the row shard path quantizes with ConvRot256')
        return x.reshape(-1, width)

    def local_maximum(self, x, input_act=None):
        """This rank's fp32 [M, 1] row maxima, the MAX exchange's input.

        'swiglu': the absmax of ConvRot256(SwiGLU(gate, up)) over the rank's
        gate/up halves (patches/tilelang_swiglu_quant.py:76-86); None: the
        absmax of the FP32 ConvRot256 of the rank's K slice
        (patches/tilelang_row_quant.py:136-146, optimized_tp.py:71-79).
        Whole 256-channel groups stay on one rank, so the maximum of the
        ranks' values is the unsharded row maximum.
        """
        flat = self._local_rows(x, input_act)
        if input_act == 'swiglu':
            if flat.dtype not in (torch.float16, torch.float32):
                flat = flat.float()
            return kernels.swiglu_quantize(flat, quantize=False, want_row_max=True)['row_max']
        return kernels.row_absmax(flat, convrot=True, round_rotated=False)

    def partial(self, x, input_act=None, *, row_max=None, accumulate=torch.float32, out=None):
        """The rank's contribution before the SUM exchange.

        Quantizes the rank's slice with the global ``row_max`` (own maximum
        when None), then the INT8 GEMM against the rank's weight columns.
        accumulate=torch.int32 returns (C_rank int32 [M, N], row_scale fp32
        [M, 1]): the ranks' accumulators add exactly to the unsharded one
        (patches/parallel_int8.py:86-91, tilelang_swiglu_quant.py:123-127
        then dequantize). accumulate=torch.float32 returns the FP32 partial
        (f32(C_rank) * a) * w, the row-order dequantization of this rank's
        accumulator alone; ``out`` may receive it (e.g. a row range of a
        larger FP32 buffer).
        """
        flat = self._local_rows(x, input_act)
        if input_act == 'swiglu':
            if flat.dtype not in (torch.float16, torch.float32):
                flat = flat.float()
            res = kernels.swiglu_quantize(flat, row_max=row_max)
            q, scale = res['q'], res['scale']
        else:
            q, scale = kernels.quantize_rows(flat, convrot=True, round_rotated=False, row_max=row_max)
        n = self.weight.shape[0]
        if accumulate == torch.int32:
            if out is not None:
                raise ValueError('out= receives the FP32 partial')
            acc = kernels.gemm(q, self.weight, epilogue=kernels.EPI_INT32)
            return acc.reshape(*x.shape[:-1], n), scale
        if accumulate != torch.float32:
            raise ValueError('accumulate must be torch.int32 or torch.float32')
        if out is not None:
            out = out.reshape(-1, n)
        y = kernels.gemm(q, self.weight, epilogue=kernels.EPI_ROW, row_scale=scale, col_scale=self.weight_scale,
                         out_dtype=torch.float32, out=out)
        return y.reshape(*x.shape[:-1], n)


def _labels(x, gate, segments):
    if gate is None:
        return None
    from .h3_tensor_flow import labels_for
    labels = labels_for(x.reshape(-1, x.shape[-1]).shape[0], segments, gate.shape[0], device=x.device)
    if labels is None:
        raise ValueError('segments must tile the rows with valid modulation-table rows')
    return labels


class DiTFeedForwardINT8(nn.Module):
    """FC1 (column, gate|up) -> fused SwiGLU/ConvRot256 prologue -> FC2 (row) + residual.

    hidden -> 2*ffn -> hidden on one GPU; fc2.weight_scale carries the
    residual divisor once prepared (h3_tensor_flow.prepare_tp).
    """

    def __init__(self, hidden, ffn, device=None, policy=None):
        super().__init__()
        self.fc1 = ColumnParallelLinearINT8(hidden, 2 * ffn, device=device, components=2)
        self.fc2 = RowParallelLinearINT8(ffn, hidden, device=device)
        policy = policy or H3OperatorPolicy()
        self.operator_policy = policy
        self.fc1.operator_policy = policy
        self.fc2.operator_policy = policy

    @classmethod
    def from_projections(cls, fc1, fc2, policy=None):
        """An FFN over existing FC1 / FC2 projection modules (e.g. a loaded
        checkpoint block's ``fc1`` and ``fc2``)."""
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.fc1, self.fc2 = fc1, fc2
        policy = policy or H3OperatorPolicy()
        self.operator_policy = policy
        self.fc1.operator_policy = policy
        self.fc2.operator_policy = policy
        return self

    def forward(self, h, residual, gate=None, segments=None):
        """residual <- residual + branch, or with the modulation ``gate`` table
        and ``segments`` the DiT gated update (tp_dit.py:356-362)."""
        y = self.fc1(h)
        return self.fc2(y, input_act='swiglu', residual=residual, gate=gate, segments=segments)

    def forward_modulated(self, x, norm, shift, scale, gate, segments):
        """The DiT FFN sublayer from the residual stream (patches/tp_dit.py:347-362):
        x + gate * FFN(modulated_norm(norm, x, shift, scale)), with the norm
        fused into FC1's activation quantization (the normalized rows never
        reach HBM) and the gated residual update in FC2's epilogue.
        """
        codes, row_scale = modulated_norm_quantize(norm, x, shift, scale, segments, convrot=self.fc1.convrot,
                                                   convrot_groupsize=self.fc1.convrot_groupsize)
        y = self.fc1(x, prepared=(codes, row_scale))
        return self.fc2(y, input_act='swiglu', residual=x, gate=gate, segments=segments)

    def forward_partial(self, h, *, row_max=None, out=None):
        """One rank's FFN shard (fc1 / fc2 loaded with world_size 2): its FC1
        gate/up columns, then its FC2 FP32 partial before the SUM exchange,
        quantized with ``row_max`` (the global FC2 row maximum) or its own.
        ``out`` (FP32 [M, hidden]) may receive the partial in place."""
        if self.fc2.world_size < 2:
            raise ValueError('forward_partial runs a rank shard (world_size > 1)')
        y = self.fc1(h)
        return self.fc2.partial(y, 'swiglu', row_max=row_max, out=out)


class DiTAttentionINT8(nn.Module):
    """The DiT attention sublayer on one GPU (patches/tp_dit.py:277-345).

    x <- x + gate_msa * out_proj(attention(rms_rope(qkv_proj(
    modulated_norm(norm1, x, shift_msa, scale_msa))))) in four library steps:
    the modulated RMSNorm fused into the QKV activation quantization, the QKV
    GEMM with the per-head RMSNorm + RoPE of Q and K in its epilogue, the
    INT8 attention reading Q, K and V in place from the packed projection and
    writing [tokens, heads, 128] rows, and the O projection with the gated
    residual update in its epilogue. Attribute names follow the reference
    block: qkv_proj (3 packed components), out_proj, q_norm / k_norm
    (RMSNorm over head_dim), heads_per_rank, head_dim, inner_per_rank.
    """

    def __init__(self, hidden, heads, head_dim=128, *, eps=1e-6, device=None, policy=None):
        super().__init__()
        if head_dim != 128:
            raise ValueError('the INT8 attention and the RoPE epilogue take 128-wide heads')
        self.heads_per_rank = heads
        self.head_dim = head_dim
        self.inner_per_rank = heads * head_dim
        self.qkv_proj = ColumnParallelLinearINT8(hidden, 3 * self.inner_per_rank, device=device, components=3)
        self.out_proj = RowParallelLinearINT8(self.inner_per_rank, hidden, device=device)
        dev = self.qkv_proj.device
        self.q_norm = nn.RMSNorm(head_dim, eps=eps, device=dev)
        self.k_norm = nn.RMSNorm(head_dim, eps=eps, device=dev)
        self.requires_grad_(False)
        policy = policy or H3OperatorPolicy()
        self.operator_policy = policy
        self.qkv_proj.operator_policy = policy
        self.out_proj.operator_policy = policy

    def qkv(self, x, rope_freqs, *, prepared=None, freqs_pairs=None):
        """(q, k, v) as [tokens, heads, 128] views of the packed projection,
        q and k normalized and rotated (patches/tp_dit.py:286-309)."""
        if rope_freqs is None:
            raise ValueError('the fused QKV route applies RMS-RoPE: rope_freqs required')
        return fused_qkv(x, self.qkv_proj.weight, self.qkv_proj.weight_scale, rope_freqs, self.q_norm.weight,
                         self.k_norm.weight, heads=self.heads_per_rank, dim=self.head_dim, epsilon=self.q_norm.eps,
                         prepared=prepared, convrot=self.qkv_proj.convrot, freqs_pairs=freqs_pairs)

    def attention(self, q, k, v):
        """Attention of [tokens, heads, 128] q, k, v (strided views allowed)
        -> [tokens, heads * 128] FP16, the layout out_proj reads
        (patches/h3_operator_policy.py:153-216 with the transpose folded
        into the kernels' strides)."""
        rows = q.shape[0]
        prep = kernels.attention_prepare(q.transpose(0, 1)[None], k.transpose(0, 1)[None],
                                         v.transpose(0, 1)[None])
        out = torch.empty((rows, self.heads_per_rank, self.head_dim), dtype=torch.float16, device=q.device)
        kernels.attention(prep, out_dtype=torch.float16, out=out.transpose(0, 1)[None])
        return out.view(rows, self.inner_per_rank)

    def forward_modulated(self, x, norm, shift, scale, gate, segments, rope_freqs, *, freqs_pairs=None):
        """x [tokens, hidden] FP16 residual stream; norm the block's norm1;
        shift / scale / gate the [R, hidden] modulation tables with
        segments [(a, b, row)] tiling the rows; rope_freqs (1, tokens, 1,
        half, 2, 2), freqs_pairs optionally rms_rope.pack_freqs(rope_freqs).
        Returns the updated residual stream."""
        codes, row_scale = modulated_norm_quantize(norm, x, shift, scale, segments, convrot=self.qkv_proj.convrot,
                                                   convrot_groupsize=self.qkv_proj.convrot_groupsize)
        q, k, v = self.qkv(x, rope_freqs, prepared=(codes, row_scale), freqs_pairs=freqs_pairs)
        del codes, row_scale
        attn = self.attention(q, k, v)
        del q, k, v
        return self.out_proj(attn, residual=x, gate=gate, segments=segments)


class TPDiTBlockINT8(nn.Module):
    """The DiT block on one GPU in the scaled FP16 tensor flow
    (patches/tp_dit.py:164-362, the ``flow is not None`` branches).

    Attribute names follow the reference block: norm1, norm2 (RMSNorm over
    hidden), adaln_proj (t_dim -> 18 * hidden, replicated, FP32), qkv_proj,
    out_proj, q_norm, k_norm, fc1, fc2. The projections live in the
    attention and FFN sublayers (``attn``, ``mlp``); the reference names
    resolve to them. Run prepare_tp(block, 'dit', TensorFlowPolicy('fp16'))
    first: it folds the residual divisor into out_proj / fc2, installs
    StableNorm and divides norm1 / norm2 eps by the divisor squared.
    forward needs rope_freqs: the fused QKV route applies RMS-RoPE.
    """

    def __init__(self, hidden=5376, heads=56, head_dim=128, ffn=14336, t_dim=8, *, eps=1e-5, qk_eps=1e-5,
                 device=None, dtype=torch.float32, apply_silu=False, policy=None):
        super().__init__()
        self.hidden = hidden
        self.heads = heads
        self.head_dim = head_dim
        self.apply_silu = apply_silu
        self.rank, self.world_size = 0, 1
        self.attn = DiTAttentionINT8(hidden, heads, head_dim, eps=qk_eps, device=device, policy=policy)
        dev = self.attn.qkv_proj.device
        self.mlp = DiTFeedForwardINT8(hidden, ffn, device=dev, policy=self.attn.operator_policy)
        self.operator_policy = self.attn.operator_policy
        self.norm1 = nn.RMSNorm(hidden, eps=eps, device=dev, dtype=dtype)
        self.norm2 = nn.RMSNorm(hidden, eps=eps, device=dev, dtype=dtype)
        self.adaln_proj = nn.Linear(t_dim, 6 * 3 * hidden, bias=True, device=dev, dtype=dtype)
        self.requires_grad_(False)

    qkv_proj = property(lambda self: self.attn.qkv_proj)
    out_proj = property(lambda self: self.attn.out_proj)
    q_norm = property(lambda self: self.attn.q_norm)
    k_norm = property(lambda self: self.attn.k_norm)
    fc1 = property(lambda self: self.mlp.fc1)
    fc2 = property(lambda self: self.mlp.fc2)

    @property
    def heads_per_rank(self):
        return self.attn.heads_per_rank

    def modulation(self, t_emb):
        """(shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp),
        each [R, hidden] (patches/tp_dit.py:273-275)."""
        adaln_out = self.adaln_proj(nn.functional.silu(t_emb) if self.apply_silu else t_emb)
        return adaln_out.view(-1, 6 * self.hidden).chunk(6, dim=-1)

    def forward(self, x, t_emb, mod_segments, rope_freqs=None, transformer_options=None, *, freqs_pairs=None):
        flow = getattr(self, 'tensor_flow', None)
        if flow is None:
            raise ValueError('the INT8 DiT block runs the scaled tensor flow: prepare_tp(block, "dit", policy) first')
        if x.dtype != flow.dtype:
            raise ValueError('DiT residual dtype does not match tensor flow')
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = self.modulation(t_emb)
        x = self.attn.forward_modulated(x, self.norm1, shift_msa, scale_msa, gate_msa, mod_segments, rope_freqs,
                                        freqs_pairs=freqs_pairs)
        return self.mlp.forward_modulated(x, self.norm2, shift_mlp, scale_mlp, gate_mlp, mod_segments)


def chunked_rows(fn, x, *others, chunk_rows=16384, out=None):
    """Apply fn(x_chunk, *other_chunks) over row chunks of 2-D x.

    Exact for W8A8 projections because every scale is per row. ``out`` (if
    given) receives the rows in place; otherwise the chunks are concatenated.
    """
    rows = x.shape[0]
    parts = []
    for start in range(0, rows, chunk_rows):
        stop = min(start + chunk_rows, rows)
        y = fn(x[start:stop], *[o[start:stop] for o in others])
        if out is not None:
            out[start:stop].copy_(y)
        else:
            parts.append(y)
    return out if out is not None else torch.cat(parts, 0)
