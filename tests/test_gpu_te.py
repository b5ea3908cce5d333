"""GPU parity of the text-encoder projections and the tensor-flow preparation.

* The six skinny TE projections (M in {1, 64, 512}; up 4096 -> 14336, down
  14336 -> 4096) end to end through the TE modules: ConvRot256 quantization,
  the GEMM and its epilogue, against the oracle bit for bit.
* The TE MLP (post-attention RMSNorm -> shared gate/up quantization -> two
  column GEMMs into one buffer -> fused FP32 SwiGLU/ConvRot256 down
  projection with the residual add) against the oracle's composition.
* row_linear_parts on both of its branches.
* prepare_tp: the eps / divisor**2 fold leaves the normalized rows of the
  scaled stream bit-identical, and the DiT block runs its two sublayers.
"""
import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of, randn16
from w8a8 import kernels, parallel_int8, workloads
from w8a8.h3_operator_policy import H3OperatorPolicy, adjacent_cat, row_linear_parts
from w8a8.h3_tensor_flow import StableNorm, TensorFlowPolicy, modulated_norm, prepare_tp
from w8a8.tp_qwen3vl import (ColumnParallelLinearINT8, RowParallelLinearINT8, TEFeedForwardINT8,
                             project_columns)

pytestmark = pytest.mark.gpu

TE_MS = (1, 64, 512)


def _load(module, w, gpu):
    q, s = workloads.quantize_weight(w, gpu)
    module.weight.data.copy_(q)
    module.weight_scale.data.copy_(s)
    return module


@pytest.mark.parametrize('m', TE_MS)
def test_te_up_and_down_projections_end_to_end(gpu, m):
    data = workloads.te_skinny(m)
    print(f'TE skinny M={m}: up 4096->14336, down 14336->4096', flush=True)
    up = _load(ColumnParallelLinearINT8(4096, 14336, device=gpu), data['w_up'], gpu)
    y = up(data['x'].to(gpu))
    assert y.shape == (m, 14336) and y.dtype == torch.float16
    want = o.column_linear(np_of(data['x']), np_of(up.weight), np_of(up.weight_scale).reshape(-1))
    assert_bits_equal(np_of(y), want, f'TE up M={m}')
    down = _load(RowParallelLinearINT8(14336, 4096, device=gpu), data['w_down'], gpu)
    z = down(data['x_down'].to(gpu))
    assert z.shape == (m, 4096) and z.dtype == torch.float16
    want = o.row_linear(np_of(data['x_down']), np_of(down.weight), np_of(down.weight_scale).reshape(-1),
                        out_dtype='f16')
    assert_bits_equal(np_of(z), want, f'TE down M={m}')
    down.operator_policy = H3OperatorPolicy()    # scaled-FP16 policy: FP32 island, same bits
    assert torch.equal(down(data['x_down'].to(gpu)), z)


def _te_ffn(gpu, hidden, inter, seed):
    g = torch.Generator().manual_seed(seed)
    ffn = TEFeedForwardINT8(hidden, inter, device=gpu)
    _load(ffn.gate_proj, torch.randn((inter, hidden), generator=g) * 0.02, gpu)
    _load(ffn.up_proj, torch.randn((inter, hidden), generator=g) * 0.02, gpu)
    _load(ffn.down_proj, torch.randn((hidden, inter), generator=g) * 0.02, gpu)
    ffn.post_attention_layernorm.weight.data.copy_((torch.rand(hidden, generator=g) + 0.5).half())
    prepare_tp(ffn, 'te', TensorFlowPolicy(mode='fp16'))
    return ffn, g


def _te_ffn_oracle(ffn, x):
    norm = ffn.post_attention_layernorm
    q, a, _ = o.norm_quantize(np_of(x), np_of(norm.weight.float()), eps=norm.eps)
    gate = o.dequantize_column(o.int_mm(q, np_of(ffn.gate_proj.weight)), a,
                               np_of(ffn.gate_proj.weight_scale).reshape(-1), 'f16')
    up = o.dequantize_column(o.int_mm(q, np_of(ffn.up_proj.weight)), a,
                             np_of(ffn.up_proj.weight_scale).reshape(-1), 'f16')
    return o.row_linear_fc2(np.concatenate([gate, up], 1), np_of(ffn.down_proj.weight),
                            np_of(ffn.down_proj.weight_scale).reshape(-1), residual=np_of(x)), gate, up


@pytest.mark.parametrize('m', TE_MS)
def test_te_mlp_against_oracle(gpu, m):
    print(f'TE MLP M={m}: 4096 -> 2 x 14336 -> 4096 with the residual add', flush=True)
    ffn, g = _te_ffn(gpu, 4096, 14336, 40 + m)
    assert isinstance(ffn.post_attention_layernorm, StableNorm)
    assert ffn.post_attention_layernorm.eps == pytest.approx(1e-6 / 512 ** 2, rel=0, abs=0)
    x = randn16(g, (m, 4096), 0.5)
    out = ffn(x.to(gpu))
    want, gate, up = _te_ffn_oracle(ffn, x)
    assert_bits_equal(np_of(out), want, f'TE MLP M={m}')
    # the pieces: shared quantization, packed gate|up, fused residual == add after
    xn = ffn.post_attention_layernorm(x.to(gpu))
    gd, ud = project_columns(xn, ffn.gate_proj, ffn.up_proj)
    assert_bits_equal(np_of(gd), gate, 'gate')
    assert_bits_equal(np_of(ud), up, 'up')
    assert adjacent_cat(gd, ud).data_ptr() == gd.data_ptr()          # no copy: up follows gate
    assert torch.equal(gd, ffn.gate_proj(xn)) and torch.equal(ud, ffn.up_proj(xn))
    branch = ffn.down_proj.forward_parts(gd, ud)
    from w8a8.h3_tensor_flow import residual_add
    assert torch.equal(ffn.down_proj.forward_parts(gd, ud, residual=x.to(gpu)), residual_add(x.to(gpu), branch))
    assert torch.equal(ffn.down_proj.forward_parts(gd.clone(), ud.clone(), residual=x.to(gpu)), out)


def test_row_linear_parts_both_branches(gpu):
    g = torch.Generator().manual_seed(50)
    down = _load(RowParallelLinearINT8(1024, 384, device=gpu), torch.randn((384, 1024), generator=g) * 0.02, gpu)
    gate = randn16(g, (70, 1024), 2.0)
    up = randn16(g, (70, 1024), 1.0)
    wq, ws = np_of(down.weight), np_of(down.weight_scale).reshape(-1)
    # fused route: FP32 SwiGLU of the FP16 halves, the row FP32 result
    down.operator_policy = H3OperatorPolicy()
    got = row_linear_parts(down, gate.to(gpu), up.to(gpu), parallel_int8.row_linear, None)
    assert got.dtype == torch.float32
    assert_bits_equal(np_of(got), o.row_linear_fc2(np.concatenate([np_of(gate), np_of(up)], 1), wq, ws,
                                                   out_dtype='f32'), 'fused parts')
    with pytest.raises(ValueError, match='Matching gate/up'):
        row_linear_parts(down, gate.to(gpu), up[:, :512].to(gpu), parallel_int8.row_linear, None)
    # native FC2 quantizer: silu(gate) * up in FP16 (torch's elementwise ops),
    # then the row projection with no input activation (FP32 island)
    down.operator_policy = H3OperatorPolicy(fc2_quantizer='native')
    act = torch.nn.functional.silu(gate.to(gpu)) * up.to(gpu)
    assert act.dtype == torch.float16
    got = row_linear_parts(down, gate.to(gpu), up.to(gpu), parallel_int8.row_linear, None)
    assert got.dtype == torch.float32
    assert_bits_equal(np_of(got), o.row_linear(np_of(act), wq, ws, out_dtype='f32'), 'native parts')
    # the torch FP16 product is within its storage rounding of the oracle's FP32 SwiGLU
    ref = o.swiglu_f32(np_of(gate).astype(np.float32), np_of(up).astype(np.float32))
    err = np.abs(np_of(act).astype(np.float32) - ref)
    assert (err <= np.abs(ref) * 2.0 ** -9 + 2.0 ** -20).all()
    # no policy: the halves' product in their dtype, FP16 out
    del down.operator_policy
    got = down.forward_parts(gate.to(gpu), up.to(gpu))
    assert got.dtype == torch.float16
    assert_bits_equal(np_of(got), o.row_linear(np_of(act), wq, ws, out_dtype='f16'), 'no-policy parts')


def test_eps_fold_is_exact_on_the_scaled_stream(gpu):
    """modulated_norm of x / 512 with eps / 512**2 == of x with eps, bit for bit."""
    g = torch.Generator().manual_seed(51)
    xs = (torch.randn((33, 1024), generator=g) / 512).half()
    x = (xs.float() * 512).half()
    assert torch.equal((x.float() / 512).half(), xs)           # both exact
    norm = torch.nn.RMSNorm(1024, eps=1e-5, device=gpu)
    norm.weight.data.copy_(torch.rand(1024, generator=g) + 0.5)

    class Block(torch.nn.Module):
        pass
    b = Block()
    b.norm1 = norm
    plain = modulated_norm(norm, x.to(gpu), None, None, None)
    prepare_tp(b, 'dit', TensorFlowPolicy(mode='fp16'))
    assert isinstance(b.norm1, StableNorm) and b.norm1.eps == 1e-5 / 512 ** 2
    scaled = modulated_norm(b.norm1, xs.to(gpu), None, None, None)
    assert torch.equal(scaled, plain)
    assert torch.equal(b.norm1(xs.to(gpu)), scaled)        # StableNorm's own forward: the same kernel
    want = o.modulated_rms_norm(np_of(xs), np_of(norm.weight), eps=1e-5 / 512 ** 2)
    assert_bits_equal(np_of(scaled), want, 'folded eps norm')


def _ordered(t):
    """16-bit floats as integers in value order (sign-magnitude to two's complement)."""
    bits = t.view(torch.int16).to(torch.int32)
    return torch.where(bits < 0, -(bits & 0x7FFF), bits)


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
def test_stable_norm_agrees_with_torch_rms_norm(gpu, dtype):
    """StableNorm's kernel (fixed-order fp32 sum, IEEE sqrt and division)
    against the reference's own expression, F.rms_norm(x.float(), ..., eps)
    cast back (patches/h3_tensor_flow.py:48-69), on the same device: at most
    one unit in the last place apart, and nearly all outputs bit-identical."""
    g = torch.Generator().manual_seed(53)
    norm = torch.nn.RMSNorm(3072, eps=1e-6, device=gpu)
    norm.weight.data.copy_(torch.rand(3072, generator=g) + 0.5)
    sn = StableNorm(norm, divisor=512.0)
    x = ((torch.randn((4096, 3072), generator=g) * torch.rand((4096, 1), generator=g) * 4) / 512).to(dtype).to(gpu)
    got = sn(x)
    want = torch.nn.functional.rms_norm(x.float(), (3072,), norm.weight.detach().float(), sn.eps).to(dtype)
    d = (_ordered(got) - _ordered(want)).abs()
    same = (d == 0).float().mean().item()
    print(f'{dtype}: max {d.max().item()} ulp apart, {same:.5f} bit-identical')
    assert d.max().item() <= 1
    assert same >= 0.99


def test_dit_block_runs_its_sublayers(gpu):
    from w8a8.tp_dit import TPDiTBlockINT8
    g = torch.Generator().manual_seed(52)
    block = TPDiTBlockINT8(hidden=512, heads=4, ffn=1024, t_dim=8, device=gpu)
    for m in (block.qkv_proj, block.out_proj, block.fc1, block.fc2):
        _load(m, torch.randn(m.weight.shape, generator=g) * 0.02, gpu)
    for n in (block.norm1, block.norm2, block.q_norm, block.k_norm):
        n.weight.data.copy_(torch.rand(n.weight.shape, generator=g) + 0.5)
    block.adaln_proj.weight.data.copy_(torch.randn(block.adaln_proj.weight.shape, generator=g) * 0.05)
    block.adaln_proj.bias.data.copy_(torch.randn(block.adaln_proj.bias.shape, generator=g) * 0.05)
    ws_out = block.out_proj.weight_scale.detach().clone()
    with pytest.raises(ValueError, match='prepare_tp'):
        block(torch.zeros(4, 512, dtype=torch.float16, device=gpu), None, [])
    prepare_tp(block, 'dit', TensorFlowPolicy(mode='fp16'))
    assert torch.equal(block.out_proj.weight_scale * 512, ws_out)
    assert isinstance(block.norm1, StableNorm) and isinstance(block.q_norm, StableNorm)
    assert block.norm2.eps == 1e-5 / 512 ** 2 and block.q_norm.eps == 1e-5
    with pytest.raises(ValueError, match='already prepared'):
        prepare_tp(block, 'dit', TensorFlowPolicy(mode='fp16'))
    s = 96
    x = (randn16(g, (s, 512), 1.0).float() / 512).half().to(gpu)
    t_emb = torch.randn((1, 8), generator=g).to(gpu)
    segments = [(0, 40, 0), (40, s, 1)]
    ang = torch.randn((s, 32), generator=g)
    freqs = torch.stack([torch.cos(ang), -torch.sin(ang), torch.sin(ang), torch.cos(ang)], -1)
    freqs = freqs.reshape(1, s, 1, 32, 2, 2).to(gpu)
    out = block(x.clone(), t_emb, segments, freqs)
    mods = block.modulation(t_emb)
    assert mods[0].shape == (3, 512)
    ref = block.attn.forward_modulated(x.clone(), block.norm1, mods[0], mods[1], mods[2], segments, freqs)
    ref = block.mlp.forward_modulated(ref, block.norm2, mods[3], mods[4], mods[5], segments)
    assert torch.equal(out, ref) and torch.isfinite(out).all()
