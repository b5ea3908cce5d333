"""GPU DiT attention sublayer (modulated norm -> QKV + RMS-RoPE -> INT8
attention -> O projection with the gated residual): every stage against the
oracle, bit for bit where the stage is exact, and the whole sublayer against
the oracle's composition."""
import numpy as np
import pytest
import torch

import oracle as o
from oracle import int8_attention as oa
from helpers import assert_bits_equal, np_of
from w8a8 import kernels, rms_rope, tp_dit

pytestmark = pytest.mark.gpu


def _freqs(g, rows, rot):
    ang = torch.rand((rows, rot // 2), generator=g, dtype=torch.float64) * 6.283185307179586
    c, s = torch.cos(ang), torch.sin(ang)
    f = torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2)
    return f.to(torch.float32).reshape(1, rows, 1, rot // 2, 2, 2)


@pytest.mark.parametrize('rows,hidden,heads,rot', [(300, 256, 2, 64), (129, 512, 4, 128)])
def test_dit_attention_sublayer(gpu, rows, hidden, heads, rot):
    g = torch.Generator().manual_seed(rows + heads)
    inner = heads * 128
    block = tp_dit.DiTAttentionINT8(hidden, heads, device=gpu)
    wqkv, sqkv = o.quantize_rows(o.convrot256((torch.randn((3 * inner, hidden), generator=g) * 0.05).numpy()))
    wo, so = o.quantize_rows(o.convrot256((torch.randn((hidden, inner), generator=g) * 0.05).numpy()))
    with torch.no_grad():
        block.qkv_proj.weight.copy_(torch.from_numpy(wqkv))
        block.qkv_proj.weight_scale.copy_(torch.from_numpy(sqkv).reshape(-1, 1))
        block.out_proj.weight.copy_(torch.from_numpy(wo))
        block.out_proj.weight_scale.copy_(torch.from_numpy(so).reshape(-1, 1))
        block.q_norm.weight.copy_(torch.rand(128, generator=g) + 0.5)
        block.k_norm.weight.copy_(torch.rand(128, generator=g) + 0.5)
    x = (torch.randn((rows, hidden), generator=g) * 2).half()
    norm = torch.nn.RMSNorm(hidden, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(hidden, generator=g) + 0.5)
    shift = torch.randn((9, hidden), generator=g) * 0.1
    scale = torch.randn((9, hidden), generator=g) * 0.1
    gate = torch.randn((9, hidden), generator=g)
    segments = [(0, rows // 3, 1), (rows // 3, rows, 6)]
    labels = np.zeros(rows, np.int64)
    for a, b, row in segments:
        labels[a:b] = row
    freqs = _freqs(g, rows, rot)
    xg = x.to(gpu)
    fg = freqs.to(gpu)
    out = block.forward_modulated(xg, norm, shift.to(gpu), scale.to(gpu), gate.to(gpu), segments, fg,
                                  freqs_pairs=rms_rope.pack_freqs(fg))
    # stage 1+2: the normalized rows, the packed projection and its RMS-RoPE
    h = o.modulated_rms_norm(np_of(x), np_of(norm.weight.detach()), np_of(shift), np_of(scale), labels,
                             eps=norm.eps)
    packed = o.column_linear(h, wqkv, sqkv)
    qo, ko = o.rms_rope(packed, np_of(freqs).reshape(rows, rot // 2, 2, 2), np_of(block.q_norm.weight.cpu()),
                        np_of(block.k_norm.weight.cpu()), heads, rot, eps=block.q_norm.eps)
    vo = packed[:, 2 * inner:].reshape(rows, heads, 128)
    codes, row_scale = tp_dit.modulated_norm_quantize(norm, xg, shift.to(gpu), scale.to(gpu), segments)
    q, k, v = block.qkv(xg, fg, prepared=(codes, row_scale))
    assert_bits_equal(np_of(q), qo, 'q')
    assert_bits_equal(np_of(k), ko, 'k')
    assert_bits_equal(np_of(v), vo, 'v')
    # stage 3: the attention operands from the packed rows, bit for bit; the
    # output within the hardware exp2 tolerance of the oracle
    heads_first = [np.ascontiguousarray(t.astype(np.float32).transpose(1, 0, 2))[None] for t in (qo, ko, vo)]
    oprep = oa.kitchen_prepare(*heads_first, cta_k=oa.GPU_CTA_K)
    ops = oa.gpu_operands(oprep)
    prep = kernels.attention_prepare(q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None])
    for name in oa.GPU_OPERANDS:
        got = np_of(prep[name])
        if got.dtype == np.float32:
            assert np.array_equal(got.view(np.uint32), ops[name].view(np.uint32)), name
        else:
            assert np.array_equal(got, ops[name]), name
    attn = block.attention(q, k, v)
    want_attn = oa.kitchen_attention(oprep)[0].transpose(1, 0, 2).reshape(rows, inner)
    err = np.abs(np_of(attn).astype(np.float64) - want_attn).max()
    print(f'attention rows: max |gpu - oracle| / max |oracle| = {err / np.abs(want_attn).max():.2e}')
    assert err <= 2 ** -10 * np.abs(want_attn).max(), err   # fp16 rows: one rounding of the restatement
    # stage 4: the gated O projection of the GPU's attention rows, bit for bit,
    # and the sublayer output
    want = o.row_linear(np_of(attn), wo, so, residual=np_of(x), gate=np_of(gate), labels=labels)
    assert_bits_equal(np_of(out), want, 'sublayer output')
    # the fused O route equals the plain projection followed by the gated add
    branch = block.out_proj(attn)
    assert_bits_equal(np_of(branch), o.row_linear(np_of(attn), wo, so, out_dtype='f16'), 'O branch')
    assert_bits_equal(np_of(out), o.gated_residual_add(np_of(x), np_of(branch), np_of(gate), labels), 'gated')
    with pytest.raises(ValueError):
        block.forward_modulated(xg, norm, shift.to(gpu), scale.to(gpu), gate.to(gpu), segments, None)
