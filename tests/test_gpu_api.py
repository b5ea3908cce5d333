"""GPU parity of the reference-shaped API (column/row projections, FFN block).

Small shapes compare whole outputs with the oracle bit for bit; the full
benchmark shapes are checked through sampled rows (every W8A8 scale is per
row, so a row's output depends only on that row's inputs).
"""
import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of, randn16
from w8a8 import dit_column_linear, kernels, parallel_int8, swiglu_quant, row_quant, column_epilogue, workloads
from w8a8.h3_tensor_flow import TensorFlowPolicy, prepare_tp
from w8a8.tp_dit import DiTFeedForwardINT8, chunked_rows

pytestmark = pytest.mark.gpu


def _wq(w, gpu):
    q, s = workloads.quantize_weight(w, gpu)
    return q, s


def test_column_linear_and_shared(gpu):
    g = torch.Generator().manual_seed(1)
    x = randn16(g, (2, 37, 1024), 2.0)
    w1 = torch.randn((384, 1024), generator=g) * 0.02
    w2 = torch.randn((128, 1024), generator=g) * 0.02
    q1, s1 = _wq(w1, gpu)
    q2, s2 = _wq(w2, gpu)
    y = dit_column_linear.column_linear(x.to(gpu), q1, s1)
    assert y.shape == (2, 37, 384) and y.dtype == torch.float16
    want = o.column_linear(np_of(x).reshape(-1, 1024), np_of(q1), np_of(s1).reshape(-1), convrot=True)
    assert_bits_equal(np_of(y).reshape(-1, 384), want, 'column_linear')
    ys = dit_column_linear.shared_column_linears(x.to(gpu), [(q1, s1), (q2, s2)])
    assert_bits_equal(np_of(ys[0]), np_of(y), 'shared[0]')
    want2 = o.column_linear(np_of(x).reshape(-1, 1024), np_of(q2), np_of(s2).reshape(-1), convrot=True)
    assert_bits_equal(np_of(ys[1]).reshape(-1, 128), want2, 'shared[1]')
    assert dit_column_linear.shared_column_linears(x.to(gpu), [(q1[:, :512], s1)]) is None
    with pytest.raises(ValueError):
        dit_column_linear.column_linear(x.to(gpu), q1, s1, backend='other')
    with pytest.raises(ValueError):
        dit_column_linear.column_linear(x.to(gpu), q1[:, :512], s1)


def test_column_linear_with_bias_no_rotation(gpu):
    data = workloads.w8a8_linear(m=256)
    wq, ws = _wq(data['w'], gpu)
    y = dit_column_linear.column_linear(data['x'].to(gpu), wq, ws, convrot=False, bias=data['bias'].to(gpu))
    want = o.column_linear(np_of(data['x']), np_of(wq), np_of(ws).reshape(-1), convrot=False,
                           bias=np_of(data['bias']))
    assert_bits_equal(np_of(y), want, 'column + bias')


def test_parallel_int8_primitives(gpu):
    g = torch.Generator().manual_seed(2)
    x = randn16(g, (45, 768), 1.5)
    w = torch.randn((640, 768), generator=g) * 0.02
    wq, ws = _wq(w, gpu)
    q, s = parallel_int8.quantize(x.to(gpu))
    rq, rs = o.quantize_rows(o.convrot256(np_of(x).astype(np.float32)))
    assert_bits_equal(np_of(q), rq, 'parallel_int8.quantize codes')
    assert_bits_equal(np_of(s).reshape(-1), rs, 'parallel_int8.quantize scale')
    acc = parallel_int8.int_mm(q, wq)
    assert_bits_equal(np_of(acc), o.int_mm(rq, np_of(wq)), 'int_mm')
    b = (torch.randn((640,), generator=g) * 0.01).half()
    y = parallel_int8.dequantize(acc, s, ws, torch.float16, bias=b.to(gpu))
    assert_bits_equal(np_of(y), o.dequantize_row(np_of(acc), rs, np_of(ws), 'f16', np_of(b)), 'dequantize')
    out = parallel_int8.row_linear(x.to(gpu), wq, ws, None, 1, bias=b.to(gpu))
    assert_bits_equal(np_of(out), o.dequantize_row(o.int_mm(rq, np_of(wq)), rs, np_of(ws), 'f16', np_of(b)),
                      'row_linear')
    with pytest.raises(ValueError):
        parallel_int8.row_linear(x.to(gpu), wq, ws, None, 2)


def test_swiglu_row_linear_and_input_act_quantize(gpu):
    g = torch.Generator().manual_seed(3)
    m, w, n = 77, 1024, 512
    x = randn16(g, (m, 2 * w), 2.0)
    w2 = torch.randn((n, w), generator=g) * 0.02
    wq, ws = _wq(w2, gpu)
    q, s = parallel_int8.quantize(x.to(gpu), input_act='swiglu')
    rq, rs, _ = o.fc2_prologue(np_of(x))
    assert_bits_equal(np_of(q), rq, 'swiglu quantize codes')
    y32 = swiglu_quant.row_linear(x.to(gpu), wq, ws, None, mode='fused_stored')
    want32 = o.dequantize_row(o.int_mm(rq, np_of(wq)), rs, np_of(ws), 'f32')
    assert_bits_equal(np_of(y32), want32, 'fused_stored fp32')
    y32r = swiglu_quant.row_linear(x.to(gpu), wq, ws, None, mode='fused_recompute')
    assert_bits_equal(np_of(y32r), want32, 'fused_recompute fp32')
    res = randn16(g, (m, n), 1 / 512)
    y16 = swiglu_quant.row_linear(x.to(gpu), wq, ws, None, residual=res.to(gpu))
    assert_bits_equal(np_of(y16), o.row_linear_fc2(np_of(x), np_of(wq), np_of(ws), residual=np_of(res)),
                      'fused residual')


def test_row_quant_and_column_epilogue_api(gpu):
    g = torch.Generator().manual_seed(4)
    rot = torch.randn((9, 1024), generator=g) * 3
    mx = rot.abs().amax(-1, keepdim=True) * 1.5
    q, s = row_quant.quantize(rot.to(gpu), mx.to(gpu), width=512, start=256)
    rq, rs = o.quantize_rows(np_of(rot)[:, 256:768], row_max=np_of(mx))
    assert_bits_equal(np_of(q), rq, 'row_quant codes')
    assert_bits_equal(np_of(s).reshape(-1), rs, 'row_quant scale')
    assert_bits_equal(np_of(row_quant.maximum(rot.to(gpu), 512, 256)).reshape(-1),
                      np.abs(np_of(rot)[:, 256:768]).max(1), 'row_quant maximum')
    with pytest.raises(ValueError):
        row_quant.maximum(rot.to(gpu), 500, 256)      # the kernel reads 16-column units
    acc = torch.randint(-2 ** 24, 2 ** 24, (9, 64), generator=g, dtype=torch.int32)
    a = torch.rand((9, 1), generator=g)
    w = torch.rand((64,), generator=g) * 1e-3
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        y = column_epilogue.dequantize(acc.to(gpu), a.to(gpu), w.to(gpu), dt)
        want = o.dequantize_column(np_of(acc), np_of(a), np_of(w), {torch.float16: 'f16', torch.bfloat16: 'bf16',
                                                                      torch.float32: 'f32'}[dt])
        assert_bits_equal(np_of(y), want, f'column epilogue {dt}')
    with pytest.raises(ValueError):
        row_quant.quantize(rot.to(gpu), mx.to(gpu), division='slow')


def _ffn_module(data, gpu, hidden, ffn):
    block = DiTFeedForwardINT8(hidden, ffn, device=gpu)
    q1, s1 = _wq(data['w1'], gpu)
    q2, s2 = _wq(data['w2'], gpu)
    block.fc1.weight.data.copy_(q1)
    block.fc1.weight_scale.data.copy_(s1)
    block.fc2.weight.data.copy_(q2)
    block.fc2.weight_scale.data.copy_(s2)
    block.out_proj = None
    prepare_tp(block, 'dit', TensorFlowPolicy(mode='fp16'))
    return block


def test_dit_ffn_block_small_exact(gpu):
    data = workloads.dit_ffn(m=512, hidden=768, ffn=1024)
    block = _ffn_module(data, gpu, 768, 1024)
    assert torch.equal(block.fc2.weight_scale.cpu(), _wq(data['w2'], gpu)[1].cpu() / 512)
    out = block(data['h'].to(gpu), data['residual'].to(gpu))
    want = o.ffn_block(np_of(data['h']), np_of(block.fc1.weight), np_of(block.fc1.weight_scale).reshape(-1),
                       np_of(block.fc2.weight), np_of(block.fc2.weight_scale).reshape(-1), np_of(data['residual']))
    assert_bits_equal(np_of(out), want, 'ffn block')


def test_dit_ffn_block_gated(gpu):
    # The DiT block's FC2 with the gate_mlp modulation table and per-frame
    # segments (patches/tp_dit.py:356-362): the fused gated residual update.
    data = workloads.dit_ffn(m=512, hidden=768, ffn=1024)
    block = _ffn_module(data, gpu, 768, 1024)
    g = torch.Generator().manual_seed(4)
    gate = torch.randn((9, 768), generator=g)
    segments = [(0, 200, 3), (200, 450, 0), (450, 512, 8)]
    out = block(data['h'].to(gpu), data['residual'].to(gpu), gate=gate.to(gpu), segments=segments)
    labels = np.zeros(512, np.int64)
    for a, b, row in segments:
        labels[a:b] = row
    want = o.ffn_block(np_of(data['h']), np_of(block.fc1.weight), np_of(block.fc1.weight_scale).reshape(-1),
                       np_of(block.fc2.weight), np_of(block.fc2.weight_scale).reshape(-1), np_of(data['residual']),
                       gate=np_of(gate), labels=labels)
    assert_bits_equal(np_of(out), want, 'gated ffn block')
    with pytest.raises(ValueError):
        block.fc2(torch.zeros((4, 2048), dtype=torch.float16, device=gpu), input_act='swiglu',
                  gate=gate.to(gpu), segments=[(0, 4, 0)])


def test_dit_ffn_sublayer_with_fused_modulated_norm(gpu):
    # x <- x + gate * FFN(modulated_norm(norm2, x, shift, scale)) (patches/tp_dit.py:347-362) with the
    # norm fused into FC1's activation quantization.
    from w8a8 import h3_tensor_flow as flow
    data = workloads.dit_ffn(m=512, hidden=768, ffn=1024)
    block = _ffn_module(data, gpu, 768, 1024)
    g = torch.Generator().manual_seed(5)
    x = (torch.randn((512, 768), generator=g) * 3).half()
    norm = torch.nn.RMSNorm(768, eps=1e-6 / 512 ** 2)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(768, generator=g) + 0.5)
    shift = torch.randn((9, 768), generator=g) * 0.1
    scale = torch.randn((9, 768), generator=g) * 0.1
    gate = torch.randn((9, 768), generator=g)
    segments = [(0, 100, 2), (100, 512, 7)]
    labels = np.zeros(512, np.int64)
    for a, b, row in segments:
        labels[a:b] = row
    out = block.forward_modulated(x.to(gpu), norm, shift.to(gpu), scale.to(gpu), gate.to(gpu), segments)
    h = o.modulated_rms_norm(np_of(x), np_of(norm.weight.detach()), np_of(shift), np_of(scale), labels,
                             eps=norm.eps)
    want = o.ffn_block(h, np_of(block.fc1.weight), np_of(block.fc1.weight_scale).reshape(-1),
                       np_of(block.fc2.weight), np_of(block.fc2.weight_scale).reshape(-1), np_of(x),
                       gate=np_of(gate), labels=labels)
    assert_bits_equal(np_of(out), want, 'ffn sublayer with fused norm')
    # the standalone norm (both routes) returns the rows the fused kernel quantized
    y = flow.modulated_norm(norm, x.to(gpu), shift.to(gpu), scale.to(gpu), segments, fused=True)
    assert_bits_equal(np_of(y), h, 'modulated_norm')
    codes, row_scale = flow.modulated_norm_quantize(norm, x.to(gpu), shift.to(gpu), scale.to(gpu), segments)
    q, s = o.prepare_activation(h, convrot=True)
    assert_bits_equal(np_of(codes), q, 'modulated_norm_quantize codes')
    assert_bits_equal(np_of(row_scale).reshape(-1), s, 'modulated_norm_quantize scales')
    with pytest.raises(ValueError):
        flow.modulated_norm(norm, x.to(gpu), shift.to(gpu), scale.to(gpu), [(0, 100, 2)])


def test_dit_ffn_block_full_size_sampled_rows(gpu):
    data = workloads.dit_ffn()
    block = _ffn_module(data, gpu, 3072, 8192)
    h = data['h'].to(gpu)
    res = data['residual'].to(gpu)
    out = block(h, res)
    torch.cuda.synchronize()
    rows = np.random.default_rng(0).choice(16384, 48, replace=False)
    rows[:2] = [0, 16383]
    want = o.ffn_block(np_of(data['h'])[rows], np_of(block.fc1.weight), np_of(block.fc1.weight_scale).reshape(-1),
                       np_of(block.fc2.weight), np_of(block.fc2.weight_scale).reshape(-1),
                       np_of(data['residual'])[rows])
    assert_bits_equal(np_of(out)[rows], want, 'ffn block M=16384 sampled rows')
    assert torch.isfinite(out).all()


def test_chunked_rows_equals_whole(gpu):
    g = torch.Generator().manual_seed(6)
    x = randn16(g, (1000, 512), 1.0)
    w = torch.randn((256, 512), generator=g) * 0.02
    wq, ws = _wq(w, gpu)
    whole = dit_column_linear.column_linear(x.to(gpu), wq, ws)
    fn = lambda xc: dit_column_linear.column_linear(xc, wq, ws)  # noqa: E731
    assert torch.equal(chunked_rows(fn, x.to(gpu), chunk_rows=384), whole)
    out = torch.empty_like(whole)
    assert torch.equal(chunked_rows(fn, x.to(gpu), chunk_rows=256, out=out), whole)


def test_gemm_w8a8_linear_full_size(gpu):
    data = workloads.w8a8_linear()
    wq, ws = _wq(data['w'], gpu)
    q, a = kernels.quantize_rows(data['x'].to(gpu))
    y = kernels.gemm(q, wq, epilogue=kernels.EPI_ROW, row_scale=a, col_scale=ws, bias=data['bias'].to(gpu))
    oq, oa = o.quantize_rows(np_of(data['x']).astype(np.float32))
    assert_bits_equal(np_of(q), oq, 'c0 codes')
    acc = kernels.gemm(q, wq)
    assert_bits_equal(np_of(acc), o.int_mm(oq, np_of(wq)), 'c0 int32')
    assert_bits_equal(np_of(y), o.dequantize_row(np_of(acc), oa, np_of(ws), 'f16', np_of(data['bias'])), 'c0 out')


def test_dit_qkv_full_size_with_bias(gpu):
    """The DiT QKV workload (53504 x 3072 -> 9216, ConvRot256, FP16 bias in
    the epilogue) on sampled rows against the oracle."""
    data = workloads.dit_qkv()
    print('DiT QKV 53504 x 3072 -> 9216 with bias', flush=True)
    wq, ws = _wq(data['w'], gpu)
    y = dit_column_linear.column_linear(data['x'].to(gpu), wq, ws, bias=data['bias'].to(gpu))
    assert y.shape == (53504, 9216) and torch.isfinite(y).all()
    rows = np.array([0, 1, 255, 256, 26751, 40000, 53248, 53502, 53503])
    want = o.column_linear(np_of(data['x'])[rows], np_of(wq), np_of(ws).reshape(-1), convrot=True,
                           bias=np_of(data['bias']))
    assert_bits_equal(np_of(y[torch.from_numpy(rows).to(gpu)]), want, 'c2 rows with bias')
    plain = dit_column_linear.column_linear(data['x'].to(gpu), wq, ws)
    assert not torch.equal(plain, y)


def test_row_linear_writes_into_a_row_range(gpu):
    g = torch.Generator().manual_seed(41)
    x = (torch.randn((70, 2 * 512), generator=g) * 0.5).half().to(gpu)
    w = torch.randn((256, 512), generator=g) * 0.02
    wq, ws = _wq(w, gpu)
    full = torch.full((100, 256), float('nan'), device=gpu)
    got = swiglu_quant.row_linear(x, wq, ws, out=full[20:90])
    want = swiglu_quant.row_linear(x, wq, ws)
    assert got.data_ptr() == full[20:90].data_ptr()
    assert torch.equal(full[20:90], want)
    assert torch.isnan(full[:20]).all() and torch.isnan(full[90:]).all()
