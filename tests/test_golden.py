"""Committed golden fixtures: the oracle reproduces them (CPU) and the HIP
kernels reproduce them bit for bit (GPU)."""
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / 'golden'


def load(name):
    with np.load(GOLDEN / f'{name}.npz', allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_golden_fixtures():
    from golden.make_golden import fixtures
    for name, arrays in fixtures().items():
        saved = load(name)
        assert set(saved) == set(arrays), name
        for k, v in arrays.items():
            assert saved[k].dtype == v.dtype and np.array_equal(saved[k].view(np.uint8), v.view(np.uint8)), (name, k)


@pytest.mark.gpu
def test_kernels_reproduce_golden_fixtures(gpu):
    import torch
    from helpers import assert_bits_equal, np_of
    from w8a8 import kernels

    d = load('quant')
    q, s = kernels.quantize_rows(torch.from_numpy(d['x']).to(gpu))
    assert_bits_equal(np_of(q), d['q'], 'golden quant codes')
    assert_bits_equal(np_of(s).reshape(-1), d['scale'], 'golden quant scale')
    d = load('quant_convrot')
    q, s = kernels.quantize_rows(torch.from_numpy(d['x']).to(gpu), convrot=True)
    assert_bits_equal(np_of(q), d['q'], 'golden convrot codes')
    d = load('swiglu')
    r = kernels.swiglu_quantize(torch.from_numpy(d['x']).to(gpu), want_group_max=True)
    assert_bits_equal(np_of(r['q']), d['q'], 'golden swiglu codes')
    assert_bits_equal(np_of(r['group_max']), d['group_max'], 'golden swiglu group max')
    d = load('gemm')
    c = kernels.gemm(torch.from_numpy(d['a']).to(gpu), torch.from_numpy(d['b']).to(gpu))
    assert_bits_equal(np_of(c), d['c'], 'golden gemm')
    d = load('epilogue')
    acc, a, w = (torch.from_numpy(d[k]).to(gpu) for k in ('acc', 'a', 'w'))
    b = torch.from_numpy(d['bias']).to(gpu)
    assert_bits_equal(np_of(kernels.dequantize(acc, a, w, epilogue=kernels.EPI_ROW, bias=b)), d['row_f16'], 'row f16')
    assert_bits_equal(np_of(kernels.dequantize(acc, a, w, epilogue=kernels.EPI_ROW, out_dtype=torch.float32)),
                      d['row_f32'], 'row f32')
    assert_bits_equal(np_of(kernels.dequantize(acc, a, w, epilogue=kernels.EPI_COLUMN, bias=b)), d['col_f16'],
                      'col f16')
    assert_bits_equal(np_of(kernels.dequantize(acc, a, w, epilogue=kernels.EPI_COLUMN, out_dtype=torch.bfloat16)),
                      d['col_bf16'], 'col bf16')


@pytest.mark.gpu
def test_kernels_reproduce_golden_fixtures_of_the_dit_rows(gpu):
    import torch
    from helpers import assert_bits_equal, np_of
    from w8a8 import kernels

    t = lambda a: torch.from_numpy(a).to(gpu)  # noqa: E731
    d = load('gated')
    got = kernels.dequantize(t(d['acc']), t(d['a']), t(d['w']), epilogue=kernels.EPI_ROW, residual=t(d['residual']),
                             gate=t(d['gate']), gate_labels=t(d['labels']))
    assert_bits_equal(np_of(got), d['out'], 'golden gated residual')
    d = load('norm_quant')
    r = kernels.norm_quantize(t(d['x']), t(d['weight']), t(d['shift']), t(d['scale']), t(d['labels']), eps=1e-6,
                              want_normalized=True)
    assert_bits_equal(np_of(r['y']), d['y'], 'golden modulated norm')
    assert_bits_equal(np_of(r['q']), d['q'], 'golden norm codes')
    assert_bits_equal(np_of(r['scale']).reshape(-1), d['row_scale'], 'golden norm row scales')
    d = load('rms_rope')
    q, k = kernels.rms_rope(t(d['packed']), t(d['freqs']), t(d['q_gain']), t(d['k_gain']), heads=2, rot_dim=96,
                            eps=1e-6)
    assert_bits_equal(np_of(q), d['q'], 'golden rms_rope q')
    assert_bits_equal(np_of(k), d['k'], 'golden rms_rope k')
    d = load('attention')
    prep = kernels.attention_prepare(t(d['q']), t(d['k']), t(d['v']))
    for name in ('q8', 'qs', 'k8', 'ks', 'vt8', 'vs', 'vsum'):
        assert_bits_equal(np_of(prep[name]), d[name], f'golden attention {name}')
    out = np_of(kernels.attention(prep, out_dtype=torch.float32)).astype(np.float64)
    # the GPU takes the hardware exp2 and its own FP32 order: within 1e-5 of
    # the oracle's output (the same u8 codes)
    err = np.abs(out - d['out']).max() / np.abs(d['out']).max()
    print(f'attention fixture: max |gpu - oracle| / max |oracle| = {err:.2e}')
    assert err <= 1e-5
