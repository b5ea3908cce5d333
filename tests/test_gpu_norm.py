"""GPU parity of the fused modulated-RMSNorm -> ConvRot256 -> INT8 kernel
against the CPU oracle (bit-exact codes, scales and normalized rows)."""
import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of, randn16, tname
from w8a8 import kernels

pytestmark = pytest.mark.gpu

EPS = 1e-6 / 512 ** 2   # the DiT norm epsilon after the residual-divisor fold


def _tables(g, cols, rows, mod_rows=9):
    w = torch.rand((cols,), generator=g) + 0.5
    shift = torch.randn((mod_rows, cols), generator=g) * 0.1
    scale = torch.randn((mod_rows, cols), generator=g) * 0.1
    labels = torch.randint(0, mod_rows, (rows,), generator=g, dtype=torch.int32)
    return w, shift, scale, labels


def _oracle(x, w, shift, scale, labels, mode, dtype, eps=EPS):
    dt = tname(dtype)
    xs = np_of(x)
    args = (None if w is None else np_of(w), None if shift is None else np_of(shift),
            None if scale is None else np_of(scale), None if labels is None else np_of(labels))
    if mode == 'norm':
        return None, None, o.modulated_rms_norm(xs, *args, eps=eps, x_dtype=dt)
    q, s, y = o.norm_quantize(xs, *args, eps=eps, x_dtype=dt, convrot=mode != 'plain',
                              round_rotated=mode != 'rot32')
    return q, s, y


def _run(x, w, shift, scale, labels, mode, gpu, eps=EPS):
    dev = lambda t: None if t is None else t.to(gpu)  # noqa: E731
    return kernels.norm_quantize(dev(x), dev(w), dev(shift), dev(scale), dev(labels), eps=eps,
                                 quantize=mode != 'norm', convrot=mode != 'plain', round_rotated=mode != 'rot32',
                                 want_normalized=True)


def _check(r, want, what):
    q, s, y = want
    assert_bits_equal(np_of(r['y']), y, f'{what}: normalized rows')
    if q is not None:
        assert_bits_equal(np_of(r['scale']).reshape(-1), s, f'{what}: scales')
        assert_bits_equal(np_of(r['q']), q, f'{what}: codes')


NORM_CASES = [
    (1, 256, 'rot'), (13, 3072, 'rot'), (7, 5376, 'rot'), (5, 8192, 'rot'), (3, 12288, 'rot'),
    (1030, 3072, 'rot'), (1030, 5376, 'rot'),
    (13, 1040, 'plain'), (9, 3072, 'plain'), (3, 16384, 'plain'),
    (11, 3072, 'rot32'), (4, 12288, 'rot32'),
    (13, 3072, 'norm'), (5, 1040, 'norm'), (3, 12288, 'norm'),
]


@pytest.mark.parametrize('rows,cols,mode', NORM_CASES)
@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
def test_norm_quantize_matches_oracle(gpu, rows, cols, mode, dtype):
    g = torch.Generator().manual_seed(rows * 17 + cols)
    x = randn16(g, (rows, cols), 4.0, dtype)
    if cols >= 64:
        x[:, 3] *= 20       # outlier channel
    if rows > 2:
        x[1] = 0            # zero row: inv = 1/sqrt(eps), the row becomes the shift row
    w, shift, scale, labels = _tables(g, cols, rows)
    r = _run(x, w, shift, scale, labels, mode, gpu)
    _check(r, _oracle(x, w, shift, scale, labels, mode, dtype), f'{rows}x{cols} {mode} {dtype}')


@pytest.mark.parametrize('with_weight,with_mod', [(False, False), (True, False), (False, True)])
def test_norm_optional_gain_and_modulation(gpu, with_weight, with_mod):
    g = torch.Generator().manual_seed(3 + with_weight * 2 + with_mod)
    rows, cols = 37, 3072
    x = randn16(g, (rows, cols), 2.0)
    w, shift, scale, labels = _tables(g, cols, rows)
    w = w if with_weight else None
    if not with_mod:
        shift = scale = labels = None
    r = _run(x, w, shift, scale, labels, 'rot', gpu)
    _check(r, _oracle(x, w, shift, scale, labels, 'rot', torch.float16), f'weight={with_weight} mod={with_mod}')


@pytest.mark.parametrize('cols', [3072, 4096, 4112])
@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
def test_norm_only_segments(gpu, cols, dtype):
    # The norm-only DiT form stages the gain and the first row's shift and
    # scale rows in each 8-row workgroup (up to 4096 columns): labels in
    # segments that start inside workgroups (rows of one workgroup with two
    # labels), a last workgroup of 3 rows, and 4112 columns on the unstaged path.
    rows = 8 * 37 + 3
    g = torch.Generator().manual_seed(cols + rows)
    x = randn16(g, (rows, cols), 4.0, dtype)
    w, shift, scale, _ = _tables(g, cols, rows)
    bounds = [0, 5, 61, 62, 130, 211, 299]
    labels = torch.zeros((rows,), dtype=torch.int32)
    for i in range(len(bounds) - 1):
        labels[bounds[i]:bounds[i + 1]] = (3 * i + 1) % 9
    r = _run(x, w, shift, scale, labels, 'norm', gpu)
    _check(r, _oracle(x, w, shift, scale, labels, 'norm', dtype), f'norm-only segments {rows}x{cols} {dtype}')


def test_norm_labels_clamped_and_segments(gpu):
    g = torch.Generator().manual_seed(8)
    rows, cols = 10, 512
    x = randn16(g, (rows, cols))
    w, shift, scale, _ = _tables(g, cols, rows, mod_rows=4)
    labels = torch.tensor([-3, 0, 1, 2, 3, 4, 9, 1, 1, 0], dtype=torch.int32)
    r = _run(x, w, shift, scale, labels, 'rot', gpu)
    _check(r, _oracle(x, w, shift, scale, labels.clamp(0, 3), 'rot', torch.float16), 'clamped labels')


def test_norm_strided_rows_extremes_and_eps(gpu):
    g = torch.Generator().manual_seed(9)
    rows, cols = 21, 3072
    big = randn16(g, (rows, cols + 256), 1.0)
    big[0, :cols] = 60000.0                  # squares near 3.6e9, sum near 1.1e13
    big[1, :cols:2] = -60000.0
    big[2, :cols] = 2.0 ** -14               # smallest normal fp16
    big[3, :cols] = 0.0
    x = big[:, :cols]                        # row stride cols + 256
    w, shift, scale, labels = _tables(g, cols, rows)
    for eps in (EPS, 1e-5, 0.5):
        r = _run(x, w, shift, scale, labels, 'rot', gpu, eps=eps)
        _check(r, _oracle(x.contiguous(), w, shift, scale, labels, 'rot', torch.float16, eps=eps),
               f'strided eps={eps}')


def test_norm_codes_equal_quantize_of_normalized_rows(gpu):
    # The fused kernel's codes are exactly those of quantizing its own
    # normalized output with the standalone quantizer.
    g = torch.Generator().manual_seed(10)
    rows, cols = 300, 3072
    x = randn16(g, (rows, cols), 3.0).to(gpu)
    w, shift, scale, labels = (t.to(gpu) for t in _tables(g, cols, rows))
    r = kernels.norm_quantize(x, w, shift, scale, labels, eps=EPS, want_normalized=True)
    q, s = kernels.quantize_rows(r['y'], convrot=True, round_rotated=True)
    assert torch.equal(q, r['q']) and torch.equal(s, r['scale'])
