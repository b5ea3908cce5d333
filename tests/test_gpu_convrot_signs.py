"""GPU parity of the seeded ConvRot sign option: every kernel that rotates
(the column path's quantizer and its maximum phase, the FC2 prologue, the
fused norm) with sign words, bit for bit against the oracle's signed
rotation, on each of the kernels' row layouts; and weights rotated with the
same signs keeping a W8A8 projection's output."""
import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of, randn16, tname
from w8a8 import convrot, kernels

pytestmark = pytest.mark.gpu

QUANT_CASES = [
    (7, 3072),       # a 16-wave workgroup per row (no more rows than CUs)
    (300, 768),      # 4-wave workgroups (more rows than CUs), one 16-column unit per thread
    (1050, 12800),   # 4-wave workgroups, four units per thread
    (2100, 512),     # a wavefront per row, one unit per lane
    (2050, 3072),    # a wavefront per row, three units per lane
    (2, 16640),      # a wavefront per row streaming a row wider than 16384 columns
]


def _f32(x):
    return x.float().numpy()


def _rounded(r, dtype):
    return torch.from_numpy(r).to(dtype).float().numpy() if dtype != torch.float32 else r


@pytest.mark.parametrize('rows,cols', QUANT_CASES)
@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32])
def test_quantize_rows_with_signs(gpu, rows, cols, dtype):
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = randn16(g, (rows, cols), 3.0, dtype)
    x[:, 5] *= 20
    x[1] = 0
    s = convrot.signs(cols, rows + cols)
    words = convrot.sign_words(s, gpu)
    xg = x.to(gpu)
    print(f'signed quantize {rows}x{cols} {dtype}', flush=True)
    q, sc = kernels.quantize_rows(xg, convrot=True, round_rotated=True, signs=words)
    wq, ws = o.prepare_activation(np_of(x), convrot=True, x_dtype=tname(dtype), signs=s.numpy())
    assert_bits_equal(np_of(sc).reshape(-1), ws, 'scales (rotation in x dtype)')
    assert_bits_equal(np_of(q), wq, 'codes (rotation in x dtype)')
    rot = o.convrot256(_f32(x), s.numpy())
    q, sc = kernels.quantize_rows(xg, convrot=True, round_rotated=False, signs=words)
    wq, ws = o.quantize_rows(rot)
    assert_bits_equal(np_of(sc).reshape(-1), ws, 'scales (fp32 rotation)')
    assert_bits_equal(np_of(q), wq, 'codes (fp32 rotation)')
    for rr in (True, False):
        m = kernels.row_absmax(xg, convrot=True, round_rotated=rr, signs=words)
        want = np.abs(_rounded(rot, dtype) if rr else rot).max(-1)
        assert_bits_equal(np_of(m).reshape(-1), want, f'row maximum round_rotated={rr}')
    # the signs matter: unsigned codes differ
    assert not torch.equal(kernels.quantize_rows(xg, convrot=True)[0].cpu(), torch.from_numpy(wq))


SWIGLU_CASES = [
    (3, 512),        # 16-wave workgroups, rotated row kept in registers
    (2, 20480),      # 16-wave workgroups, two passes
    (1, 66048),      # 16-wave workgroups, streaming (258 groups)
    (300, 3072),     # 4-wave workgroups (more rows than CUs)
    (300, 20480),    # 4-wave workgroups, streaming
]


@pytest.mark.parametrize('rows,width', SWIGLU_CASES)
@pytest.mark.parametrize('dtype', [torch.float16, torch.float32])
def test_swiglu_quantize_with_signs(gpu, rows, width, dtype):
    g = torch.Generator().manual_seed(rows + width)
    x = randn16(g, (rows, 2 * width), 3.0, dtype)
    s = convrot.signs(width, width + 1)
    print(f'signed swiglu {rows}x{width} {dtype}', flush=True)
    res = kernels.swiglu_quantize(x.to(gpu), want_row_max=True, want_group_max=True,
                                  signs=convrot.sign_words(s, gpu))
    wq, ws, wg = o.fc2_prologue(np_of(x), x_dtype=tname(dtype), signs=s.numpy())
    assert_bits_equal(np_of(res['group_max']), wg, 'group maxima')
    assert_bits_equal(np_of(res['row_max']).reshape(-1), wg.max(-1), 'row maxima')
    assert_bits_equal(np_of(res['scale']).reshape(-1), ws, 'scales')
    assert_bits_equal(np_of(res['q']), wq, 'codes')


NORM_CASES = [(13, 3072, True), (1030, 3072, True), (7, 5376, True), (4, 12288, False), (11, 3072, False)]


@pytest.mark.parametrize('rows,cols,round_rotated', NORM_CASES)
@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
def test_norm_quantize_with_signs(gpu, rows, cols, round_rotated, dtype):
    g = torch.Generator().manual_seed(rows * 3 + cols)
    x = randn16(g, (rows, cols), 4.0, dtype)
    w = torch.rand((cols,), generator=g) + 0.5
    shift = torch.randn((5, cols), generator=g) * 0.1
    scale = torch.randn((5, cols), generator=g) * 0.1
    labels = torch.randint(0, 5, (rows,), generator=g, dtype=torch.int32)
    s = convrot.signs(cols, cols)
    eps = 1e-6
    print(f'signed norm {rows}x{cols} round_rotated={round_rotated} {dtype}', flush=True)
    r = kernels.norm_quantize(x.to(gpu), w.to(gpu), shift.to(gpu), scale.to(gpu), labels.to(gpu), eps=eps,
                              round_rotated=round_rotated, want_normalized=True, signs=convrot.sign_words(s, gpu))
    q, sc, y = o.norm_quantize(np_of(x), np_of(w), np_of(shift), np_of(scale), np_of(labels), eps=eps,
                               x_dtype=tname(dtype), round_rotated=round_rotated, signs=s.numpy())
    assert_bits_equal(np_of(r['y']), y, 'normalized rows (signs do not touch them)')
    assert_bits_equal(np_of(r['scale']).reshape(-1), sc, 'scales')
    assert_bits_equal(np_of(r['q']), q, 'codes')


def test_rotated_weights_keep_the_projection(gpu):
    """x W^T through the INT8 path with signed rotation on both sides: the
    error against float64 is the quantization's (as without signs), while
    weights rotated without the signs give an unrelated result."""
    g = torch.Generator().manual_seed(8)
    x = torch.randn((64, 1536), generator=g)
    w = torch.randn((512, 1536), generator=g) * 0.05
    s = convrot.signs(1536, 21)
    ref = x.double() @ w.double().t()

    def project(signs, wrot):
        qa, sa = kernels.quantize_rows(x.half().to(gpu), convrot=True, signs=signs)
        qw, sw = kernels.quantize_rows(wrot.to(gpu))
        return kernels.gemm(qa, qw, epilogue=kernels.EPI_ROW, row_scale=sa, col_scale=sw,
                            out_dtype=torch.float32).cpu().double()

    def rel(y):
        return float((y - ref).norm() / ref.norm())

    signed = rel(project(convrot.sign_words(s, gpu), convrot.rotate_weight(w, s)))
    plain = rel(project(None, convrot.rotate_weight(w)))
    mixed = rel(project(convrot.sign_words(s, gpu), convrot.rotate_weight(w)))
    print(f'relative error: signed {signed:.4f}, unsigned {plain:.4f}, mismatched {mixed:.4f}')
    assert signed < 0.02 and plain < 0.02 and signed < 1.5 * plain
    assert mixed > 0.5
