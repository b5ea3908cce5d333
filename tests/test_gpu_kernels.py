"""GPU parity of each libw8a8 kernel against the CPU oracle (bit-exact).

Inputs are drawn on the CPU (seeded), copied to the GPU, and the GPU result
is compared with the oracle on the same bytes: int8 codes, int32
accumulators, fp32 scales and the stored fp16/bf16/fp32 outputs must be
bit-identical.
"""
import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of, randi8, randn16, tname
from w8a8 import kernels

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ GEMM int32
GEMM_SHAPES = [(1, 16, 16), (13, 48, 64), (64, 64, 128), (256, 256, 64), (300, 520, 192), (257, 260, 80),
               (1000, 1100, 3072), (4096, 3072, 3072),
               # weight-streaming (M <= 64) shapes: text-encoder up/down, ragged N
               (1, 14336, 4096), (64, 4096, 14336), (37, 1000, 1024), (5, 520, 192), (65, 4096, 512),
               # 64 weight rows per workgroup (M 49..64, N >= 12288), ragged last workgroup
               (64, 14336, 4096), (50, 12352, 256),
               # up to 8 rows: the register-batched kernel where its 16-row grid fills 128..256 CUs
               # (N = 4000), the streaming kernel elsewhere (one 16-row block; N = 16 below one
               # 64-row block, N = 5000 past the CUs)
               (6, 4000, 1024), (2, 16, 128), (8, 5000, 1024)]


@pytest.mark.parametrize('m,n,k', GEMM_SHAPES)
def test_gemm_int32_exact(gpu, m, n, k):
    g = torch.Generator().manual_seed(m * 7 + n * 3 + k)
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_INT32)
    assert_bits_equal(np_of(got), o.int_mm(np_of(a), np_of(b)), f'gemm {m}x{n}x{k}')


def _dispatch_sweep_shapes(count=48, seed=2024):
    """Seeded shapes spread over every kernel choice of the GEMM dispatch:
    M = 1 (GEMV), 2..8 and 9..16 (register-batched or weight-streaming by N),
    17..64 (weight streaming, split K or not), 65..3000 (persistent tiles of
    each shape, split K or not), ragged N from one partial tile to past the
    CU count in 64-row blocks, and K from 16 (multiples of 16, 64, 128, 256)."""
    rng = np.random.default_rng(seed)
    shapes = []
    while len(shapes) < count:
        m = int(rng.choice([1, rng.integers(2, 9), rng.integers(9, 17), rng.integers(17, 65),
                            rng.integers(65, 701), rng.integers(701, 3001)]))
        n = int(rng.choice([rng.integers(1, 600), rng.integers(2049, 4097), rng.integers(4097, 22000)]))
        k = int(rng.choice([16, 64, 128, 256]) * rng.integers(1, 48))
        if m * n * k <= 4e9:
            shapes.append((m, n, k))
    return shapes


@pytest.mark.parametrize('m,n,k', _dispatch_sweep_shapes())
def test_gemm_dispatch_sweep(gpu, m, n, k):
    print(f'sweep gemm {m}x{n}x{k}', flush=True)
    g = torch.Generator().manual_seed(m * 131 + n * 17 + k)
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    acc = o.int_mm(np_of(a), np_of(b))
    ag, bg = a.to(gpu), b.to(gpu)
    assert_bits_equal(np_of(kernels.gemm(ag, bg)), acc, f'int32 {m}x{n}x{k}')
    rs = torch.rand((m, 1), generator=g) * 0.01 + 1e-4
    ws = torch.rand((n, 1), generator=g) * 1e-3 + 1e-6
    want = o.dequantize_row(acc, np_of(rs), np_of(ws), 'f16')
    none = torch.empty(0, dtype=torch.uint8, device=gpu)
    for workspace in (None, none):     # the split the shape plans, and unsplit
        got = kernels.gemm(ag, bg, epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                           out_dtype=torch.float16, workspace=workspace)
        assert_bits_equal(np_of(got), want, f'row f16 {m}x{n}x{k} ws={workspace is None}')


def test_gemm_signed_extremes_and_layout(gpu):
    k = 5120
    a = torch.full((33, k), -128, dtype=torch.int8)
    b = torch.full((40, k), -128, dtype=torch.int8)
    b[7] = 127
    a[5, ::2] = 127
    got = np_of(kernels.gemm(a.to(gpu), b.to(gpu)))
    assert_bits_equal(got, o.int_mm(np_of(a), np_of(b)), 'extremes')
    assert got[0, 0] == k * 128 * 128
    # one-hot operands pin the row/column placement of every accumulator
    eye_a = torch.zeros((48, 64), dtype=torch.int8)
    eye_b = torch.zeros((80, 64), dtype=torch.int8)
    for i in range(48):
        eye_a[i, i % 64] = 1 + (i % 5)
    for j in range(80):
        eye_b[j, j % 64] = 1 + (j % 3)
    got = np_of(kernels.gemm(eye_a.to(gpu), eye_b.to(gpu)))
    assert_bits_equal(got, o.int_mm(np_of(eye_a), np_of(eye_b)), 'one-hot')


def test_gemm_strided_operands_and_empty(gpu):
    g = torch.Generator().manual_seed(5)
    big = randi8(g, (70, 160))
    a = big[:, :96]              # row stride 160
    b = randi8(g, (33, 96))
    got = kernels.gemm(a.to(gpu), b.to(gpu))
    assert_bits_equal(np_of(got), o.int_mm(np_of(a).copy(), np_of(b)), 'strided')
    empty = kernels.gemm(torch.zeros((0, 64), dtype=torch.int8, device=gpu),
                         torch.zeros((8, 64), dtype=torch.int8, device=gpu))
    assert empty.shape == (0, 8)


# ------------------------------------------------------------------ epilogues
@pytest.mark.parametrize('epi', ['row', 'column'])
@pytest.mark.parametrize('out_dtype', [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize('bias_dtype', [None, torch.float16, torch.float32])
def test_gemm_fused_epilogue(gpu, epi, out_dtype, bias_dtype):
    g = torch.Generator().manual_seed(11)
    # 521 x 300: full tiles (staged epilogue) and ragged edge tiles (128 x 256 tiles on 256 CUs)
    m, n, k = 521, 300, 256
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.05 + 1e-4
    ws = torch.rand((n, 1), generator=g) * 1e-3 + 1e-6
    bias = None if bias_dtype is None else (torch.randn((n,), generator=g) * 0.5).to(bias_dtype)
    code = kernels.EPI_ROW if epi == 'row' else kernels.EPI_COLUMN
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=code, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       bias=None if bias is None else bias.to(gpu), out_dtype=out_dtype)
    acc = o.int_mm(np_of(a), np_of(b))
    fn = o.dequantize_row if epi == 'row' else o.dequantize_column
    want = fn(acc, np_of(rs).reshape(-1), np_of(ws).reshape(-1), tname(out_dtype),
              None if bias is None else np_of(bias))
    assert_bits_equal(np_of(got), want, f'{epi} {out_dtype} {bias_dtype}')


@pytest.mark.parametrize('m', [1, 33, 64])
@pytest.mark.parametrize('epi,out_dtype,bias_dtype', [('row', torch.float16, torch.float16),
                                                      ('column', torch.bfloat16, None),
                                                      ('row', torch.float32, torch.float32),
                                                      ('column', torch.float16, torch.float32)])
def test_gemm_skinny_epilogues(gpu, m, epi, out_dtype, bias_dtype):
    g = torch.Generator().manual_seed(m + 17)
    n, k = 1000, 2048
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.05 + 1e-4
    ws = torch.rand((n, 1), generator=g) * 1e-3 + 1e-6
    bias = None if bias_dtype is None else (torch.randn((n,), generator=g) * 0.5).to(bias_dtype)
    code = kernels.EPI_ROW if epi == 'row' else kernels.EPI_COLUMN
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=code, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       bias=None if bias is None else bias.to(gpu), out_dtype=out_dtype)
    fn = o.dequantize_row if epi == 'row' else o.dequantize_column
    want = fn(o.int_mm(np_of(a), np_of(b)), np_of(rs).reshape(-1), np_of(ws).reshape(-1), tname(out_dtype),
              None if bias is None else np_of(bias))
    assert_bits_equal(np_of(got), want, f'skinny m={m} {epi} {out_dtype} {bias_dtype}')


GEMV_CASES = [
    # (n, k): M == 1 takes the GEMV. On 256 CUs a wave owns 4 weight rows
    # when N >= 16381, 2 when N >= 8191, else 1; ragged N leaves the last wave
    # fewer rows, and K that is not a multiple of a batch (64 lanes x 4 or 8
    # chunks of 16 bytes) leaves lanes without a chunk.
    (16386, 1040), (8194, 4096), (4097, 14336), (1001, 1040), (3, 16),
]


@pytest.mark.parametrize('n,k', GEMV_CASES)
def test_gemv(gpu, n, k):
    print(f'gemv 1x{n}x{k}', flush=True)
    g = torch.Generator().manual_seed(n + k)
    a = randi8(g, (1, k))
    b = randi8(g, (n, k))
    rs = torch.rand((1, 1), generator=g) * 0.01 + 1e-4
    ws = (torch.rand((n, 1), generator=g) * 1e-3 + 1e-6) / 512
    bias = (torch.randn((n,), generator=g) * 0.01).half()
    res = randn16(g, (1, n), 1 / 512)
    acc = o.int_mm(np_of(a), np_of(b))
    ag, bg = a.to(gpu), b.to(gpu)
    assert_bits_equal(np_of(kernels.gemm(ag, bg)), acc, f'gemv int32 1x{n}x{k}')
    got = kernels.gemm(ag, bg, epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       bias=bias.to(gpu), residual=res.to(gpu), out_dtype=torch.float16)
    want = o.residual_add(np_of(res), o.dequantize_row(acc, np_of(rs), np_of(ws), 'f16', np_of(bias)))
    assert_bits_equal(np_of(got), want, f'gemv row+bias+residual 1x{n}x{k}')
    got = kernels.gemm(ag, bg, epilogue=kernels.EPI_COLUMN, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       out_dtype=torch.float32)
    assert_bits_equal(np_of(got), o.dequantize_column(acc, np_of(rs), np_of(ws), 'f32'), f'gemv column 1x{n}x{k}')


def test_gemv_extremes(gpu):
    # |sum| reaches K * 128 * 128 = 2^31 * 0.109 at K = 14336: exact in int32.
    k = 14336
    a = torch.full((1, k), -128, dtype=torch.int8)
    b = torch.full((9, k), -128, dtype=torch.int8)
    b[3] = 127
    b[5, 1::2] = 127
    got = np_of(kernels.gemm(a.to(gpu), b.to(gpu)))
    assert_bits_equal(got, o.int_mm(np_of(a), np_of(b)), 'gemv extremes')
    assert got[0, 0] == k * 128 * 128 and got[0, 3] == -k * 128 * 127


STREAM_CASES = [
    # (m, n, k): 2 <= M <= 64 with K % 128 == 0 takes the weight-streaming kernel
    # (up to 8 rows only where the register-batched kernel's grid would not fill the CUs).
    # On 256 CUs these split K two (40 x 10750: 168 row blocks of 64), four
    # (64 x 4100 and the text-encoder down shapes) or eight ways (17 x 203,
    # 33 x 512 x 5120: five steps per workgroup), partials in the workspace,
    # unless the workspace is withheld; ragged N and M. 33 x 20500 x 640 has
    # more row blocks (321) than CUs and does not split.
    (20, 4096, 14336), (64, 4100, 4096), (17, 203, 14336), (49, 4096, 14336), (40, 10750, 1024),
    (33, 512, 5120), (33, 20500, 640),
    # one 16-row activation block: 3 rows (K split two ways), 12 rows (four ways, ragged N)
    (3, 5120, 1280), (12, 4000, 2048),
]


@pytest.mark.parametrize('m,n,k', STREAM_CASES)
def test_gemm_stream_split_and_whole(gpu, m, n, k):
    print(f'stream gemm {m}x{n}x{k}', flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.01 + 1e-4
    ws = (torch.rand((n, 1), generator=g) * 1e-3 + 1e-6) / 512
    bias = (torch.randn((n,), generator=g) * 0.01).half()
    res = randn16(g, (m, n), 1 / 512)
    assert (kernels.gemm_workspace_bytes(m, n, k, gpu) > 0) == (n <= 16384)   # the default call splits K
    acc = o.int_mm(np_of(a), np_of(b))
    ag, bg = a.to(gpu), b.to(gpu)
    none = torch.empty(0, dtype=torch.uint8, device=gpu)
    for workspace in (None, none):
        assert_bits_equal(np_of(kernels.gemm(ag, bg, workspace=workspace)), acc, f'int32 ws={workspace is None}')
        got = kernels.gemm(ag, bg, epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                           bias=bias.to(gpu), residual=res.to(gpu), out_dtype=torch.float16, workspace=workspace)
        want = o.residual_add(np_of(res), o.dequantize_row(acc, np_of(rs), np_of(ws), 'f16', np_of(bias)))
        assert_bits_equal(np_of(got), want, f'row+bias+residual ws={workspace is None}')
        got = kernels.gemm(ag, bg, epilogue=kernels.EPI_COLUMN, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                           out_dtype=torch.float32, workspace=workspace)
        assert_bits_equal(np_of(got), o.dequantize_column(acc, np_of(rs), np_of(ws), 'f32'),
                          f'column f32 ws={workspace is None}')


def test_gemm_stream_strided_weight_and_short_k(gpu):
    g = torch.Generator().manual_seed(23)
    wide = randi8(g, (300, 1536))
    b = wide[:, :1024]                  # weight row stride 1536
    a = randi8(g, (33, 1024))
    got = kernels.gemm(a.to(gpu), wide.to(gpu)[:, :1024])
    assert_bits_equal(np_of(got), o.int_mm(np_of(a), np_of(b).copy()), 'strided weight')
    # K = 128 and 256: one or two steps, so some of the four waves get none
    for k in (128, 256, 384):
        a = randi8(g, (64, k))
        b = randi8(g, (130, k))
        assert_bits_equal(np_of(kernels.gemm(a.to(gpu), b.to(gpu))), o.int_mm(np_of(a), np_of(b)), f'k={k}')


@pytest.mark.parametrize('m,n,k', [(4096, 3072, 3072), (2000, 2900, 16384), (700, 3000, 1024), (353, 5120, 12800),
                                   (353, 512, 5120)])
def test_gemm_tile_shapes(gpu, m, n, k):
    # Shapes the host plans with the narrower tiles, on 256 CUs: 256 x 192
    # tiles, 16 x 16 = 256 of them filling the GPU where 256 x 256 leaves 64
    # CUs idle (4096 x 3072), and with K split two ways and ragged edges in M
    # and N (2000 x 2900: last tiles of 208 rows and 20 columns); 128 x 256
    # tiles for M of a few hundred rows, unsplit (700 x 3000: last tile of 60
    # rows), K split four (353 x 5120) and eight ways (353 x 512: two tile
    # columns, the second of 256). Every epilogue variant.
    print(f'tile shapes {m}x{n}x{k}', flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.01 + 1e-4
    ws = (torch.rand((n, 1), generator=g) * 1e-3 + 1e-6) / 512
    bias = (torch.randn((n,), generator=g) * 0.01).half()
    res = randn16(g, (m, n), 1 / 512)
    gate = torch.randn((5, n), generator=g)
    labels = torch.randint(0, 5, (m,), generator=g, dtype=torch.int32)
    acc = o.int_mm(np_of(a), np_of(b))
    ag, bg = a.to(gpu), b.to(gpu)
    assert_bits_equal(np_of(kernels.gemm(ag, bg)), acc, 'int32')
    row16 = o.dequantize_row(acc, np_of(rs), np_of(ws), 'f16', np_of(bias))
    got = kernels.gemm(ag, bg, epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       bias=bias.to(gpu), out_dtype=torch.float16)
    assert_bits_equal(np_of(got), row16, 'row + bias')
    got = kernels.gemm(ag, bg, epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       bias=bias.to(gpu), residual=res.to(gpu), out_dtype=torch.float16)
    assert_bits_equal(np_of(got), o.residual_add(np_of(res), row16), 'row + bias + residual')
    got = kernels.gemm(ag, bg, epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       out_dtype=torch.float16, residual=res.to(gpu), gate=gate.to(gpu), gate_labels=labels.to(gpu))
    branch = o.dequantize_row(acc, np_of(rs), np_of(ws), 'f16')
    assert_bits_equal(np_of(got), o.gated_residual_add(np_of(res), branch, np_of(gate), np_of(labels)), 'gated')
    for out_dtype in (torch.float32, torch.bfloat16):
        got = kernels.gemm(ag, bg, epilogue=kernels.EPI_COLUMN, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                           out_dtype=out_dtype)
        assert_bits_equal(np_of(got), o.dequantize_column(acc, np_of(rs), np_of(ws), tname(out_dtype)),
                          f'column {out_dtype}')


def test_gemm_scalar_weight_scale_and_residual(gpu):
    g = torch.Generator().manual_seed(12)
    m, n, k = 130, 96, 512
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.01
    ws = torch.tensor([[3.0e-5]])
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_COLUMN, row_scale=rs.to(gpu),
                       col_scale=ws.to(gpu), out_dtype=torch.float16)
    acc = o.int_mm(np_of(a), np_of(b))
    assert_bits_equal(np_of(got), o.dequantize_column(acc, np_of(rs), np_of(ws), 'f16'), 'scalar scale')
    res = randn16(g, (m, n), 1 / 512)
    ws2 = (torch.rand((n, 1), generator=g) * 1e-3) / 512
    res_gpu = res.to(gpu)
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu),
                       col_scale=ws2.to(gpu), out_dtype=torch.float16, residual=res_gpu, out=res_gpu)
    want = o.residual_add(np_of(res), o.dequantize_row(acc, np_of(rs), np_of(ws2), 'f16'))
    assert_bits_equal(np_of(got), want, 'in-place residual')


@pytest.mark.parametrize('k', [64, 128, 192, 256, 320])
def test_gemm_more_tiles_than_cus(gpu, k):
    # 17 x 17 = 289 tiles of 256x256 on at most 256 persistent workgroups: a
    # workgroup runs several tiles (ragged edges included) and the operand
    # ring crosses tile boundaries after 1..5 K steps.
    g = torch.Generator().manual_seed(k)
    m, n = 4352, 4200
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_INT32)
    assert_bits_equal(np_of(got), o.int_mm(np_of(a), np_of(b)), f'gemm {m}x{n}x{k}')


@pytest.mark.parametrize('m,n,k', [(100, 70000, 128), (100, 70000, 384), (65, 66000, 640)])
def test_gemm_128_row_tiles_more_than_cus(gpu, m, n, k):
    # M <= 128 rows takes 128 x 256 tiles; past 65536 columns there are more
    # tiles than CUs (274 and 258), so a workgroup runs several tiles and the
    # three-stage operand ring crosses tile boundaries after 1, 3 or 5 K
    # steps, with the epilogue staging through a ring slot in between.
    print(f'128-row tiles {m}x{n}x{k}', flush=True)
    g = torch.Generator().manual_seed(m + k)
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.01 + 1e-4
    ws = (torch.rand((n, 1), generator=g) * 1e-3 + 1e-6) / 512
    res = randn16(g, (m, n), 1 / 512)
    acc = o.int_mm(np_of(a), np_of(b))
    ag, bg = a.to(gpu), b.to(gpu)
    assert_bits_equal(np_of(kernels.gemm(ag, bg)), acc, 'int32')
    got = kernels.gemm(ag, bg, epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       residual=res.to(gpu), out_dtype=torch.float16)
    want = o.residual_add(np_of(res), o.dequantize_row(acc, np_of(rs), np_of(ws), 'f16'))
    assert_bits_equal(np_of(got), want, 'row + residual')


@pytest.mark.parametrize('epi,out_dtype,bias_dtype,residual', [
    ('column', torch.float16, torch.float16, False), ('row', torch.float16, None, True),
    ('row', torch.float32, torch.float32, False), ('column', torch.bfloat16, None, False),
    ('row', torch.float16, torch.float32, True)])
def test_gemm_more_tiles_than_cus_epilogues(gpu, epi, out_dtype, bias_dtype, residual):
    g = torch.Generator().manual_seed(99)
    m, n, k = 4400, 4300, 128       # 18 x 17 tiles, ragged in both directions
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.05 + 1e-4
    ws = torch.rand((n, 1), generator=g) * 1e-3 + 1e-6
    bias = None if bias_dtype is None else (torch.randn((n,), generator=g) * 0.5).to(bias_dtype)
    res = randn16(g, (m, n), 0.25) if residual else None
    code = kernels.EPI_ROW if epi == 'row' else kernels.EPI_COLUMN
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=code, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       bias=None if bias is None else bias.to(gpu), out_dtype=out_dtype,
                       residual=None if res is None else res.to(gpu))
    fn = o.dequantize_row if epi == 'row' else o.dequantize_column
    want = fn(o.int_mm(np_of(a), np_of(b)), np_of(rs).reshape(-1), np_of(ws).reshape(-1), tname(out_dtype),
              None if bias is None else np_of(bias))
    if residual:
        want = o.residual_add(np_of(res), want)
    assert_bits_equal(np_of(got), want, f'{epi} {out_dtype} {bias_dtype} residual={residual}')


SPLITK_CASES = [
    # (m, n, k, epilogue, out dtype, bias dtype, residual): grids smaller than the CU count
    (512, 4096, 14336, 'int32', None, None, False),     # text-encoder down at M=512: 64 tiles of 128 x 256
    (300, 520, 2048, 'row', torch.float16, None, True),  # ragged rows and columns
    (300, 520, 2048, 'column', torch.bfloat16, torch.float16, False),
    (257, 1000, 1024, 'row', torch.float32, torch.float32, False),
]


@pytest.mark.parametrize('m,n,k,epi,out_dtype,bias_dtype,residual', SPLITK_CASES)
def test_gemm_split_k(gpu, m, n, k, epi, out_dtype, bias_dtype, residual):
    assert kernels.gemm_workspace_bytes(m, n, k, gpu) > 0, 'shape expected to split K'
    g = torch.Generator().manual_seed(m + n + k)
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    acc = o.int_mm(np_of(a), np_of(b))
    need = kernels.gemm_workspace_bytes(m, n, k, gpu)
    if epi == 'int32':
        got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_INT32)
        assert_bits_equal(np_of(got), acc, 'split-K int32')
        short = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_INT32,
                             workspace=torch.empty(need - 16, dtype=torch.uint8, device=gpu))
        assert_bits_equal(np_of(short), acc, 'int32 with a workspace too small to split')
        return
    rs = torch.rand((m, 1), generator=g) * 0.05 + 1e-4
    ws = torch.rand((n, 1), generator=g) * 1e-3 + 1e-6
    bias = None if bias_dtype is None else (torch.randn((n,), generator=g) * 0.5).to(bias_dtype)
    res = randn16(g, (m, n), 0.25) if residual else None
    code = kernels.EPI_ROW if epi == 'row' else kernels.EPI_COLUMN
    kw = dict(epilogue=code, row_scale=rs.to(gpu), col_scale=ws.to(gpu), out_dtype=out_dtype,
              bias=None if bias is None else bias.to(gpu), residual=None if res is None else res.to(gpu))
    got = kernels.gemm(a.to(gpu), b.to(gpu), **kw)
    unsplit = kernels.gemm(a.to(gpu), b.to(gpu), workspace=torch.empty(0, dtype=torch.uint8, device=gpu), **kw)
    # A workspace 16 bytes short of the partials: the GEMM runs unsplit.
    short = kernels.gemm(a.to(gpu), b.to(gpu), workspace=torch.empty(need - 16, dtype=torch.uint8, device=gpu), **kw)
    assert_bits_equal(np_of(short), np_of(got), 'a workspace too small to split')
    fn = o.dequantize_row if epi == 'row' else o.dequantize_column
    want = fn(acc, np_of(rs).reshape(-1), np_of(ws).reshape(-1), tname(out_dtype),
              None if bias is None else np_of(bias))
    if residual:
        want = o.residual_add(np_of(res), want)
    assert_bits_equal(np_of(got), want, f'split-K {epi} {out_dtype}')
    assert_bits_equal(np_of(unsplit), np_of(got), 'split-K equals the unsplit GEMM')


def test_gemm_split_k_gated_residual_and_reused_workspace(gpu):
    # The DiT gate in the split-K finish; the same workspace serves three
    # calls in a row (filled with 0xA5 first: the splits write every partial
    # before the finish reads it).
    m, n, k = 300, 520, 2048
    assert kernels.gemm_workspace_bytes(m, n, k, gpu) > 0
    g = torch.Generator().manual_seed(19)
    ws_buf = torch.full((kernels.gemm_workspace_bytes(m, n, k, gpu),), 0xA5, dtype=torch.uint8, device=gpu)
    for call in range(3):
        a = randi8(g, (m, k))
        b = randi8(g, (n, k))
        rs = torch.rand((m, 1), generator=g) * 0.01 + 1e-4
        ws = (torch.rand((n, 1), generator=g) * 1e-3 + 1e-6) / 512
        res = randn16(g, (m, n), 1 / 512)
        gate = torch.randn((9, n), generator=g)
        labels = torch.randint(0, 9, (m,), generator=g, dtype=torch.int32)
        got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu),
                           col_scale=ws.to(gpu), out_dtype=torch.float16, residual=res.to(gpu), gate=gate.to(gpu),
                           gate_labels=labels.to(gpu), workspace=ws_buf)
        branch = o.dequantize_row(o.int_mm(np_of(a), np_of(b)), np_of(rs).reshape(-1), np_of(ws).reshape(-1), 'f16')
        want = o.gated_residual_add(np_of(res), branch, np_of(gate), np_of(labels))
        assert_bits_equal(np_of(got), want, f'split-K gated residual, call {call}')


def test_gemm_unaligned_output_rows(gpu):
    # ldc * 2 bytes not a multiple of 16: every tile takes the element-wise
    # store path of the staged epilogue.
    g = torch.Generator().manual_seed(3)
    m, n, k = 600, 517, 192
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.05 + 1e-4
    ws = torch.rand((n, 1), generator=g) * 1e-3 + 1e-6
    res = randn16(g, (m, n), 0.25)
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       out_dtype=torch.float16, residual=res.to(gpu))
    want = o.residual_add(np_of(res), o.dequantize_row(o.int_mm(np_of(a), np_of(b)), np_of(rs).reshape(-1),
                                                       np_of(ws).reshape(-1), 'f16'))
    assert_bits_equal(np_of(got), want, 'unaligned rows')


ADVERSARIAL = ('random', 'zero', 'bounds', 'cancellation', 'ties_outliers')


@pytest.mark.parametrize('pattern', ADVERSARIAL)
@pytest.mark.parametrize('epi', ['row', 'column'])
def test_dequantize_adversarial_int32(gpu, pattern, epi):
    # Patterns of benchmarks/test_tp2_p2_epilogue.py:18-25 (INT32 values near
    # and beyond 2^24, exact bounds, cancellations, ties).
    g = torch.Generator().manual_seed(744)
    rows, width, k = 17, 256, 7168
    acc = torch.randint(-10000000, 10000000, (rows, width), generator=g, dtype=torch.int32)
    if pattern == 'zero':
        acc.zero_()
    if pattern == 'bounds':
        acc.fill_(k * 128 * 128)
    if pattern == 'cancellation':
        acc = -acc + 17
    if pattern == 'ties_outliers':
        acc.zero_()
        acc[:, 0] = 16777217
        acc[:, 1] = -8388609
        acc[:, 2:10] = torch.tensor([1, -1, 3, -3, 127, -127, 65535, -65535], dtype=torch.int32)
    a = torch.rand((rows, 1), generator=g) * 0.1
    w = torch.rand((width,), generator=g) * 0.001
    code = kernels.EPI_ROW if epi == 'row' else kernels.EPI_COLUMN
    fn = o.dequantize_row if epi == 'row' else o.dequantize_column
    for out_dtype in (torch.float32, torch.float16):
        got = kernels.dequantize(acc.to(gpu), a.to(gpu), w.to(gpu), epilogue=code, out_dtype=out_dtype)
        want = fn(np_of(acc), np_of(a), np_of(w), tname(out_dtype))
        assert_bits_equal(np_of(got), want, f'{pattern} {epi} {out_dtype}')


# ------------------------------------------------------------------ quantize
QUANT_CASES = [
    (1, 16, False), (7, 3072, False), (33, 4096, False), (5, 5120, False), (9, 8192, False),
    (3, 16384, False), (2, 2064, False),
    (1, 256, True), (7, 3072, True), (33, 4096, True), (4, 8192, True), (3, 12800, True), (2, 16384, True),
    # 1024..2047 rows: a 4-wave workgroup per row
    (1100, 512, False), (1030, 3072, True), (1024, 9216, False), (1050, 12800, True),
    # one wavefront per row: 2048 rows or more up to 4096 columns, 8192 rows or more past that (registers),
    # and rows wider than 16384 columns (the streaming path, each row read twice)
    (2100, 512, False), (2050, 3072, True), (8200, 4352, False), (2100, 16400, False),
]


@pytest.mark.parametrize('rows,cols,rot', QUANT_CASES)
@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32])
def test_quantize_rows(gpu, rows, cols, rot, dtype):
    g = torch.Generator().manual_seed(rows * 31 + cols)
    x = randn16(g, (rows, cols), 3.0, dtype)
    if cols >= 64:
        x[:, 5] *= 20
    x[0, -1] = 0
    if rows > 2:
        x[2] = 0          # zero row: scale floor
    got_q, got_s = kernels.quantize_rows(x.to(gpu), convrot=rot, round_rotated=True)
    want_q, want_s = o.prepare_activation(np_of(x), convrot=rot, x_dtype=tname(dtype))
    assert_bits_equal(np_of(got_s).reshape(-1), want_s, f'scale {rows}x{cols} rot={rot} {dtype}')
    assert_bits_equal(np_of(got_q), want_q, f'codes {rows}x{cols} rot={rot} {dtype}')


@pytest.mark.parametrize('dtype', [torch.float16, torch.float32])
def test_quantize_fp32_rotation_and_external_max(gpu, dtype):
    g = torch.Generator().manual_seed(21)
    x = randn16(g, (19, 3072), 2.0, dtype)
    q, s = kernels.quantize_rows(x.to(gpu), convrot=True, round_rotated=False)
    rot = o.convrot256(np_of(x).astype(np.float32))
    wq, ws = o.quantize_rows(rot)
    assert_bits_equal(np_of(s).reshape(-1), ws, 'fp32-rotation scale')
    assert_bits_equal(np_of(q), wq, 'fp32-rotation codes')
    ext = torch.rand((19,), generator=g) * 4 + 0.5
    q, s = kernels.quantize_rows(x.to(gpu), row_max=ext.to(gpu))
    wq, ws = o.quantize_rows(np_of(x).astype(np.float32), row_max=np_of(ext))
    assert_bits_equal(np_of(s).reshape(-1), ws, 'external-max scale')
    assert_bits_equal(np_of(q), wq, 'external-max codes (saturating)')


def test_quantize_ties_and_strided_rows(gpu):
    # Rows whose quotients land exactly on half-integers exercise the exact
    # division path of the reciprocal quantizer.
    x = torch.zeros((4, 64), dtype=torch.float32)
    x[:, 0] = 254.0                      # scale exactly 2.0
    x[:, 1:33] = 2 * torch.arange(-16, 16, dtype=torch.float32) + 1   # x / 2 = k + 0.5
    x[1, 1:40] = torch.arange(1, 40, dtype=torch.float32) * 1.0
    x[2] = torch.linspace(-254, 254, 64)
    big = torch.zeros((4, 96), dtype=torch.float32)
    big[:, :64] = x
    q, s = kernels.quantize_rows(big.to(gpu)[:, :64])
    wq, ws = o.quantize_rows(np_of(x))
    assert_bits_equal(np_of(s).reshape(-1), ws, 'tie scales')
    assert_bits_equal(np_of(q), wq, 'tie codes')


# ------------------------------------------------------------------ FC2 prologue
SWIGLU_CASES = [(1, 256), (3, 512), (64, 3072), (5, 8192), (2, 12800), (2, 20480), (130, 4096),
                # more rows than CUs: 1 wave per row (2048, 3072), 2 (4096, 6144), 4 (8192),
                # 8 (12800, 20480) and, past 96 groups, 16 (24832)
                (300, 2048), (270, 3072), (300, 4096), (300, 6144), (280, 8192), (300, 12800), (260, 20480),
                (260, 24832)]


@pytest.mark.parametrize('rows,width', SWIGLU_CASES)
def test_swiglu_quantize(gpu, rows, width):
    g = torch.Generator().manual_seed(rows + width)
    x = randn16(g, (rows, 2 * width), 3.0)
    x[0, 0] = 60000.0        # huge gate: exp underflow branch
    x[0, 1] = -60000.0       # huge negative gate: exp overflow branch
    res = kernels.swiglu_quantize(x.to(gpu), want_row_max=True, want_group_max=True)
    wq, ws, wg = o.fc2_prologue(np_of(x))
    assert_bits_equal(np_of(res['group_max']), wg, f'group max {rows}x{width}')
    assert_bits_equal(np_of(res['row_max']).reshape(-1), wg.max(-1), 'row max')
    assert_bits_equal(np_of(res['scale']).reshape(-1), ws, 'scale')
    assert_bits_equal(np_of(res['q']), wq, f'codes {rows}x{width}')


@pytest.mark.parametrize('rows,width,ld', [(300, 2048, 4608), (300, 4096, 16384), (7, 8192, 16896)])
def test_swiglu_quantize_row_stride(gpu, rows, width, ld):
    """Rows read from a wider buffer (row stride ld > 2W), as the FFN
    prologue reads a column slice of a larger FC1 output."""
    g = torch.Generator().manual_seed(rows * 3 + width)
    big = randn16(g, (rows, ld), 2.0)
    res = kernels.swiglu_quantize(big.to(gpu)[:, 256:256 + 2 * width], want_group_max=True)
    wq, ws, wg = o.fc2_prologue(np_of(big[:, 256:256 + 2 * width].contiguous()))
    assert_bits_equal(np_of(res['group_max']), wg, f'group max {rows}x{width} ld {ld}')
    assert_bits_equal(np_of(res['scale']).reshape(-1), ws, 'scale')
    assert_bits_equal(np_of(res['q']), wq, f'codes {rows}x{width} ld {ld}')


def test_swiglu_external_max_fp32_input_and_phases(gpu):
    g = torch.Generator().manual_seed(77)
    x = randn16(g, (9, 2 * 1024), 2.0, torch.float32)
    ext = torch.rand((9, 1), generator=g) * 3 + 1
    res = kernels.swiglu_quantize(x.to(gpu), row_max=ext.to(gpu))
    wq, ws, _ = o.fc2_prologue(np_of(x), x_dtype='f32', row_max=np_of(ext))
    assert_bits_equal(np_of(res['scale']).reshape(-1), ws, 'external scale')
    assert_bits_equal(np_of(res['q']), wq, 'external codes')
    only = kernels.swiglu_quantize(x.to(gpu), quantize=False, want_row_max=True)
    assert set(only) == {'row_max'}
    assert_bits_equal(np_of(only['row_max']).reshape(-1), o.fc2_prologue(np_of(x), x_dtype='f32')[2].max(-1),
                      'maximum phase')


def test_swiglu_every_finite_fp16_gate(gpu):
    """One row per finite fp16 gate value (W = 256, up = 1). With a single
    nonzero gate every rotated element is +-a / 16 for a = g / (1 + exp(-g)),
    so the group maximum is |a| / 16 exactly: every gate's activation, from
    the reciprocal division or the IEEE one, is compared bit for bit."""
    bits = np.arange(65536, dtype=np.uint32)
    finite = bits[(bits & 0x7C00) != 0x7C00].astype(np.uint16)
    print(f'swiglu: {finite.size} finite fp16 gates', flush=True)
    x = torch.zeros((finite.size, 512), dtype=torch.float16)
    x[:, 256:] = 1.0
    x[:, 0] = torch.from_numpy(finite.view(np.float16))
    res = kernels.swiglu_quantize(x.to(gpu), want_row_max=True, want_group_max=True)
    gates = finite.view(np.float16).astype(np.float32)
    want = (np.abs(o.swiglu_f32(gates, np.ones_like(gates))) * np.float32(1.0 / 16.0)).astype(np.float32)
    assert_bits_equal(np_of(res['group_max'])[:, 0], want, 'group max = |silu(g)| / 16, every finite gate')
    idx = np.arange(0, finite.size, 97)
    wq, ws, wg = o.fc2_prologue(np_of(x)[idx])
    assert_bits_equal(np_of(res['q'])[idx], wq, 'codes of sampled gate rows')
    assert_bits_equal(np_of(res['scale']).reshape(-1)[idx], ws, 'scales of sampled gate rows')


def test_swiglu_infinite_gate(gpu):
    # A +inf gate is outside the reciprocal division's range: inf / (1 + 0)
    # is inf, and the group maximum with it.
    x = torch.zeros((2, 512), dtype=torch.float16)
    x[:, 256:] = 1.0
    x[0, 3] = float('inf')
    x[1, 3] = 60000.0
    res = kernels.swiglu_quantize(x.to(gpu), want_group_max=True)
    xs = np_of(x).astype(np.float32)
    with np.errstate(invalid='ignore'):
        rot = o.convrot256(o.swiglu_f32(xs[:, :256], xs[:, 256:]))
    assert_bits_equal(np_of(res['group_max']), np.abs(rot).max(-1, keepdims=True), 'group max with an infinite gate')
    assert np.isinf(np_of(res['group_max'])[0, 0])


# ------------------------------------------------------------------ DiT gated residual update
GATE_CASES = [
    # (m, n, k): persistent tiles with ragged edges, the skinny path, split K
    (600, 520, 512), (4400, 3072, 256), (48, 1000, 1024), (300, 520, 2048),
]


@pytest.mark.parametrize('m,n,k', GATE_CASES)
@pytest.mark.parametrize('label_kind', ['random', 'segments'])
def test_gemm_gated_residual(gpu, m, n, k, label_kind):
    g = torch.Generator().manual_seed(m + 3 * n + k)
    a = randi8(g, (m, k))
    b = randi8(g, (n, k))
    rs = torch.rand((m, 1), generator=g) * 0.01 + 1e-4
    ws = (torch.rand((n, 1), generator=g) * 1e-3 + 1e-6) / 512
    res = randn16(g, (m, n), 1 / 512)
    gate = torch.randn((9, n), generator=g)
    if label_kind == 'random':
        # Every epilogue pass mixes labels: each row reads its own table row.
        labels = torch.randint(0, 9, (m,), generator=g, dtype=torch.int32)
    else:
        # DiT frames: long runs of one label, so most 32-row passes read one
        # table row, and the boundaries (not multiples of 32) fall inside passes.
        bounds = [0] + sorted(torch.randperm(m - 1, generator=g)[:4].add(1).tolist()) + [m]
        labels = torch.cat([torch.full((bounds[i + 1] - bounds[i],), i % 9, dtype=torch.int32)
                            for i in range(len(bounds) - 1)])
    got = kernels.gemm(a.to(gpu), b.to(gpu), epilogue=kernels.EPI_ROW, row_scale=rs.to(gpu), col_scale=ws.to(gpu),
                       out_dtype=torch.float16, residual=res.to(gpu), gate=gate.to(gpu), gate_labels=labels.to(gpu))
    branch = o.dequantize_row(o.int_mm(np_of(a), np_of(b)), np_of(rs).reshape(-1), np_of(ws).reshape(-1), 'f16')
    want = o.gated_residual_add(np_of(res), branch, np_of(gate), np_of(labels))
    assert_bits_equal(np_of(got), want, f'gated residual {m}x{n}x{k}')


def test_dequantize_gated_residual(gpu):
    g = torch.Generator().manual_seed(17)
    rows, width = 37, 300
    acc = torch.randint(-3000000, 3000000, (rows, width), generator=g, dtype=torch.int32)
    a = torch.rand((rows, 1), generator=g) * 1e-3
    w = torch.rand((width,), generator=g) * 1e-3
    res = randn16(g, (rows, width))
    gate = torch.randn((3, width), generator=g)
    labels = torch.randint(0, 3, (rows,), generator=g, dtype=torch.int32)
    got = kernels.dequantize(acc.to(gpu), a.to(gpu), w.to(gpu), epilogue=kernels.EPI_ROW, residual=res.to(gpu),
                             gate=gate.to(gpu), gate_labels=labels.to(gpu))
    want = o.gated_residual_add(np_of(res), o.dequantize_row(np_of(acc), np_of(a), np_of(w), 'f16'), np_of(gate),
                                np_of(labels))
    assert_bits_equal(np_of(got), want, 'dequantize gated')
