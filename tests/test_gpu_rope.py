"""GPU parity of the packed-QKV RMS-RoPE kernel against the CPU oracle (bit-exact)."""
import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of, tname
from w8a8 import kernels, rms_rope

pytestmark = pytest.mark.gpu


def _freqs(g, rows, rot, dtype):
    ang = torch.rand((rows, rot // 2), generator=g, dtype=torch.float64) * 6.283185307179586
    c, s = torch.cos(ang), torch.sin(ang)
    f = torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2)
    return f.to(dtype)


CASES = [
    # rows, heads, rot_dim, in, freq, out
    (1, 2, 96, torch.float16, torch.float16, torch.float16),
    (37, 28, 96, torch.float16, torch.float16, torch.float16),     # the H3 DiT rank shape
    (13, 24, 96, torch.float16, torch.float32, torch.float32),
    (9, 4, 128, torch.float32, torch.float32, torch.float16),
    (5, 6, 2, torch.float16, torch.float16, torch.float32),
    (7, 3, 64, torch.float32, torch.float16, torch.float32),       # odd head count: a partial block
    (1030, 8, 96, torch.float16, torch.float16, torch.float16),
]


@pytest.mark.parametrize('rows,heads,rot,in_dt,fq_dt,out_dt', CASES)
def test_rms_rope_matches_oracle(gpu, rows, heads, rot, in_dt, fq_dt, out_dt):
    g = torch.Generator().manual_seed(rows * 131 + heads * 7 + rot)
    packed = (torch.randn((rows, 3 * heads * 128), generator=g) * 3).to(in_dt)
    packed[0, :128] = 0                      # an all-zero head: inv = 1/sqrt(eps)
    if rows > 1:
        packed[1, 128:256] = 30000.0 if in_dt == torch.float16 else 1e6
    f = _freqs(g, rows, rot, fq_dt)
    gq = torch.rand(128, generator=g) + 0.5
    gk = torch.rand(128, generator=g) + 0.5
    q, k = kernels.rms_rope(packed.to(gpu), f.to(gpu), gq.to(gpu), gk.to(gpu), heads=heads, rot_dim=rot, eps=1e-6,
                            out_dtype=out_dt)
    wq, wk = o.rms_rope(np_of(packed), np_of(f).astype(np.float32), np_of(gq), np_of(gk), heads, rot, eps=1e-6,
                        in_dtype=tname(in_dt), out_dtype=tname(out_dt))
    assert_bits_equal(np_of(q), wq, f'q {rows}x{heads} rot={rot}')
    assert_bits_equal(np_of(k), wk, f'k {rows}x{heads} rot={rot}')


def test_rms_rope_reference_api_and_strided_packed_row(gpu):
    g = torch.Generator().manual_seed(3)
    rows, heads, rot = 50, 28, 96
    big = (torch.randn((rows, 3 * heads * 128 + 64), generator=g)).half()
    packed = big[:, :3 * heads * 128]
    f = _freqs(g, rows, rot, torch.float16)
    gq = torch.rand(128, generator=g) + 0.5
    gk = torch.rand(128, generator=g) + 0.5
    freqs6 = f.reshape(1, rows, 1, rot // 2, 2, 2).to(gpu)
    q, k = rms_rope.execute(packed.contiguous().to(gpu), freqs6, gq.to(gpu), gk.to(gpu), heads=heads, epsilon=1e-6)
    q2, k2 = kernels.rms_rope(packed.to(gpu), f.to(gpu), gq.to(gpu), gk.to(gpu), heads=heads, rot_dim=rot, eps=1e-6)
    assert torch.equal(q, q2) and torch.equal(k, k2)
    wq, wk = o.rms_rope(np_of(packed), np_of(f).astype(np.float32), np_of(gq), np_of(gk), heads, rot, eps=1e-6)
    assert_bits_equal(np_of(q), wq, 'execute q')
    assert_bits_equal(np_of(k), wk, 'execute k')
    assert not rms_rope.supported(packed.to(gpu), freqs6, heads, 64)
    with pytest.raises(ValueError):
        rms_rope.execute(packed.contiguous().to(gpu), freqs6, gq.to(gpu), gk.to(gpu), heads=heads, dim=64)


def _qkv_case(g, gpu, m, n, k, freq_dtype, rot):
    x = (torch.randn((m, k), generator=g) * 2).half().to(gpu)
    w = torch.randn((n, k), generator=g) * 0.03
    wq, ws = kernels.quantize_rows(w.to(gpu))
    codes, a = kernels.quantize_rows(x, convrot=k % 256 == 0)
    f = _freqs(g, m, rot, freq_dtype).to(gpu)
    gq = (torch.rand(128, generator=g) + 0.5).to(gpu)
    gk = (torch.rand(128, generator=g) + 0.5).to(gpu)
    return x, codes, a, wq, ws, f, gq, gk


GEMM_ROPE_CASES = [
    # m, heads, extra V columns, k, rot_dim, freq dtype, epilogue
    (300, 2, 2 * 128, 256, 96, torch.float16, kernels.EPI_COLUMN),    # partial row tile
    (1030, 3, 3 * 128, 384, 96, torch.float32, kernels.EPI_ROW),      # a 256-column tile half past n
    (257, 4, 100, 128, 128, torch.float16, kernels.EPI_COLUMN),       # V ends inside a 16-byte chunk
    (512, 1, 0, 512, 64, torch.float16, kernels.EPI_COLUMN),          # no V columns
    (777, 28, 28 * 128, 1024, 96, torch.float16, kernels.EPI_COLUMN), # the H3 DiT rank layout
]


@pytest.mark.parametrize('m,heads,extra,k,rot,fq_dt,epi', GEMM_ROPE_CASES)
def test_gemm_rope_epilogue_equals_gemm_then_rms_rope(gpu, m, heads, extra, k, rot, fq_dt, epi):
    g = torch.Generator().manual_seed(m + 17 * heads + rot)
    n = 2 * heads * 128 + extra
    _, codes, a, wq, ws, f, gq, gk = _qkv_case(g, gpu, m, n, k, fq_dt, rot)
    codes[0].zero_()                                  # an all-zero row: inv = 1/sqrt(eps)
    ldc = (n + 7) // 8 * 8
    out = torch.full((m, ldc), float('nan'), dtype=torch.float16, device=gpu)[:, :n]
    rope = {'heads': heads, 'rot_dim': rot, 'freqs': f, 'q_gain': gq, 'k_gain': gk, 'eps': 1e-6}
    fused = kernels.gemm(codes, wq, epilogue=epi, row_scale=a, col_scale=ws, out=out, rope=rope)
    plain = kernels.gemm(codes, wq, epilogue=epi, row_scale=a, col_scale=ws, out_dtype=torch.float16)
    q, kk = kernels.rms_rope(plain, f, gq, gk, heads=heads, rot_dim=rot, eps=1e-6)
    width = heads * 128
    assert torch.equal(fused[:, :width].view(torch.int16), q.reshape(m, width).view(torch.int16))
    assert torch.equal(fused[:, width:2 * width].view(torch.int16), kk.reshape(m, width).view(torch.int16))
    assert torch.equal(fused[:, 2 * width:].view(torch.int16), plain[:, 2 * width:].view(torch.int16))


def test_gemm_rope_epilogue_matches_oracle(gpu):
    g = torch.Generator().manual_seed(11)
    m, heads, k, rot = 130, 2, 256, 96
    n = 3 * heads * 128
    x, codes, a, wq, ws, f, gq, gk = _qkv_case(g, gpu, m, n, k, torch.float16, rot)
    rope = {'heads': heads, 'rot_dim': rot, 'freqs': f, 'q_gain': gq, 'k_gain': gk, 'eps': 1e-6}
    fused = kernels.gemm(codes, wq, epilogue=kernels.EPI_COLUMN, row_scale=a, col_scale=ws, rope=rope)
    packed = o.column_linear(np_of(x), np_of(wq), np_of(ws).reshape(-1), convrot=True)
    wq_, wk_ = o.rms_rope(packed, np_of(f).astype(np.float32), np_of(gq), np_of(gk), heads, rot, eps=1e-6)
    width = heads * 128
    got = np_of(fused)
    assert_bits_equal(got[:, :width].reshape(m, heads, 128), wq_, 'fused q')
    assert_bits_equal(got[:, width:2 * width].reshape(m, heads, 128), wk_, 'fused k')
    assert_bits_equal(got[:, 2 * width:], packed[:, 2 * width:], 'fused v')


def test_fused_qkv_api_equals_projection_then_execute(gpu):
    from w8a8 import dit_column_linear
    g = torch.Generator().manual_seed(5)
    m, heads, k, rot = 333, 4, 512, 96
    n = 3 * heads * 128
    x, codes, a, wq, ws, f, gq, gk = _qkv_case(g, gpu, m, n, k, torch.float16, rot)
    freqs6 = f.reshape(1, m, 1, rot // 2, 2, 2)
    q, kk, v = rms_rope.fused_qkv(x, wq, ws, freqs6, gq, gk, heads=heads, epsilon=1e-6)
    qkv = dit_column_linear.column_linear(x, wq, ws)
    q2, k2 = rms_rope.execute(qkv, freqs6, gq, gk, heads=heads, epsilon=1e-6)
    assert torch.equal(q, q2) and torch.equal(kk, k2)
    assert torch.equal(v, qkv[:, 2 * heads * 128:].reshape(m, heads, 128))
    q3, k3, v3 = rms_rope.fused_qkv(None, wq, ws, freqs6, gq, gk, heads=heads, epsilon=1e-6, prepared=(codes, a))
    assert torch.equal(q3, q) and torch.equal(k3, kk) and torch.equal(v3, v)
    with pytest.raises(ValueError):
        rms_rope.fused_qkv(x, wq[:-128], ws[:-128], freqs6, gq, gk, heads=heads)


def test_gemm_rope_epilogue_full_dit_shape(gpu):
    """The benchmarked shape (53504 tokens, 3072 -> 3 x 24 heads): the fused
    output equals the GEMM + RMS-RoPE pair everywhere, and sampled rows equal
    the oracle (every scale and norm is per row)."""
    from w8a8 import workloads
    data = workloads.dit_qkv_rope()
    m, k = data['x'].shape
    heads, rot = data['heads'], data['rot_dim']
    wq, ws = workloads.quantize_weight(data['w'], gpu)
    x = data['x'].to(gpu)
    f, gq, gk = (data[t].to(gpu) for t in ('freqs', 'q_gain', 'k_gain'))
    codes, a = kernels.quantize_rows(x, convrot=True)
    rope = {'heads': heads, 'rot_dim': rot, 'freqs': f, 'q_gain': gq, 'k_gain': gk, 'eps': 1e-6}
    fused = kernels.gemm(codes, wq, epilogue=kernels.EPI_COLUMN, row_scale=a, col_scale=ws, rope=rope)
    plain = kernels.gemm(codes, wq, epilogue=kernels.EPI_COLUMN, row_scale=a, col_scale=ws)
    q, kk = kernels.rms_rope(plain, f, gq, gk, heads=heads, rot_dim=rot, eps=1e-6)
    width = heads * 128
    assert torch.equal(fused[:, :width].view(torch.int16), q.reshape(m, width).view(torch.int16))
    assert torch.equal(fused[:, width:2 * width].view(torch.int16), kk.reshape(m, width).view(torch.int16))
    assert torch.equal(fused[:, 2 * width:].view(torch.int16), plain[:, 2 * width:].view(torch.int16))
    del plain, q, kk
    rows = torch.tensor([0, 1, 255, 256, 30001, m - 1])
    packed = o.column_linear(np_of(data['x'][rows]), np_of(wq), np_of(ws).reshape(-1), convrot=True)
    wq_, wk_ = o.rms_rope(packed, np_of(data['freqs'][rows]).astype(np.float32), np_of(data['q_gain']),
                          np_of(data['k_gain']), heads, rot, eps=1e-6)
    got = np_of(fused[rows.to(gpu)])
    assert_bits_equal(got[:, :width].reshape(-1, heads, 128), wq_, 'full-shape q rows')
    assert_bits_equal(got[:, width:2 * width].reshape(-1, heads, 128), wk_, 'full-shape k rows')
    assert_bits_equal(got[:, 2 * width:], packed[:, 2 * width:], 'full-shape v rows')


@pytest.mark.parametrize('fq_dt', [torch.float16, torch.float32])
def test_gemm_rope_paired_frequency_layout(gpu, fq_dt):
    g = torch.Generator().manual_seed(23)
    m, heads, k, rot = 301, 3, 256, 96
    n = 3 * heads * 128
    x, codes, a, wq, ws, f, gq, gk = _qkv_case(g, gpu, m, n, k, fq_dt, rot)
    rope = {'heads': heads, 'rot_dim': rot, 'freqs': f, 'q_gain': gq, 'k_gain': gk, 'eps': 1e-6}
    plain = kernels.gemm(codes, wq, epilogue=kernels.EPI_COLUMN, row_scale=a, col_scale=ws, rope=rope)
    packed = rms_rope.pack_freqs(f)
    assert packed.shape == (m, 2, rot // 2, 2)
    fr = f.reshape(m, rot // 2, 2, 2)
    assert torch.equal(packed[:, 1, :, 0], fr[:, :, 1, 1]) and torch.equal(packed[:, 1, :, 1], fr[:, :, 1, 0])
    paired = kernels.gemm(codes, wq, epilogue=kernels.EPI_COLUMN, row_scale=a, col_scale=ws,
                          rope=dict(rope, freqs=packed, pairs=True))
    assert torch.equal(paired.view(torch.int16), plain.view(torch.int16))
    freqs6 = f.reshape(1, m, 1, rot // 2, 2, 2)
    q1, k1, v1 = rms_rope.fused_qkv(x, wq, ws, freqs6, gq, gk, heads=heads)
    q2, k2, v2 = rms_rope.fused_qkv(x, wq, ws, freqs6, gq, gk, heads=heads, freqs_pairs=packed)
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)
