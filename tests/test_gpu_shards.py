"""One tensor-parallel rank's half of a DiT block on one GPU.

A block loaded with world_size 2 runs each rank's shard at its real shape:
column shards are complete; row shards stop where the reference exchanges
data (the MAX of the row maxima, the SUM of the int32 partials). Both ranks
run here one after the other, so the exchanges can be done by hand and
checked: with the global maximum the two int32 partials add up exactly to
the unsharded accumulator, and each rank's FP32 partial matches the oracle.
The half-shard workload (M = 204336 in 16384-row chunks, QKV 3072 -> 4608,
FC1 3072 -> 2 x 4096, FC2 4096 -> 3072 with an FP32 partial) is checked on
sampled rows against the oracle and chunked against whole.
"""
import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of, randn16
from w8a8 import checkpoint as ck
from w8a8 import kernels, workloads
from w8a8.tp_dit import ColumnParallelLinearINT8, DiTFeedForwardINT8, RowParallelLinearINT8, chunked_rows

pytestmark = pytest.mark.gpu


def _block_file(tmp_path, hidden=512, ffn=1024, seed=31):
    g = torch.Generator().manual_seed(seed)

    def q(n, k):
        w = torch.randn((n, k), generator=g) * 0.02
        return o.quantize_weight(w.numpy())

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a))
    weights = {}
    for name, (n, k) in {'qkv_proj': (3 * hidden, hidden), 'out_proj': (hidden, hidden), 'fc1': (2 * ffn, hidden),
                         'fc2': (hidden, ffn)}.items():
        wq, ws = q(n, k)
        weights[name] = (t(wq), t(ws).reshape(-1, 1))
    rep = {'norm1.weight': torch.rand(hidden, generator=g), 'norm2.weight': torch.rand(hidden, generator=g),
           'q_norm.weight': torch.rand(128, generator=g), 'k_norm.weight': torch.rand(128, generator=g),
           'adaln_proj.weight': torch.randn((18 * hidden, 8), generator=g),
           'adaln_proj.bias': torch.randn(18 * hidden, generator=g)}
    return ck.save_block(tmp_path / 'block.safetensors', 'dit', 5, weights, rep), weights


def test_rank_halves_of_the_ffn_sum_to_the_whole(gpu, tmp_path):
    path, weights = _block_file(tmp_path)
    whole = ck.load_block(path, 'dit', 5, device=gpu)
    halves = [ck.load_block(path, 'dit', 5, rank=r, world_size=2, device=gpu) for r in (0, 1)]
    print('rank halves: FFN 300 x 512 -> 2 x 1024 -> 512', flush=True)
    g = torch.Generator().manual_seed(32)
    h = randn16(g, (300, 512), 1.0)
    h[7] = 0
    hd = h.to(gpu)
    y = whole.fc1(hd)
    ys = [b.fc1(hd) for b in halves]
    f = 1024
    for r in (0, 1):   # a rank's FC1 columns are its gate half then its up half
        want = torch.cat([y[:, r * f // 2:(r + 1) * f // 2], y[:, f + r * f // 2:f + (r + 1) * f // 2]], 1)
        assert torch.equal(ys[r], want)
    full = kernels.swiglu_quantize(y, want_row_max=True)
    acc = kernels.gemm(full['q'], whole.fc2.weight)
    maxima = [b.fc2.local_maximum(yr, 'swiglu') for b, yr in zip(halves, ys)]
    gmax = torch.maximum(maxima[0], maxima[1])
    assert torch.equal(gmax, full['row_max'])
    parts = [b.fc2.partial(yr, 'swiglu', row_max=gmax, accumulate=torch.int32) for b, yr in zip(halves, ys)]
    assert torch.equal(parts[0][0] + parts[1][0], acc)
    assert torch.equal(parts[0][1], full['scale']) and torch.equal(parts[1][1], full['scale'])
    w2 = np_of(weights['fc2'][0])
    ws2 = np_of(weights['fc2'][1]).reshape(-1)
    for r, b in enumerate(halves):
        p = b.fc2(ys[r], input_act='swiglu', row_max=gmax)     # forward of a row shard: the FP32 partial
        assert p.dtype == torch.float32 and p.shape == (300, 512)
        oacc, oa = o.row_partial(np_of(ys[r]), w2[:, r * f // 2:(r + 1) * f // 2], row_max=np_of(gmax), swiglu=True)
        assert_bits_equal(np_of(parts[r][0]), oacc, f'rank {r} int32 partial')
        assert_bits_equal(np_of(p), o.dequantize_row(oacc, oa, ws2, 'f32'), f'rank {r} fp32 partial')
        ffn = DiTFeedForwardINT8.from_projections(b.fc1, b.fc2)
        assert torch.equal(ffn.forward_partial(hd, row_max=gmax), p)
    # without the exchanged maximum a rank quantizes with its own: another operator
    own = halves[0].fc2.partial(ys[0], 'swiglu', accumulate=torch.int32)
    assert not torch.equal(own[1], full['scale'])
    with pytest.raises(ValueError, match='SUM exchange'):
        halves[0].fc2(ys[0], input_act='swiglu', residual=torch.zeros(300, 512, dtype=torch.float16, device=gpu))
    with pytest.raises(ValueError, match='requires reduction'):
        halves[0].fc2(ys[0], reduce_sum=False, input_act='swiglu')


def test_rank_halves_of_the_o_projection_and_qkv(gpu, tmp_path):
    path, weights = _block_file(tmp_path, seed=33)
    whole = ck.load_block(path, 'dit', 5, device=gpu)
    halves = [ck.load_block(path, 'dit', 5, rank=r, world_size=2, device=gpu) for r in (0, 1)]
    print('rank halves: O projection 129 x 512 -> 512, QKV 512 -> 3 x 512', flush=True)
    g = torch.Generator().manual_seed(34)
    x = randn16(g, (129, 512), 0.7)
    xd = x.to(gpu)
    qkv = whole.qkv_proj(xd)
    for r, b in enumerate(halves):   # component-wise column shards: q, k and v halves
        part = b.qkv_proj(xd)
        want = torch.cat([qkv[:, c * 512 + r * 256:c * 512 + (r + 1) * 256] for c in range(3)], 1)
        assert torch.equal(part, want)
    xs = [xd[:, :256], xd[:, 256:]]
    gmax = torch.maximum(*[b.out_proj.local_maximum(xr) for b, xr in zip(halves, xs)])
    qw, aw = kernels.quantize_rows(xd, convrot=True, round_rotated=False)
    assert torch.equal(gmax.reshape(-1), kernels.row_absmax(xd, convrot=True, round_rotated=False).reshape(-1))
    acc = kernels.gemm(qw, whole.out_proj.weight)
    parts = [b.out_proj.partial(xr, row_max=gmax, accumulate=torch.int32) for b, xr in zip(halves, xs)]
    assert torch.equal(parts[0][0] + parts[1][0], acc) and torch.equal(parts[1][1], aw)
    wo = np_of(weights['out_proj'][0])
    wso = np_of(weights['out_proj'][1]).reshape(-1)
    for r, b in enumerate(halves):
        p = b.out_proj(xs[r], row_max=gmax)
        oacc, oa = o.row_partial(np_of(xs[r].contiguous()), wo[:, r * 256:(r + 1) * 256], row_max=np_of(gmax))
        assert_bits_equal(np_of(p), o.dequantize_row(oacc, oa, wso, 'f32'), f'O rank {r} fp32 partial')
    assert_bits_equal(np_of(gmax).reshape(-1), o.rank_row_max(np_of(x)), 'O global row max')


def _half_shard_modules(data, gpu):
    qkv = ColumnParallelLinearINT8(3072, 2 * 4608, rank=0, world_size=2, components=3, device=gpu)
    fc1 = ColumnParallelLinearINT8(3072, 2 * 8192, rank=0, world_size=2, components=2, device=gpu)
    fc2 = RowParallelLinearINT8(2 * 4096, 3072, rank=0, world_size=2, device=gpu)
    for m, w in ((qkv, data['w_qkv']), (fc1, data['w1']), (fc2, data['w2'])):
        q, s = workloads.quantize_weight(w, gpu)
        m.weight.data.copy_(q)
        m.weight_scale.data.copy_(s)
    return qkv, fc1, fc2


def test_half_shard_workload_chunks_against_oracle_and_whole(gpu):
    """The half-shard workload: 12 chunks of 16384 rows and a 7728-row tail."""
    data = workloads.dit_half_shard()
    m = data['h'].shape[0]
    assert m == 12 * 16384 + 7728
    qkv, fc1, fc2 = _half_shard_modules(data, gpu)
    assert qkv.weight.shape == (4608, 3072) and fc1.weight.shape == (8192, 3072) and fc2.weight.shape == (3072, 4096)
    h = data['h'].to(gpu)
    print('half shard: M=204336 QKV / FC1 / FC2 fp32 partial, chunked and whole', flush=True)
    rows = np.array([0, 1, 16383, 16384, 99999, 196607, 196608, 196609, 200000, m - 2, m - 1])
    hn = np_of(data['h'])[rows]
    sel = torch.from_numpy(rows).to(gpu)
    qkv_whole = qkv(h)
    assert torch.equal(chunked_rows(qkv, h, chunk_rows=16384), qkv_whole)
    want = o.column_linear(hn, np_of(qkv.weight), np_of(qkv.weight_scale).reshape(-1))
    assert_bits_equal(np_of(qkv_whole[sel]), want, 'half-shard QKV rows')
    del qkv_whole
    y = fc1(h)
    assert torch.equal(chunked_rows(fc1, h, chunk_rows=16384), y)
    want = o.column_linear(hn, np_of(fc1.weight), np_of(fc1.weight_scale).reshape(-1))
    assert_bits_equal(np_of(y[sel]), want, 'half-shard FC1 rows')
    part = torch.full((m, 3072), float('nan'), device=gpu)
    for start in range(0, m, 16384):
        stop = min(start + 16384, m)
        fc2(y[start:stop], input_act='swiglu', out=part[start:stop])
    whole = fc2(y, input_act='swiglu')
    assert torch.equal(part, whole)
    oacc, oa = o.row_partial(np_of(y[sel]), np_of(fc2.weight), swiglu=True)
    assert_bits_equal(np_of(whole[sel]), o.dequantize_row(oacc, oa, np_of(fc2.weight_scale).reshape(-1), 'f32'),
                      'half-shard FC2 fp32 partial rows')
    tail = y[196608:]
    assert tail.shape[0] == 7728
    assert torch.equal(fc2(tail, input_act='swiglu'), whole[196608:])
