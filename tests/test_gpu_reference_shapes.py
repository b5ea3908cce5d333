"""The reference's own published operator shapes (one TP2 rank of
MiniMax-H3: DiT S=6814, hidden 5376; text encoder S=353, hidden 5120)
through the API, against the oracle on sampled rows (every scale is per row,
so a row's output depends on that row alone)."""
import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of
from w8a8 import workloads
from w8a8.dit_column_linear import column_linear
from w8a8.tp_dit import RowParallelLinearINT8

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('name', sorted(workloads.REFERENCE_SHAPES))
def test_reference_shape_against_oracle(gpu, name):
    role, m, n, k = workloads.REFERENCE_SHAPES[name][:4]
    print(f'reference shape {name}: {role} M={m} N={n} K={k}', flush=True)
    data = workloads.reference_shape(name)
    wq, ws = workloads.quantize_weight(data['w'], gpu)
    x = data['x'].to(gpu)
    rows = np.unique(np.array([0, 1, 31, 32, m // 2, m - 2, m - 1]))
    sel = torch.from_numpy(rows).to(gpu)
    xs = np_of(data['x'])[rows]
    wn, wsn = np_of(wq), np_of(ws).reshape(-1)
    if role == 'column':
        y = column_linear(x, wq, ws)
        assert y.shape == (m, n) and y.dtype == torch.float16
        want = o.column_linear(xs, wn, wsn)
    else:
        shard = RowParallelLinearINT8(2 * k, n, world_size=2, device=gpu)
        shard.weight.data.copy_(wq)
        shard.weight_scale.data.copy_(ws)
        y = shard(x, input_act='swiglu' if role == 'fc2' else None)
        assert y.shape == (m, n) and y.dtype == torch.float32
        acc, a = o.row_partial(xs, wn, swiglu=role == 'fc2')
        want = o.dequantize_row(acc, a, wsn, 'f32')
    assert_bits_equal(np_of(y[sel]), want, f'{name} sampled rows')
    assert torch.isfinite(y).all()
