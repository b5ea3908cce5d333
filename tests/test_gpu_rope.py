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
