"""Shared helpers of the GPU parity tests: torch <-> numpy in the oracle's conventions."""
import numpy as np
import torch


def np_of(t):
    """CPU numpy view of a tensor; bf16 as uint16 bit patterns (the oracle's form)."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def tname(dtype):
    return {torch.float16: 'f16', torch.bfloat16: 'bf16', torch.float32: 'f32'}[dtype]


def assert_bits_equal(got, want, what=''):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.dtype.kind == 'f':
        gb = got.view(np.uint16 if got.dtype.itemsize == 2 else np.uint32)
        wb = want.astype(got.dtype).view(gb.dtype)
        bad = gb != wb
        # NaN payloads aside, require identical bits (signed zeros included).
    else:
        bad = got != want
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f'{what}: {int(bad.sum())} of {bad.size} differ; first {idx.tolist()}: '
                             f'got {[got[tuple(i)] for i in idx]} want {[want[tuple(i)] for i in idx]}')


def randn16(gen, shape, scale=1.0, dtype=torch.float16):
    return (torch.randn(shape, generator=gen) * scale).to(dtype)


def randi8(gen, shape):
    return torch.randint(-128, 128, shape, generator=gen, dtype=torch.int8)
