"""The no-allocation GEMM entry point (w8a8_gemm_noalloc) through the C ABI.

Its split-K partials live in the library's file-scope device scratch array
instead of a caller workspace. Two calls in a row (the second smaller, so
stale partials of the first remain in the array) must equal w8a8_gemm with a torch-allocated workspace bit for
bit, and the oracle. A shape whose split would need more scratch than the
array holds runs unsplit, with the same result; a caller workspace is
refused. A split call captured in a HIP graph replays bit-identically, with
other calls reusing the scratch between the replays.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as o
from helpers import assert_bits_equal, np_of, randi8
from w8a8 import _abi, kernels

pytestmark = pytest.mark.gpu


def _args(q, w, out, epilogue, row_scale=None, col_scale=None, workspace=None, workspace_bytes=0):
    dtype = _abi.DTYPE_CODE[out.dtype]
    return _abi.GemmArgs(struct_size=ctypes.sizeof(_abi.GemmArgs), epilogue=epilogue, a=q.data_ptr(),
                         lda=q.stride(0), b=w.data_ptr(), ldb=w.stride(0), m=q.shape[0], n=w.shape[0], k=q.shape[1],
                         row_scale=_abi.ptr(row_scale), col_scale=_abi.ptr(col_scale),
                         col_scale_stride=1 if col_scale is not None else 0, out_dtype=dtype, out=out.data_ptr(),
                         ldc=out.stride(0), workspace=workspace, workspace_bytes=workspace_bytes,
                         stream=_abi.stream_of(q))


def _noalloc(args):
    lib = _abi.load()
    rc = lib.w8a8_gemm_noalloc(ctypes.byref(args))
    return rc, lib.w8a8_last_error().decode()


@pytest.mark.parametrize('call', [0, 1])
def test_noalloc_gemm_equals_gemm_on_two_calls(gpu, call):
    del call   # the whole sequence runs twice: the second time the array holds the last shape's partials
    # persistent tiles with split K, then the weight-streaming kernel's split
    for m, n, k in ((512, 4096, 14336), (200, 1000, 4096), (64, 4096, 14336), (24, 1000, 4096)):
        print(f'noalloc gemm {m}x{n}x{k}', flush=True)
        need = kernels.gemm_workspace_bytes(m, n, k, gpu)
        assert 0 < need <= _abi.GEMM_SCRATCH_BYTES      # the shape splits K and fits the scratch
        g = torch.Generator().manual_seed(m + n + k)
        q = randi8(g, (m, k)).to(gpu)
        w = randi8(g, (n, k)).to(gpu)
        a = (torch.rand((m, 1), generator=g) * 1e-2).to(gpu)
        s = (torch.rand((n, 1), generator=g) * 1e-3).to(gpu)
        ref = kernels.gemm(q, w)                           # w8a8_gemm with a torch workspace
        got = torch.full((m, n), -7, dtype=torch.int32, device=gpu)
        rc, msg = _noalloc(_args(q, w, got, _abi.EPI_INT32))
        assert rc == _abi.OK, msg
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        assert_bits_equal(np_of(got), o.int_mm(np_of(q), np_of(w)), f'noalloc int32 {m}x{n}x{k}')
        ref16 = kernels.gemm(q, w, epilogue=kernels.EPI_ROW, row_scale=a, col_scale=s, out_dtype=torch.float16)
        got16 = torch.full((m, n), float('nan'), dtype=torch.float16, device=gpu)
        rc, msg = _noalloc(_args(q, w, got16, _abi.EPI_ROW, a.reshape(-1), s.reshape(-1)))
        assert rc == _abi.OK, msg
        torch.cuda.synchronize()
        assert torch.equal(got16.view(torch.int16), ref16.view(torch.int16))


def test_noalloc_gemm_runs_unsplit_what_it_cannot_hold(gpu):
    m, n, k = 768, 12288, 65536      # 256 x 192 tiles, K split four ways: 144 MB of partials
    need = kernels.gemm_workspace_bytes(m, n, k, gpu)
    assert need > _abi.GEMM_SCRATCH_BYTES
    gg = torch.Generator(device=gpu).manual_seed(9)
    q = torch.randint(-128, 128, (m, k), dtype=torch.int8, device=gpu, generator=gg)
    w = torch.randint(-128, 128, (n, k), dtype=torch.int8, device=gpu, generator=gg)
    ref = kernels.gemm(q, w)                               # split K in a torch workspace
    out = torch.full((m, n), 5, dtype=torch.int32, device=gpu)
    rc, msg = _noalloc(_args(q, w, out, _abi.EPI_INT32))
    assert rc == _abi.OK, msg
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    ws = torch.empty(1024, dtype=torch.uint8, device=gpu)
    small = torch.full((200, 1000), 5, dtype=torch.int32, device=gpu)
    rc, msg = _noalloc(_args(q[:200, :4096], w[:1000, :4096], small, _abi.EPI_INT32, workspace=ws.data_ptr(),
                             workspace_bytes=1024))
    assert rc == _abi.ERR_INVALID and 'replaces the workspace' in msg
    torch.cuda.synchronize()
    assert bool((small == 5).all())                        # nothing was launched


def test_noalloc_split_gemm_replays_in_a_graph(gpu):
    m, n, k = 512, 4096, 14336       # 128 x 256 tiles, K split four ways, partials added by a second kernel
    assert 0 < kernels.gemm_workspace_bytes(m, n, k, gpu) <= _abi.GEMM_SCRATCH_BYTES
    g = torch.Generator().manual_seed(10)
    q = randi8(g, (m, k)).to(gpu)
    w = randi8(g, (n, k)).to(gpu)
    a = (torch.rand((m, 1), generator=g) * 1e-2).to(gpu)
    s = (torch.rand((n, 1), generator=g) * 1e-3).to(gpu)
    ref = kernels.gemm(q, w, epilogue=kernels.EPI_ROW, row_scale=a, col_scale=s, out_dtype=torch.float16)
    q2 = randi8(g, (200, 4096)).to(gpu)                    # another split shape sharing the scratch
    w2 = randi8(g, (1000, 4096)).to(gpu)
    ref2 = kernels.gemm(q2, w2)
    out = torch.zeros((m, n), dtype=torch.float16, device=gpu)
    out2 = torch.zeros((200, 1000), dtype=torch.int32, device=gpu)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        rc, msg = _noalloc(_args(q, w, out, _abi.EPI_ROW, a.reshape(-1), s.reshape(-1)))   # eager, on the stream
        assert rc == _abi.OK, msg
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            rc, msg = _noalloc(_args(q, w, out, _abi.EPI_ROW, a.reshape(-1), s.reshape(-1)))
        assert rc == _abi.OK, msg
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for rep in range(4):
        out.fill_(float('nan'))
        out2.fill_(-1)
        rc, msg = _noalloc(_args(q2, w2, out2, _abi.EPI_INT32))   # overwrites the scratch between replays
        assert rc == _abi.OK, msg
        torch.cuda.synchronize()
        assert torch.equal(out2, ref2), rep
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), rep
