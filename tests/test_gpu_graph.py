"""The W8A8 entry points under HIP graph capture: a captured DiT FFN block
(FC1 input quantize, column GEMM, FC2 prologue, split-K row GEMM with a
residual), the fused modulated norm and RMS-RoPE, replayed several times with
eager work in between, each replay bit-identical to the eager result."""
import pytest
import torch

from helpers import randn16
from w8a8 import kernels, workloads
from w8a8.h3_tensor_flow import prepare_tp, TensorFlowPolicy
from w8a8.tp_dit import DiTFeedForwardINT8

pytestmark = pytest.mark.gpu


def test_captured_graph_replays_match_eager(gpu):
    data = workloads.dit_ffn(m=512, hidden=768, ffn=1024)
    block = DiTFeedForwardINT8(768, 1024, device=gpu)
    wq1, ws1 = workloads.quantize_weight(data['w1'], gpu)
    wq2, ws2 = workloads.quantize_weight(data['w2'], gpu)
    block.fc1.weight.data.copy_(wq1)
    block.fc1.weight_scale.data.copy_(ws1)
    block.fc2.weight.data.copy_(wq2)
    block.fc2.weight_scale.data.copy_(ws2)
    prepare_tp(block, 'dit', TensorFlowPolicy(mode='fp16'))
    assert kernels.gemm_workspace_bytes(512, 768, 1024, gpu) > 0      # the FC2 GEMM splits K here
    h = data['h'].to(gpu)
    res = data['residual'].to(gpu)
    g = torch.Generator().manual_seed(7)
    x = randn16(g, (300, 3072), 3.0).to(gpu)
    w = (torch.rand(3072, generator=g) + 0.5).to(gpu)
    shift = (torch.randn((9, 3072), generator=g) * 0.1).to(gpu)
    scale = (torch.randn((9, 3072), generator=g) * 0.1).to(gpu)
    labels = torch.randint(0, 9, (300,), generator=g, dtype=torch.int32).to(gpu)
    packed = randn16(g, (200, 3 * 8 * 128), 2.0).to(gpu)
    ang = torch.rand((200, 48), generator=g, dtype=torch.float64) * 6.283185307179586
    freqs = torch.stack([torch.stack([ang.cos(), -ang.sin()], -1), torch.stack([ang.sin(), ang.cos()], -1)], -2)
    freqs = freqs.half().to(gpu)
    gq = (torch.rand(128, generator=g) + 0.5).to(gpu)

    def work():
        y = block(h, res)
        nq = kernels.norm_quantize(x, w, shift, scale, labels, eps=1e-6 / 512 ** 2)
        q, k = kernels.rms_rope(packed, freqs, gq, gq, heads=8, rot_dim=96, eps=1e-6)
        return y, nq['q'], nq['scale'], q, k

    eager = [t.clone() for t in work()]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        work()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            outs = work()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for rep in range(4):
        for t in outs:
            t.fill_(0)                      # replays must rewrite every output
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(outs, eager)):
            assert torch.equal(got, want), (rep, i)
        again = work()                      # eager work between replays
        torch.cuda.synchronize()
        for got, want in zip(again, eager):
            assert torch.equal(got, want), rep
