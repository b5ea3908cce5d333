"""Host-side contracts of the Python API (CPU only): guards raise before any
library call, policies validate, weights shard like the reference."""
import pytest
import torch

from w8a8 import dit_column_linear, kernels, parallel_int8, row_quant, swiglu_quant, workloads
from w8a8.h3_operator_policy import H3OperatorPolicy
from w8a8.h3_tensor_flow import TensorFlowPolicy, fold_linear, residual_add


def test_cpu_tensors_are_rejected_not_computed():
    x = torch.randn(4, 256).half()
    w = torch.randint(-127, 127, (32, 256), dtype=torch.int8)
    s = torch.rand(32, 1)
    with pytest.raises(ValueError, match='HIP device'):
        kernels.quantize_rows(x)
    with pytest.raises(ValueError, match='HIP device'):
        kernels.gemm(torch.zeros(4, 256, dtype=torch.int8), w)
    with pytest.raises(ValueError, match='HIP device'):
        dit_column_linear.column_linear(x, w, s)
    with pytest.raises(ValueError):
        row_quant.quantize(x.float(), torch.ones(4, 1))


def test_contract_errors_match_reference_messages():
    x = torch.randn(4, 256).half()
    w = torch.randint(-127, 127, (32, 128), dtype=torch.int8)
    with pytest.raises(ValueError, match='Unknown column linear backend'):
        dit_column_linear.column_linear(x, w, torch.rand(32, 1), backend='x')
    with pytest.raises(ValueError, match='inner dimensions'):
        dit_column_linear.column_linear(x, w, torch.rand(32, 1))
    with pytest.raises(ValueError, match='Packed components'):
        parallel_int8.packed_rows(torch.zeros(10, 4), torch.zeros(10, 1), 0, 2, 3)
    with pytest.raises(ValueError, match='world_size'):
        parallel_int8.row_linear(x, w, torch.rand(32, 1), None, 2)
    with pytest.raises(ValueError):
        swiglu_quant.prepare(x, None, mode='control')
    with pytest.raises(ValueError, match='P0-3'):
        swiglu_quant.prepare(x, None, mode='fused_recompute', consume_input=True)


def test_packed_rows_component_split():
    w = torch.arange(12).reshape(12, 1)
    s = torch.arange(12).reshape(12, 1).float()
    w0, s0 = parallel_int8.packed_rows(w, s, 0, 2, 3)
    w1, _ = parallel_int8.packed_rows(w, s, 1, 2, 3)
    assert w0.flatten().tolist() == [0, 1, 4, 5, 8, 9] and w1.flatten().tolist() == [2, 3, 6, 7, 10, 11]
    assert s0.flatten().tolist() == [0, 1, 4, 5, 8, 9]


def test_policies_validate():
    H3OperatorPolicy()
    for bad in (dict(row_linear_backend='x'), dict(fc2_quantizer='x'), dict(column_linear_backend='x')):
        with pytest.raises(ValueError):
            H3OperatorPolicy(**bad)
    p = TensorFlowPolicy(mode='fp16')
    assert p.enabled and p.divisor == 512.0 and p.dtype == torch.float16
    with pytest.raises(ValueError):
        TensorFlowPolicy(mode='x')
    with pytest.raises(ValueError):
        TensorFlowPolicy(residual_exponent=13)


def test_fold_linear_is_exact_power_of_two():
    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.weight_scale = torch.nn.Parameter(torch.rand(8, 1) * 1e-3, requires_grad=False)
    m = M()
    before = m.weight_scale.detach().clone()
    fold_linear(m, 512.0)
    assert torch.equal(m.weight_scale * 512.0, before)
    with pytest.raises(ValueError):
        fold_linear(torch.nn.Linear(2, 2), 512.0)


def test_residual_add_rounding_order():
    x = torch.tensor([1.0, 2048.0], dtype=torch.float16)
    b = torch.tensor([0.0004883, 1.0], dtype=torch.float16)
    assert residual_add(x, b).tolist() == [1.0, 2048.0]


def test_workload_shapes_and_determinism():
    a = workloads.w8a8_linear(m=64)
    b = workloads.w8a8_linear(m=64)
    assert torch.equal(a['x'], b['x']) and a['x'].dtype == torch.float16 and a['w'].shape == (3072, 3072)
    # 8 outlier channels are scaled x20
    big = (a['x'].float().abs().amax(0) > 30).sum().item()
    assert 1 <= big <= 8
    f = workloads.dit_ffn(m=32)
    assert f['w1'].shape == (16384, 3072) and f['w2'].shape == (3072, 8192) and f['residual'].shape == (32, 3072)


def test_segment_labels():
    from w8a8.h3_tensor_flow import labels_for, segment_key
    assert segment_key(5, [(0, 2, 7), (2, 5, 0)]) == ((0, 2, 7), (2, 5, 0))
    for segments in ([(0, 2, 0)], [(0, 3, 0), (2, 5, 1)], [(0, 5, 9)]):
        assert segment_key(5, segments) is None      # gap, overlap, row out of range
    assert labels_for(5, [(2, 5, 0), (0, 2, 7)]).tolist() == [7, 7, 0, 0, 0]
    assert labels_for(5, [(0, 4, 1)]) is None


def test_output_buffers_are_validated_before_any_launch():
    x = torch.randn(8, 256).half()
    with pytest.raises(ValueError, match='out must be int8'):
        kernels.quantize_rows(x, out=torch.empty(4, 256, dtype=torch.int8))
    with pytest.raises(ValueError, match='out must be int8'):
        kernels.quantize_rows(x, out=torch.empty(8, 256, dtype=torch.int16))
    with pytest.raises(ValueError, match='out must be int8'):
        kernels.quantize_rows(x, out=torch.empty(256, 8, dtype=torch.int8).t())
    with pytest.raises(ValueError, match='scale_out'):
        kernels.quantize_rows(x, scale_out=torch.empty(4, 1))
    with pytest.raises(ValueError, match='scale_out'):
        kernels.quantize_rows(x, scale_out=torch.empty(8, 1, dtype=torch.float16))
    q = torch.zeros(8, 256, dtype=torch.int8)
    w = torch.zeros(32, 256, dtype=torch.int8)
    with pytest.raises(ValueError, match='out must be int32'):
        kernels.gemm(q, w, out=torch.empty(4, 32, dtype=torch.int32))
    with pytest.raises(ValueError, match='out must be int32'):
        kernels.gemm(q, w, out=torch.empty(32, 8, dtype=torch.int32).t())
    with pytest.raises(ValueError, match='out must be'):
        kernels.gemm(q, w, epilogue=kernels.EPI_ROW, row_scale=torch.ones(8), col_scale=torch.ones(32),
                     out=torch.empty(8, 16, dtype=torch.float16))
    with pytest.raises(ValueError, match='HIP device'):      # shapes right: the device check follows
        kernels.gemm(q, w, out=torch.empty(8, 32, dtype=torch.int32))


class _Recorder:
    def __init__(self):
        self.calls = []

    def __call__(self, x, weight, weight_scale, comm, world_size, groupsize, input_act):
        self.calls.append((x, input_act))
        return torch.zeros(x.shape[0], weight.shape[0], dtype=x.dtype)


def test_row_linear_parts_branches_on_the_host():
    from w8a8.h3_operator_policy import H3OperatorPolicy, row_linear_parts
    from w8a8.tp_qwen3vl import RowParallelLinearINT8
    m = RowParallelLinearINT8(256, 32, device='cpu')
    gate = torch.randn(4, 256).half()
    up = torch.randn(4, 256).half()
    m.operator_policy = H3OperatorPolicy()
    with pytest.raises(ValueError, match='Matching gate/up'):     # only the fused route checks
        row_linear_parts(m, gate, up.float(), _Recorder(), None)
    m.operator_policy = H3OperatorPolicy(fc2_quantizer='native')
    rec = _Recorder()
    row_linear_parts(m, gate, up, rec, None)
    (x, act), = rec.calls
    assert act is None and x.dtype == torch.float32    # the scaled-FP16 backend's FP32 island
    assert torch.equal(x, (torch.nn.functional.silu(gate) * up).float())
    rec = _Recorder()
    row_linear_parts(m, gate, up.float(), rec, None)    # mismatched halves are fine off the fused route
    assert rec.calls[0][1] is None


def test_prepare_tp_folds_norms_and_projections():
    from w8a8.h3_tensor_flow import StableNorm, prepare_tp
    from w8a8.tp_dit import TPDiTBlockINT8
    b = TPDiTBlockINT8(hidden=256, heads=2, ffn=512, device='cpu')
    for m in (b.out_proj, b.fc2, b.fc1):
        m.weight_scale.data.copy_(torch.rand(m.weight_scale.shape) + 1e-3)
    before = {n: getattr(b, n).weight_scale.detach().clone() for n in ('out_proj', 'fc2', 'fc1')}
    prepare_tp(b, 'dit', TensorFlowPolicy(mode='fp16'))
    assert torch.equal(b.out_proj.weight_scale * 512, before['out_proj'])
    assert torch.equal(b.fc2.weight_scale * 512, before['fc2'])
    assert torch.equal(b.fc1.weight_scale, before['fc1'])          # column projections are not folded
    for n in ('norm1', 'norm2', 'q_norm', 'k_norm'):
        assert isinstance(getattr(b, n), StableNorm), n
    assert b.norm1.eps == 1e-5 / 512 ** 2 and b.norm2.eps == 1e-5 / 512 ** 2 and b.k_norm.eps == 1e-5
    with pytest.raises(ValueError, match='already prepared'):
        prepare_tp(b, 'dit', TensorFlowPolicy(mode='fp16'))
    legacy = TPDiTBlockINT8(hidden=256, heads=2, ffn=512, device='cpu')
    assert prepare_tp(legacy, 'dit', TensorFlowPolicy()) is legacy and legacy.norm1.eps == 1e-5
    # StableNorm on FP32 rows: torch's fp32 RMSNorm with the folded eps
    x = torch.randn(5, 256)
    want = torch.nn.functional.rms_norm(x, (256,), b.norm1.weight.float(), 1e-5 / 512 ** 2)
    assert torch.equal(b.norm1(x), want)


def test_te_prepare_and_adjacent_columns():
    from w8a8.h3_operator_policy import adjacent_cat
    from w8a8.h3_tensor_flow import StableNorm, prepare_tp
    from w8a8.tp_qwen3vl import TEFeedForwardINT8
    ffn = TEFeedForwardINT8(256, 512, device='cpu')
    ffn.down_proj.weight_scale.data.fill_(1.0)
    prepare_tp(ffn, 'te', TensorFlowPolicy(mode='fp16'))
    assert isinstance(ffn.post_attention_layernorm, StableNorm)
    assert ffn.post_attention_layernorm.eps == 1e-6 / 512 ** 2
    assert torch.all(ffn.down_proj.weight_scale == 1 / 512)
    buf = torch.randn(6, 40)
    g, u = buf[:, 4:20], buf[:, 20:36]
    cat = adjacent_cat(g, u)
    assert cat.data_ptr() == g.data_ptr() and torch.equal(cat, torch.cat((g, u), -1))
    other = adjacent_cat(buf[:, :16], buf[:, 20:36])          # not adjacent: a copy
    assert other.data_ptr() != buf.data_ptr() and torch.equal(other, torch.cat((buf[:, :16], buf[:, 20:36]), -1))


def test_rank_shard_contracts():
    from w8a8.tp_dit import RowParallelLinearINT8
    m = RowParallelLinearINT8(1024, 64, rank=1, world_size=2, device='cpu')
    assert m.in_features_per_rank == 512
    with pytest.raises(ValueError, match='rank shard takes'):
        m.partial(torch.zeros(3, 1024).half())
    with pytest.raises(ValueError, match='rank shard takes'):
        m.local_maximum(torch.zeros(3, 512).half(), 'swiglu')
    with pytest.raises(ValueError, match='SUM exchange'):
        m(torch.zeros(3, 512).half(), residual=torch.zeros(3, 64).half())
    with pytest.raises(ValueError, match='requires reduction'):
        m(torch.zeros(3, 512).half(), reduce_sum=False)
    with pytest.raises(ValueError, match='HIP device'):       # contract met: the CPU tensor is refused
        m.partial(torch.zeros(3, 512).half())
    whole = RowParallelLinearINT8(1024, 64, device='cpu')
    with pytest.raises(ValueError, match='MAX exchange'):
        whole(torch.zeros(3, 1024).half(), row_max=torch.ones(3, 1))
