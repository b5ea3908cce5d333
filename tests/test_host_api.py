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
