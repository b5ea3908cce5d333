"""MI355X-native W8A8 INT8 linear path (gfx950 HIP kernels behind a C ABI).

Modules mirror the reference's operator API for this path:
  parallel_int8      - quantize / int_mm / dequantize / row_linear / packed_rows
  dit_column_linear  - column_linear / shared_column_linears
  swiglu_quant       - fused FP32 SwiGLU + ConvRot256 FC2 prologue, row_linear
  row_quant          - external-maximum quantizer
  convrot            - seeded ConvRot sign vectors and the matching weight rotation
  column_epilogue    - column-order INT32 dequantization
  h3_operator_policy - operator selection for the row projections
  h3_tensor_flow     - residual divisor folding and residual add
  tp_dit             - Column/RowParallelLinearINT8, the DiT FFN block
  kernels            - typed wrappers of the C ABI
  workloads          - seeded synthetic inputs of the benchmark shapes
"""
from . import _abi  # noqa: F401

__all__ = ['kernels', 'parallel_int8', 'dit_column_linear', 'swiglu_quant', 'row_quant', 'column_epilogue',
           'h3_operator_policy', 'h3_tensor_flow', 'tp_dit', 'workloads', 'convrot']
