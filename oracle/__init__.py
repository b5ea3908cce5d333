"""CPU oracle of the W8A8 INT8 linear path - TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's torch
quantize + ``_int_mm`` + dequantize path and of its fused FC2 prologue, so
that the HIP kernels can be checked bit for bit. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it, and only as the checker (or the timed CPU baseline): the product
path (the ``w8a8`` package and ``libw8a8.so``) never calls it and has no CPU
fallback.

Pinning (what checks each function, beyond "the same formula retyped"):

* ``quantize_rows``     - hand-computed known answers, exact ties (half to
  even), zero rows (scale 1e-30), the absmax element mapping to +-127, and a
  scale that distinguishes ``amax * fp32(1/127)`` from ``amax / 127``.
* ``convrot256``        - the closed form H[i][j] = (-1)^#{digits with
  i_d + j_d = 3} / 16 in float64 (exact on small integer inputs), H.H = I,
  unit vectors mapping to columns, norm preservation.
* ``exp_f32``           - against float64 ``exp`` over a dense sweep (<= 2
  ulp), exact at 0, overflow/underflow thresholds.
* ``swiglu_f32``        - against float64 ``g*u/(1+exp(-g))`` (few ulp) and
  special values.
* ``int_mm``            - brute-force int64 products on small inputs and the
  all -128 known answer K*16384.
* ``dequantize_*``      - the reference's hand example
  (benchmarks/test_fp16_fc2_experiment.py:11-29), and order-sensitive cases
  where (C*a)*w and C*(a*w) round differently.
* ``fc2_prologue``      - composition of the pinned pieces, plus the
  invariant that rotated row norms equal the SwiGLU row norms.
* ``row_linear``        - composition of the pinned pieces; rotating the
  activation and the weight rows alike leaves x.W^T unchanged (H H^T = I),
  so the result tracks float64 x.W^T within the INT8 error, which a
  rotation missing on either side fails.
* ``row_partial``, ``rank_row_max`` - the sharding identity: over two
  rank halves (whole 256-channel groups each) the maximum of the ranks'
  row maxima equals the unsharded row maximum, and the ranks' int32
  partials quantized with it add up exactly to the unsharded accumulator;
  a wrong K slice, a wrong gate/up pairing or a local maximum fails it.
* ``fma_f32``           - exact rational arithmetic (fractions) on random
  and constructed midpoint cases, where the unfused a*b+c rounds differently.
* ``gated_residual_add`` - composition of fma_f32 with the FP16 branch and
  residual casts; the reference's own torch restatement
  (benchmarks/test_h3_dit_fusion.py:95-106) on inputs where fused and unfused
  agree.
* ``rms_sum_squares``   - exact totals on integer squares (any order),
  hand-computed known answers whose value depends on the lane order and on
  the butterfly (absorption of small squares by a 2^24 partial), padding
  of a partial last lane block, and a float64 error bound on random rows.
* ``modulated_rms_norm`` - numpy's float32 sqrt and division checked against
  float64 rounded once (exact for these two operations); closed cases
  (constant power-of-two rows give +-1 exactly; scale = -1 yields the shift
  table row exactly, which pins the label indexing), and a float64 bound
  against torch's own fp32 F.rms_norm on random rows.
* ``head_sum_squares`` - exact integer totals; a hand-computed absorption
  case that fixes the slice order and the descending butterfly offsets.
* ``rms_rope``          - identity frequencies (F = I) reduce it to the
  pinned norm times the gain; a quarter turn (F = [[0,-1],[1,0]]) swaps the
  halves with a sign, exactly; scaling the input by a power of two leaves the
  output unchanged; against a float64 torch restatement on random inputs.
* ``norm_quantize``     - composition of the pinned norm with the pinned
  ``prepare_activation`` / ``convrot256`` + ``quantize_rows``.
* ``int8_attention``    - (module) the permutation of the transposed V
  layout; an exact chunked key mean on integer data; absmax elements mapping
  to +-127 and the folded softmax scale; identical keys give the mean of the
  quantized values, one dominant key gives its value row; random inputs
  within cosine 0.999 of float64 softmax attention, which a wrong softmax
  scale fails. ``kitchen_attention`` (the reference's vendored kernel,
  restated): u8 tiles of exactly 255 on identical keys (the log2 255 offset),
  a dominant key returning its value row, the kernel's per-thread scale
  groups, cosine 0.9998 against float64 attention and agreement between its
  two key-block sizes. Kitchen's quantizer and CUDA's ex2.approx / rcp.approx
  are absent, so its bits are unpinned.

Functions that only an import of the absent third-party comfy-kitchen 0.2.37
could pin bit for bit (its GEMM-based rotation summation order) are noted
"parity unpinned" in the function docstrings.
"""
from .w8a8_oracle import (  # noqa: F401
    R127, SCALE_FLOOR, INV16,
    quantize_rows, convrot256, hadamard256, exp_f32, swiglu_f32,
    prepare_activation, fc2_prologue, int_mm, dequantize_row,
    dequantize_column, residual_add, to_bf16_bits, from_bf16_bits,
    cast_out, quantize_weight, column_linear, row_linear, row_linear_fc2, ffn_block,
    fma_f32, gated_residual_add, rms_sum_squares, modulated_rms_norm,
    norm_quantize, head_sum_squares, rms_rope, row_partial, rank_row_max,
)
