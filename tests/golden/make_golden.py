"""Write the small golden fixtures of the W8A8 path (run from the repository root).

    python tests/golden/make_golden.py

The reference holds no tensor fixtures for this path (its arithmetic pins need
comfy-kitchen, TileLang and CUDA), so these vectors are produced by this
build's oracle from seeded inputs, after the oracle itself is pinned by
tests/test_oracle.py. They freeze the oracle's bits (a CPU test regenerates and
compares) and give the GPU tests an input/output set that does not depend on
running the oracle at test time. Inputs follow the reference's test patterns:
row tails (benchmarks/test_bounded_column_int8.py:11-28), signed extremes
(benchmarks/test_te_column_layout.py:28-34), adversarial INT32 values
(benchmarks/test_tp2_p2_epilogue.py:18-25). The later fixtures (gated residual,
modulated norm + quantize, RMS-RoPE, INT8 attention) draw from a second seeded
generator so the earlier files stay byte-identical.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import oracle as o  # noqa: E402


def fixtures():
    rng = np.random.default_rng(20261201)
    out = {}
    # 1. per-row quantize, fp16 rows incl. a zero row and outlier channels
    x = (rng.standard_normal((13, 512)) * 2).astype(np.float16)
    x[3] = 0
    x[:, 7] *= 20
    q, s = o.quantize_rows(x.astype(np.float32))
    out['quant'] = dict(x=x, q=q, scale=s)
    # 2. ConvRot256 column preparation (rotation rounded to fp16)
    q, s = o.prepare_activation(x, convrot=True, x_dtype='f16')
    out['quant_convrot'] = dict(x=x, q=q, scale=s)
    # 3. FC2 prologue
    xs = (rng.standard_normal((5, 1024)) * 3).astype(np.float16)
    xs[0, 0], xs[0, 1] = 60000.0, -60000.0
    q, s, g = o.fc2_prologue(xs)
    out['swiglu'] = dict(x=xs, q=q, scale=s, group_max=g)
    # 4. INT8 GEMM with signed extremes and a K tail
    a = rng.integers(-128, 128, (33, 80)).astype(np.int8)
    b = rng.integers(-128, 128, (48, 80)).astype(np.int8)
    a[0] = -128
    b[0] = -128
    out['gemm'] = dict(a=a, b=b, c=o.int_mm(a, b))
    # 5. epilogues on adversarial int32 accumulators
    acc = rng.integers(-10_000_000, 10_000_000, (17, 256)).astype(np.int32)
    acc[:, 0] = 16777217
    acc[:, 1] = -8388609
    acc[:, 2:10] = [1, -1, 3, -3, 127, -127, 65535, -65535]
    acc[:, 10] = 7168 * 128 * 128
    ra = (rng.random(17) * 0.1).astype(np.float32)
    wa = (rng.random(256) * 0.001).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.01).astype(np.float16)
    out['epilogue'] = dict(acc=acc, a=ra, w=wa, bias=bias,
                           row_f16=o.dequantize_row(acc, ra, wa, 'f16', bias),
                           row_f32=o.dequantize_row(acc, ra, wa, 'f32'),
                           col_f16=o.dequantize_column(acc, ra, wa, 'f16', bias),
                           col_bf16=o.dequantize_column(acc, ra, wa, 'bf16'))
    rng = np.random.default_rng(20261202)
    # 6. DiT gated residual update in the row epilogue
    res = (rng.standard_normal((17, 256)) * 0.05).astype(np.float16)
    gate = rng.standard_normal((3, 256)).astype(np.float32)
    labels = rng.integers(0, 3, 17).astype(np.int32)
    branch = o.dequantize_row(acc, ra, wa, 'f16')
    out['gated'] = dict(acc=acc, a=ra, w=wa, residual=res, gate=gate, labels=labels,
                        out=o.gated_residual_add(res, branch, gate, labels))
    # 7. modulated RMSNorm -> ConvRot256 -> INT8 (one zero row, one outlier channel)
    xn = (rng.standard_normal((13, 512)) * 3).astype(np.float16)
    xn[5] = 0
    xn[:, 11] *= 20
    nw = (rng.random(512) + 0.5).astype(np.float32)
    shift = (rng.standard_normal((4, 512)) * 0.1).astype(np.float32)
    scale = (rng.standard_normal((4, 512)) * 0.1).astype(np.float32)
    nl = rng.integers(0, 4, 13).astype(np.int32)
    qn, sn, y = o.norm_quantize(xn, nw, shift, scale, nl, eps=1e-6)
    out['norm_quant'] = dict(x=xn, weight=nw, shift=shift, scale=scale, labels=nl, y=y, q=qn, row_scale=sn)
    # 8. per-head RMS norm + split-half RoPE of a packed QKV row block (2 heads, rotary prefix 96)
    packed = (rng.standard_normal((7, 3 * 2 * 128)) * 2).astype(np.float16)
    ang = rng.random((7, 48)) * 2 * np.pi
    c, sn_ = np.cos(ang), np.sin(ang)
    freqs = np.stack([np.stack([c, -sn_], -1), np.stack([sn_, c], -1)], -2).astype(np.float32)
    gq = (rng.random(128) + 0.5).astype(np.float32)
    gk = (rng.random(128) + 0.5).astype(np.float32)
    rq, rk = o.rms_rope(packed, freqs, gq, gk, 2, 96, eps=1e-6)
    out['rms_rope'] = dict(packed=packed, freqs=freqs, q_gain=gq, k_gain=gk, q=rq, k=rk)
    # 9. INT8 attention (the reference kernel's scheme, 128-key blocks):
    # prepared operands (exact) and the oracle output
    from oracle import int8_attention as oa
    qa = rng.standard_normal((1, 2, 37, 128)).astype(np.float16)
    ka = (rng.standard_normal((1, 2, 70, 128)) + 0.5).astype(np.float16)
    va = rng.standard_normal((1, 2, 70, 128)).astype(np.float16)
    prep = oa.kitchen_prepare(qa.astype(np.float32), ka.astype(np.float32), va.astype(np.float32),
                              cta_k=oa.GPU_CTA_K)
    out['attention'] = dict(q=qa, k=ka, v=va, **oa.gpu_operands(prep), out=oa.kitchen_attention(prep))
    return out


def main():
    for name, arrays in fixtures().items():
        np.savez_compressed(HERE / f'{name}.npz', **arrays)
        print('wrote', HERE / f'{name}.npz')


if __name__ == '__main__':
    main()
