"""Seeded synthetic inputs for the W8A8 path's benchmark shapes.

All tensors are drawn on the CPU with torch.Generator(seed) so any consumer
(GPU kernels, the CPU baseline) sees identical bytes. Activations are FP16
N(0, sigma) with a few outlier channels scaled x20; weights are FP32
N(0, 0.02) to be quantized per output channel; biases FP16 N(0, 0.01).

Shapes:
  w8a8_linear     M=4096 tokens, K=3072, N=3072, bias, 8 outlier channels
  dit_ffn         M=16384, hidden 3072, FFN 8192 (FC1 3072 -> 2x8192 gate|up,
                  FC2 8192 -> 3072), FP16 residual N(0,1)/512
  dit_qkv         M=53504 (16 frames x 76x44 patches), 3072 -> 9216, bias,
                  0.1% outlier channels
  te_skinny       M in {1, 64, 512}, 4096 -> 14336 (up), 14336 -> 4096 (down),
                  activations N(0, 0.5)
  dit_half_shard  M=204336 in 16384-row chunks; QKV 3072 -> 4608, FC1
                  3072 -> 2x4096, FC2 4096 -> 3072 with an FP32 output
  reference_shapes  the shapes of the reference's own published operator
                  timings (one TP2 rank of MiniMax-H3): DiT S=6814 with hidden
                  5376 (QKV 5376 -> 10752, O 3584 -> 5376, FC1 5376 -> 14336,
                  FC2 7168 -> 5376) and the text encoder at S=353 with hidden
                  5120 (q 5120 -> 4096, k/v 5120 -> 512, gate/up 5120 -> 12800,
                  down 12800 -> 5120)
"""
import torch

RESIDUAL_DIVISOR = 512.0

SHAPES = {
    'w8a8_linear': dict(seed=0, m=4096, k=3072, n=3072, outliers=8),
    'dit_ffn': dict(seed=1, m=16384, hidden=3072, ffn=8192, outliers=8),
    'dit_qkv': dict(seed=2, m=53504, k=3072, n=9216, outliers=3),
    'te_skinny': dict(seed=3, ms=(1, 64, 512), hidden=4096, ffn=14336),
    'dit_half_shard': dict(seed=4, m=204336, hidden=3072, qkv=4608, ffn=4096, chunk=16384, outliers=8),
    # DiT residual stream -> norm2 with the AdaLN tables (9 modulation rows,
    # per-frame segments) -> FC1 input; eps after the 512^2 fold.
    # The QKV output of the c2 projection (53504 tokens, 3 x 24 heads of 128),
    # the H3 rotary prefix of 96 dims and fp16 rotation matrices.
    'dit_rms_rope': dict(seed=6, m=53504, heads=24, rot_dim=96),
    # The c2 QKV projection (53504 tokens, 3072 -> 3 x 24 heads of 128, no
    # bias) with the RMS-RoPE of its Q and K heads fused into the epilogue.
    'dit_qkv_rope': dict(seed=7, m=53504, k=3072, heads=24, rot_dim=96, outliers=3),
    # Attention of one DiT rank at the c2 token count: 24 heads of 128.
    'dit_attention': dict(seed=8, m=53504, heads=24),
    'dit_norm': dict(seed=5, m=16384, hidden=3072, mod_rows=9, frames=16, eps=1e-6 / RESIDUAL_DIVISOR ** 2),
    # The DiT attention sublayer of one rank at the c2 token count: residual
    # stream (divided by 512) -> norm1 + AdaLN -> QKV 3072 -> 3 x 24 heads of
    # 128 with RMS-RoPE (96-dim rotary prefix) -> attention -> O 3072 -> 3072
    # with the gated residual update.
    'dit_attention_block': dict(seed=9, m=53504, hidden=3072, heads=24, rot_dim=96, mod_rows=9, frames=16,
                                outliers=3, eps=1e-6 / RESIDUAL_DIVISOR ** 2),
}


def activations(gen, m, k, outliers, sigma=1.0):
    x = torch.randn((m, k), generator=gen, dtype=torch.float32) * sigma
    if outliers:
        cols = torch.randperm(k, generator=gen)[:outliers]
        x[:, cols] *= 20.0
    return x.half()


def weights(gen, n, k, std=0.02):
    return torch.randn((n, k), generator=gen, dtype=torch.float32) * std


def bias(gen, n):
    return (torch.randn((n,), generator=gen, dtype=torch.float32) * 0.01).half()


def w8a8_linear(m=None, seed=None):
    s = SHAPES['w8a8_linear']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m = m or s['m']
    x = activations(g, m, s['k'], s['outliers'])
    w = weights(g, s['n'], s['k'])
    b = bias(g, s['n'])
    return dict(x=x, w=w, bias=b)


def dit_ffn(m=None, hidden=None, ffn=None, seed=None):
    s = SHAPES['dit_ffn']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m, hidden, ffn = m or s['m'], hidden or s['hidden'], ffn or s['ffn']
    h = activations(g, m, hidden, s['outliers'])
    w1 = weights(g, 2 * ffn, hidden)        # rows [0, ffn) gate, [ffn, 2ffn) up
    w2 = weights(g, hidden, ffn)
    residual = (torch.randn((m, hidden), generator=g) / RESIDUAL_DIVISOR).half()
    return dict(h=h, w1=w1, w2=w2, residual=residual)


def dit_qkv(m=None, seed=None):
    s = SHAPES['dit_qkv']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m = m or s['m']
    x = activations(g, m, s['k'], s['outliers'])
    w = weights(g, s['n'], s['k'])
    b = bias(g, s['n'])
    return dict(x=x, w=w, bias=b)


def te_skinny(m, seed=None):
    s = SHAPES['te_skinny']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    x = (torch.randn((m, s['hidden']), generator=g) * 0.5).half()
    w_up = weights(g, s['ffn'], s['hidden'])
    w_down = weights(g, s['hidden'], s['ffn'])
    x_down = (torch.randn((m, s['ffn']), generator=g) * 0.5).half()
    return dict(x=x, w_up=w_up, w_down=w_down, x_down=x_down)


def dit_half_shard(m=None, seed=None):
    s = SHAPES['dit_half_shard']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m = m or s['m']
    h = activations(g, m, s['hidden'], s['outliers'])
    w_qkv = weights(g, s['qkv'], s['hidden'])
    w1 = weights(g, 2 * s['ffn'], s['hidden'])
    w2 = weights(g, s['hidden'], s['ffn'])
    return dict(h=h, w_qkv=w_qkv, w1=w1, w2=w2)


def dit_norm(m=None, hidden=None, seed=None):
    """Residual-stream rows, RMSNorm gain, AdaLN shift/scale tables and
    per-frame segments (equal row blocks cycling over the table rows)."""
    s = SHAPES['dit_norm']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m, hidden = m or s['m'], hidden or s['hidden']
    x = activations(g, m, hidden, 8, sigma=3.0)
    weight = torch.rand((hidden,), generator=g) + 0.5
    shift = torch.randn((s['mod_rows'], hidden), generator=g) * 0.1
    scale = torch.randn((s['mod_rows'], hidden), generator=g) * 0.1
    frames = min(s['frames'], m)
    bounds = [m * i // frames for i in range(frames + 1)]
    segments = [(bounds[i], bounds[i + 1], i % s['mod_rows']) for i in range(frames) if bounds[i] < bounds[i + 1]]
    return dict(x=x, weight=weight, shift=shift, scale=scale, segments=segments, eps=s['eps'])


def dit_rms_rope(m=None, seed=None):
    """Packed fp16 QKV rows, fp16 split-half rotation matrices, fp32 gains."""
    s = SHAPES['dit_rms_rope']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m = m or s['m']
    packed = (torch.randn((m, 3 * s['heads'] * 128), generator=g) * 2).half()
    ang = torch.rand((m, s['rot_dim'] // 2), generator=g, dtype=torch.float64) * 6.283185307179586
    c, sn = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([c, -sn], -1), torch.stack([sn, c], -1)], -2).half()
    q_gain = torch.rand(128, generator=g) + 0.5
    k_gain = torch.rand(128, generator=g) + 0.5
    return dict(packed=packed, freqs=freqs, q_gain=q_gain, k_gain=k_gain, heads=s['heads'], rot_dim=s['rot_dim'])


def dit_qkv_rope(m=None, seed=None):
    """fp16 activation, QKV weights [3 * heads * 128, k], fp16 rotation matrices, fp32 gains."""
    s = SHAPES['dit_qkv_rope']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m = m or s['m']
    x = activations(g, m, s['k'], s['outliers'])
    w = weights(g, 3 * s['heads'] * 128, s['k'])
    ang = torch.rand((m, s['rot_dim'] // 2), generator=g, dtype=torch.float64) * 6.283185307179586
    c, sn = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([c, -sn], -1), torch.stack([sn, c], -1)], -2).half()
    q_gain = torch.rand(128, generator=g) + 0.5
    k_gain = torch.rand(128, generator=g) + 0.5
    return dict(x=x, w=w, freqs=freqs, q_gain=q_gain, k_gain=k_gain, heads=s['heads'], rot_dim=s['rot_dim'])


def dit_attention(m=None, seed=None):
    """q, k, v [1, heads, m, 128] fp16 ~ N(0, 1) (the RMS-normalized Q/K scale)."""
    s = SHAPES['dit_attention']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m = m or s['m']
    shape = (1, s['heads'], m, 128)
    return {n: torch.randn(shape, generator=g, dtype=torch.float32).half() for n in ('q', 'k', 'v')}


def dit_attention_block(m=None, seed=None):
    """Residual rows (/512), norm1 gain, AdaLN shift/scale/gate tables with
    per-frame segments, QKV and O weights (fp32, ConvRot-domain), fp16
    rotation matrices (1, m, 1, rot_dim / 2, 2, 2) and the Q/K norm gains."""
    s = SHAPES['dit_attention_block']
    g = torch.Generator().manual_seed(s['seed'] if seed is None else seed)
    m, hidden, heads = m or s['m'], s['hidden'], s['heads']
    x = (activations(g, m, hidden, s['outliers']).float() / RESIDUAL_DIVISOR).half()
    weight = torch.rand((hidden,), generator=g) + 0.5
    shift, scale, gate = (torch.randn((s['mod_rows'], hidden), generator=g) * 0.1 for _ in range(3))
    frames = min(s['frames'], m)
    bounds = [m * i // frames for i in range(frames + 1)]
    segments = [(bounds[i], bounds[i + 1], i % s['mod_rows']) for i in range(frames) if bounds[i] < bounds[i + 1]]
    w_qkv = weights(g, 3 * heads * 128, hidden)
    w_o = weights(g, hidden, heads * 128)
    half = s['rot_dim'] // 2
    ang = torch.rand((m, half), generator=g, dtype=torch.float64) * 6.283185307179586
    c, sn = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([c, -sn], -1), torch.stack([sn, c], -1)], -2).half().reshape(1, m, 1, half, 2, 2)
    q_gain = torch.rand(128, generator=g) + 0.5
    k_gain = torch.rand(128, generator=g) + 0.5
    return dict(x=x, weight=weight, shift=shift, scale=scale, gate=gate, segments=segments, eps=s['eps'],
                w_qkv=w_qkv, w_o=w_o, freqs=freqs, q_gain=q_gain, k_gain=k_gain, heads=heads, hidden=hidden)


# name: (role, M, N, K, the reference's T4 rank-0 time in ms for the same
# operator, its source). Roles: 'column' (ConvRot256 quantize + GEMM + column
# dequant), 'row' (FP32 ConvRot256 quantize of the rank's K slice + GEMM ->
# FP32 partial), 'fc2' (fused SwiGLU/ConvRot256 prologue on [M, 2K] + GEMM ->
# FP32 partial). The T4 times are the GEMM alone for the DiT shapes
# (docs/reports/TP2_OPERATOR_RESULTS.md:132-135) and the complete row
# projection (prologue, GEMM and scaled-FP16 SUM) for the TE down projection
# (docs/reports/FP16_FC2_FUSION_VIDEO_SPLIT_20261022.md:149).
REFERENCE_SHAPES = {
    'dit_qkv': ('column', 6814, 10752, 5376, 20.02, 'TP2_OPERATOR_RESULTS.md:132'),
    'dit_o': ('row', 6814, 5376, 3584, 6.51, 'TP2_OPERATOR_RESULTS.md:133'),
    'dit_fc1': ('column', 6814, 14336, 5376, 28.69, 'TP2_OPERATOR_RESULTS.md:134'),
    'dit_fc2': ('fc2', 6814, 5376, 7168, 14.23, 'TP2_OPERATOR_RESULTS.md:135'),
    'te_q': ('column', 353, 4096, 5120, None, None),
    'te_kv': ('column', 353, 512, 5120, None, None),
    'te_gate_up': ('column', 353, 12800, 5120, None, None),
    'te_down': ('fc2', 353, 5120, 12800, 1.906, 'FP16_FC2_FUSION_VIDEO_SPLIT_20261022.md:149'),
}


def reference_shape(name, seed=10):
    """Seeded inputs of one reference shape: x fp16 [M, K] (N(0,1) with x20
    outlier channels; [M, 2K] gate|up for the 'fc2' role) and w fp32 [N, K]."""
    role, m, n, k = REFERENCE_SHAPES[name][:4]
    g = torch.Generator().manual_seed(seed + sorted(REFERENCE_SHAPES).index(name))
    if role == 'fc2':
        x = (torch.randn((m, 2 * k), generator=g)).half()
    else:
        x = activations(g, m, k, 8)
    return dict(role=role, x=x, w=weights(g, n, k))


def quantize_weight(w, device):
    """Per-output-channel INT8 weights and FP32 scales [N, 1] on the GPU (libw8a8)."""
    from . import kernels
    return kernels.quantize_rows(w.to(device=device, dtype=torch.float32))
