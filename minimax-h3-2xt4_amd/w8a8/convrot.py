"""Seeded sign vectors for ConvRot256.

ConvRot256 multiplies each 256-column group of an activation row by
H = (H4r)^{(x)4} / 16, H4r = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]]
(the regular-H4 butterfly the quantize kernels run, as in
patches/tilelang_swiglu_quant.py:26-36), with the weights stored rotated the
same way. The reference's rotation has fixed signs. As an option of this
build, a seeded +-1 vector s turns the rotation into diag(s) then H: the
kernels negate the marked columns before the butterfly (sign words, one per
column), and weights rotated by rotate_weight(w, s) keep every projection
unchanged, since diag(s) H is orthogonal (H is symmetric with H H = I).
Leaving the signs out is the reference's rotation.
"""
import torch

GROUP = 256


def signs(cols, seed):
    """+-1 int8 vector of length cols drawn from torch's CPU generator seeded
    with seed (the same seed gives the same vector everywhere)."""
    if cols % GROUP:
        raise ValueError('ConvRot signs cover whole 256-column groups')
    g = torch.Generator().manual_seed(int(seed))
    return (torch.randint(0, 2, (cols,), generator=g, dtype=torch.int8) * 2 - 1).to(torch.int8)


def sign_words(s, device):
    """The kernels' form of a sign vector: int32 words, 0 where s > 0 and
    0x80000000 (the fp32 sign bit) where s < 0, contiguous on device."""
    s = torch.as_tensor(s)
    return torch.where(s.reshape(-1) < 0, torch.tensor(-2 ** 31, dtype=torch.int32),
                       torch.tensor(0, dtype=torch.int32)).contiguous().to(device)


def hadamard256(dtype=torch.float64, device=None):
    """H = (H4r)^{(x)4} / 16: H[i][j] = (-1)^{#base-4 digits d with i_d + j_d = 3} / 16."""
    idx = torch.arange(GROUP, device=device)
    digits = torch.stack([(idx >> (2 * d)) & 3 for d in range(4)], dim=-1)
    count = ((digits[:, None, :] + digits[None, :, :]) == 3).sum(-1)
    return torch.where(count % 2 == 0, 1.0, -1.0).to(dtype) / 16.0


def rotate_weight(w, s=None):
    """Weights [N, K] (K % 256 == 0) rotated as the activations are: each
    256-column group of each row becomes w_g diag(s_g) H, in float64, returned
    as float32 (to be quantized per output channel like any weight)."""
    w = torch.as_tensor(w)
    n, k = w.shape
    if k % GROUP:
        raise ValueError('ConvRot needs whole 256-column groups')
    w64 = w.to(torch.float64).reshape(n, k // GROUP, GROUP)
    if s is not None:
        w64 = w64 * torch.as_tensor(s).to(torch.float64).reshape(k // GROUP, GROUP)
    h = hadamard256(torch.float64, w64.device)
    return (w64 @ h).reshape(n, k).to(torch.float32)
