"""Seeded ConvRot sign vectors on the host: the generator, the kernels' sign
words and the weight rotation that keeps every projection unchanged."""
import numpy as np
import pytest
import torch

import oracle as o
from w8a8 import convrot


def test_signs_are_seeded_pm1():
    a = convrot.signs(768, 11)
    assert a.dtype == torch.int8 and a.shape == (768,)
    assert set(a.tolist()) == {-1, 1}
    assert torch.equal(a, convrot.signs(768, 11))
    assert not torch.equal(a, convrot.signs(768, 12))
    assert 300 < int((a > 0).sum()) < 468
    with pytest.raises(ValueError):
        convrot.signs(300, 1)


def test_sign_words_are_fp32_sign_bits():
    s = convrot.signs(512, 3)
    w = convrot.sign_words(s, 'cpu')
    assert w.dtype == torch.int32 and w.is_contiguous()
    assert torch.equal(w == 0, s > 0)
    # XOR with the word negates exactly the marked columns of an fp32 row
    x = torch.randn(512)
    flipped = (x.view(torch.int32) ^ w).view(torch.float32)
    assert torch.equal(flipped, x * s)


def test_hadamard_matches_the_oracle():
    assert np.array_equal(convrot.hadamard256().numpy(), o.hadamard256())


def test_rotated_weights_keep_the_projection():
    # (x diag(s) H) (W diag(s) H)^T = x W^T: diag(s) H is orthogonal.
    g = torch.Generator().manual_seed(2)
    x = torch.randn((6, 768), generator=g, dtype=torch.float64)
    w = torch.randn((40, 768), generator=g, dtype=torch.float64)
    s = convrot.signs(768, 5)
    h = convrot.hadamard256()
    xr = ((x * s.double()).reshape(6, 3, 256) @ h).reshape(6, 768)
    got = xr @ convrot.rotate_weight(w, s).double().t()
    assert torch.allclose(got, x @ w.t(), rtol=0, atol=1e-4)
    # without signs it is the reference's rotation: W H per group
    assert torch.equal(convrot.rotate_weight(torch.eye(256)), h.float())
    # and with signs the rows of W diag(s) H: row j of the identity becomes s_j H[j]
    s256 = convrot.signs(256, 9)
    assert torch.equal(convrot.rotate_weight(torch.eye(256), s256), (s256.double()[:, None] * h).float())
    with pytest.raises(ValueError):
        convrot.rotate_weight(torch.zeros((4, 100)))
