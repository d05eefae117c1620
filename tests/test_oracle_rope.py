"""The RoPE oracle against what the mathematics fixes (CPU only)."""

import numpy as np
import torch

from oracle import rope as R


def _x(shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape)


def test_rotation_preserves_pair_norms_and_unit_frequency_is_identity():
    x = _x((2, 5, 3, 16))
    f = R.freqs_cis(16, 5)
    y = R.rope(x, f)
    np.testing.assert_allclose(np.hypot(y[..., 0::2], y[..., 1::2]), np.hypot(x[..., 0::2], x[..., 1::2]), rtol=1e-12)
    np.testing.assert_allclose(y[:, 0], x[:, 0], rtol=0, atol=0)  # position 0: angle 0


def test_rotations_compose():
    x = _x((1, 7, 2, 8), seed=1)
    f1, f2 = R.freqs_cis(8, 7), R.freqs_cis(8, 7, theta=77.0)
    np.testing.assert_allclose(R.rope(R.rope(x, f1), f2), R.rope(x, f1 * f2), rtol=1e-12, atol=1e-12)


def test_per_sequence_frequencies_select_rows():
    x = _x((3, 4, 2, 8), seed=2)
    table = R.freqs_cis(8, 10)
    pos = np.array([[0, 1, 2, 3], [5, 6, 7, 8], [2, 2, 9, 0]])
    y = R.rope(x, table[pos])
    for b in range(3):
        np.testing.assert_allclose(y[b:b + 1], R.rope(x[b:b + 1], table[pos[b]]), rtol=0, atol=0)


def test_matches_the_reference_op_sequence_in_torch():
    # model.py:225-230 with torch (view_as_complex, complex multiply, view_as_real) in fp32.
    x = _x((2, 6, 3, 32), seed=3).astype(np.float32)
    f = torch.polar(torch.ones(6, 16), torch.outer(torch.arange(6).float(), 1.0 / (10000.0 ** (torch.arange(0, 32, 2).float() / 32))))
    xt = torch.from_numpy(x)
    z = torch.view_as_complex(xt.reshape(*xt.shape[:-1], -1, 2))
    ref = torch.view_as_real(z * f.view(1, 6, 1, 16)).flatten(3).numpy()
    np.testing.assert_allclose(R.rope(x, f.numpy()), ref, rtol=1e-5, atol=1e-6)
    # and the oracle's own table follows the reference's precompute_freqs_cis (model.py:134-158)
    np.testing.assert_allclose(R.freqs_cis(32, 6), f.numpy(), rtol=1e-5, atol=1e-5)
