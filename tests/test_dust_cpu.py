"""DUST's head error (run.py:121-137, 380-389) on the CPU: the oracle pinned by brute force (the full
soft-capped cross-entropy recomputed with one logit moved) and by the sigma -> 0 limit (the exact
derivative (softmax - onehot) * cap'), and the C ABI's argument checks."""
import numpy as np
import pytest

from oracle import dust as odust


def _ce(raw, y):
    z = odust.softcap(raw)
    m = z.max()
    return m + np.log(np.exp(z - m).sum()) - z[y]


def test_closed_form_matches_brute_force():
    rng = np.random.default_rng(0)
    raw = rng.normal(0, 6, size=(5, 8))
    y = np.array([3, 0, 7, -1, 5])
    sigma = 0.1
    got = odust.coordinate_differences(raw, y, sigma)
    for r in range(5):
        for j in range(8):
            if y[r] < 0:
                assert got[r, j] == 0.0
                continue
            upv, dnv = raw[r].copy(), raw[r].copy()
            upv[j] += sigma
            dnv[j] -= sigma
            ref = (_ce(upv, y[r]) - _ce(dnv, y[r])) / (2 * sigma)
            assert abs(got[r, j] - ref) < 1e-12, (r, j, got[r, j], ref)


def test_small_sigma_limit_is_the_derivative():
    rng = np.random.default_rng(1)
    raw = rng.normal(0, 5, size=(3, 64))
    y = np.array([0, 17, 63])
    z = odust.softcap(raw)
    w = np.exp(z - z.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    onehot = np.zeros_like(w)
    onehot[np.arange(3), y] = 1
    deriv = (w - onehot) * (1 - np.tanh(raw / 15) ** 2)
    got = odust.coordinate_differences(raw, y, 1e-4)
    assert np.abs(got - deriv).max() < 1e-7


def test_head_error_pads_with_zeros():
    raw = np.random.default_rng(2).normal(size=(2, 4, 12))
    y = np.array([[1, 2, 3, -1], [0, 0, 9, 9]])
    got = odust.head_error(raw, y, 10, 0.1)
    assert np.all(got[..., 10:] == 0) and np.all(got[0, 3] == 0)
    assert np.allclose(got[..., :10], odust.coordinate_differences(raw[..., :10], y, 0.1), rtol=0, atol=0)


def test_coordinate_differences_invalid_arguments():
    from noise_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail('libnoise_amd.so is not built')
    L = _lib.lib()
    assert L.noise_coordinate_differences(16, 1, 4, 4096, 4096, 16, 0.1, 16, 4000, 4096, None) == -1
    assert 'out_width' in L.noise_last_error().decode()
    assert L.noise_coordinate_differences(16, 1, 4, 4096, 4096, 16, 0.0, 16, 4096, 4096, None) == -1
    assert 'sigma' in L.noise_last_error().decode()
