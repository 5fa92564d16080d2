"""EGGROLL's update reassembly (eggroll.py:151-165) on the CPU: the oracle pinned by closed forms, torch
library routines and algebraic invariants; the C ABI's argument checks (no GPU needed)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import update as oupdate
from oracle import noise as onoise

DRAW = (0, 0, 2 ** 19)  # the reference buffer's draw on MI355X: seed 0, offset 0, 2^19 threads


def test_fitness_weights_closed_form():
    # members 4, pairs 2: fitness [1, 3], unbiased std sqrt(2)
    w = oupdate.fitness_weights([0.0, 1.0, 0.0, 3.0], 2)
    s = np.float32(np.sqrt(2.0)) + np.float32(1e-8)
    assert np.allclose(w, [1.0 / s, 3.0 / s], rtol=1e-7, atol=0)


def test_fitness_weights_match_torch_library():
    # eggroll.py:151-154 with torch's own std and index_add_ (members > 2 pairs: directions repeat)
    g = torch.Generator().manual_seed(5)
    losses = 8.3 + 0.01 * torch.randn(48, generator=g)
    pairs = 8
    fitness = losses[1::2] - losses[0::2]
    fitness = fitness / (fitness.std() + 1e-8)
    ref = torch.zeros(pairs).index_add_(0, torch.arange(len(fitness)) % pairs, fitness)
    got = oupdate.fitness_weights(losses.numpy(), pairs)
    assert np.allclose(got, ref.double().numpy(), rtol=1e-5, atol=1e-6)


def test_one_direction_is_an_outer_product():
    # weight = e_d: the gradient is scale * a_d b_d^T with a_d = the first `rows` elements of the slice
    offsets = {'m': np.array([123456, 77], dtype=np.int64)}
    g = oupdate.gradients_from_weights([0.0, 1.0], offsets, {'m': (3, 5)}, DRAW, -0.5)['m']
    s = onoise.randn(*DRAW, np.arange(77, 77 + 8)).astype(np.float64)
    assert g.shape == (3, 5)
    assert np.array_equal(g, -0.5 * np.outer(s[:3], s[3:]))


def test_one_dimensional_parameters_sum_their_slices():
    offsets = {'v': np.array([10, 1000, 5], dtype=np.int64)}
    w = np.array([0.5, -2.0, 1.0])
    g = oupdate.gradients_from_weights(w, offsets, {'v': (8,)}, DRAW, 1.0)['v']
    rows = [onoise.randn(*DRAW, np.arange(o, o + 8)).astype(np.float64) for o in offsets['v']]
    assert np.allclose(g, sum(wi * r for wi, r in zip(w, rows)), rtol=1e-14, atol=1e-14)


def test_gradient_is_linear_in_the_weights():
    offsets = {'m': np.array([0, 4096, 99999, 12], dtype=np.int64), 'v': np.array([7, 8, 9, 10], dtype=np.int64)}
    shapes = {'m': (6, 4), 'v': (3,)}
    w1, w2 = np.array([1.0, -0.5, 0.25, 2.0]), np.array([-1.5, 0.0, 3.0, 0.5])
    g1 = oupdate.gradients_from_weights(w1, offsets, shapes, DRAW, 1.0)
    g2 = oupdate.gradients_from_weights(w2, offsets, shapes, DRAW, 1.0)
    g12 = oupdate.gradients_from_weights(w1 + w2, offsets, shapes, DRAW, 1.0)
    for n in shapes:
        assert np.allclose(g12[n], g1[n] + g2[n], rtol=1e-12, atol=1e-12)


def test_update_is_minus_weighted_mean_over_fitness_count():
    # p.grad = -(sum_d w_d a_d b_d^T) / len(fitness) (eggroll.py:160, 165)
    losses = np.array([1.0, 2.0, 3.0, 1.0, 0.5, 0.25], dtype=np.float32)
    offsets = {'m': np.array([5, 500, 50000], dtype=np.int64)}
    g = oupdate.update_gradients(losses, 3, offsets, {'m': (2, 2)}, DRAW)['m']
    w = oupdate.fitness_weights(losses, 3)
    ref = oupdate.gradients_from_weights(w, offsets, {'m': (2, 2)}, DRAW, 1.0)['m']
    assert np.allclose(g, -ref / 3, rtol=1e-14, atol=0)


# ---- C ABI argument checks (rejected on the host, before any HIP call) ----

@pytest.fixture(scope='module')
def lib():
    from noise_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail(f'{_lib.LIB_PATH} is not built (run __graft_entry__.build())')
    return _lib


def _params(lib, shapes):
    arr = (lib.UpdateParam * len(shapes))()
    for i, (r, c) in enumerate(shapes):
        arr[i] = lib.UpdateParam(16, 16, r, c)  # aligned dummy device addresses: never dereferenced here
    return arr


def test_update_workspace_bytes(lib):
    arr = _params(lib, [(512, 512), (2048, 512), (8, 32), (8, 0)])
    # big parameters only: (rows + cols) * 2 (the hi and lo halves) * chunk (rounded up to 256) bf16, then the
    # GEMM's partial tiles: 4 + 16 tiles of 256 x 256 fill a 256-CU device split in 4 (fp32)
    partials = (4 + 16) * 4 * 256 * 256 * 4
    assert lib.lib().noise_update_workspace_bytes(arr, 4, 1000, 300) == (1024 + 2560) * 2 * 512 * 2 + partials
    assert lib.lib().noise_update_workspace_bytes(arr, 4, 64, 4096) == (1024 + 2560) * 2 * 256 * 2 + partials
    assert lib.lib().noise_update_workspace_bytes(arr, 4, 0, 256) == -1


def test_update_invalid_arguments(lib):
    L = lib.lib()
    err = lambda: L.noise_last_error().decode()
    assert L.noise_update_weights(16, 3, 2, 16, None) == -1 and 'even' in err()
    assert L.noise_update_weights(16, 2, 1, 16, None) == -1 and '>= 4' in err()
    arr = _params(lib, [(300, 300)])
    st = L.noise_update_gradients(arr, 1, 64, 16, -1.0, 256, 2 ** 28, 0, 0, 2 ** 19, None, None, 0, None)
    assert st == -1 and 'neither a multiple of 256' in err()
    arr = _params(lib, [(512, 512)])
    st = L.noise_update_gradients(arr, 1, 64, 16, -1.0, 256, 2 ** 28, 0, 0, 2 ** 19, None, None, 0, None)
    assert st == -1 and 'workspace' in err()
    st = L.noise_update_gradients(arr, 1, 64, 16, -1.0, 256, 2 ** 28, 0, 2, 2 ** 19, None, None, 0, None)
    assert st == -1 and 'multiple of 4' in err()
    arr = _params(lib, [(512, 512)] * 65)
    st = L.noise_update_gradients(arr, 65, 64, 16, -1.0, 256, 2 ** 28, 0, 0, 2 ** 19, None, None, 0, None)
    assert st == -1 and '64 parameters' in err()
