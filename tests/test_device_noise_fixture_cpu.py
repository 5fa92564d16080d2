"""The oracle's draw layout against values torch-ROCm's own device generator produced on an MI355X
(tests/golden/make_device_noise_fixture.py): step-0 Eggroll offsets exactly; elements of the seed-0 randn
buffer to within the host-libm vs device-intrinsic Box-Muller difference (a few ulp)."""
from pathlib import Path

import numpy as np
import pytest

from oracle import noise as on

GOLDEN = Path(__file__).resolve().parent / 'golden'


@pytest.fixture(scope='module')
def fx():
    on.build()
    return np.load(GOLDEN / 'device_noise_fixture.npz', allow_pickle=False)


def test_fixture_device(fx):
    assert int(fx['cus']) == 256 and int(fx['max_threads']) == 2048


def test_offsets_exact(fx):
    """Eggroll.offsets(0) (eggroll.py:117-120): 60 randint draws of 512 on one generator, in
    named_parameters order; the oracle's closed form reproduces every value."""
    from noise_amd.model import make_model
    params = dict(make_model('cpu', 0).named_parameters())
    assert [str(n) for n in fx['param_names']] == list(params)
    g = on.OracleGenerator(0, int(fx['cus']), int(fx['max_threads']))
    for i, p in enumerate(params.values()):
        got = g.randint(0, 2 ** 28 - sum(p.shape), 512)
        assert np.array_equal(got, fx['offsets'][i].astype(np.int64)), i


def test_buffer_elements_within_ulps(fx):
    """torch.randn(2**28) on the device (eggroll.py:114) at fixed and random indices, incl. both ends
    and a thread-plane boundary: the oracle's host Box-Muller is within 2e-6 relative (+1e-6 absolute)."""
    S = on.grid_threads(2 ** 28, int(fx['cus']), int(fx['max_threads']))
    assert S == 2 ** 19
    got = on.randn(0, 0, S, fx['buffer_idx'])
    ref = fx['buffer_val']
    assert np.all(np.abs(got - ref) <= 2e-6 * np.abs(ref) + 1e-6)
    # a wrong lane / thread mapping is off by O(1), not by ulps
    shifted = on.randn(0, 0, S, fx['buffer_idx'] + 1)
    assert np.mean(np.abs(shifted - ref) > 1e-3) > 0.9


def test_zipf_token_fixture():
    """The benchmark's tokens: 2049 ids ~ Zipf(1.1) over [0, 4096) from torch.multinomial, CPU seed 0."""
    import sys
    sys.path.insert(0, str(GOLDEN.parent.parent))
    from bench import zipf_tokens
    tok = np.load(GOLDEN / 'zipf_tokens_2049_seed0.npy', allow_pickle=False)
    assert tok.shape == (2049,) and tok.min() >= 0 and tok.max() < 4096
    assert np.array_equal(zipf_tokens(2049).numpy(), tok)
    assert np.bincount(tok, minlength=4096)[0] > np.bincount(tok, minlength=4096)[100]
