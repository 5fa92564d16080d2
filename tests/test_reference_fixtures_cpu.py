"""The oracle and the product's model init against vectors the reference's own code wrote
(tests/golden/make_reference_fixtures.py, run in the build container from /root/reference)."""
import hashlib
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import model as om

GOLDEN = Path(__file__).resolve().parent / 'golden'
sys.path.insert(0, str(GOLDEN))
from make_reference_fixtures import population_inputs  # noqa: E402


@pytest.fixture(scope='module')
def fx():
    return np.load(GOLDEN / 'reference_fixtures.npz', allow_pickle=False)


@pytest.fixture(scope='module')
def params():
    from noise_amd.model import make_model
    return make_model('cpu', 0).state_dict()


def test_seed0_init_is_bit_identical(fx, params):
    """make_model('cpu', 0): every tensor's fp32 bytes equal the reference's (eggroll.py:38-53)."""
    names = [str(n) for n in fx['init_names']]
    assert names == list(params.keys())
    for n, h in zip(names, fx['init_sha256']):
        got = hashlib.sha256(params[n].float().contiguous().numpy().tobytes()).hexdigest()
        assert got == str(h), n


def test_oracle_forward_matches_reference(fx, params):
    """GPT.forward (model.py:193-209): the oracle's fp32 dense-attention forward vs the reference's flex
    forward on the same inputs, at init and with the head x30."""
    P = {k: v.float() for k, v in params.items()}
    seqs = torch.from_numpy(fx['fwd_seqs'])
    x, y = seqs[:, :-1], seqs[:, 1:]
    assert abs(om.gpt_forward(P, x, y).item() - float(fx['fwd_loss_init'])) < 2e-5
    P['lm_head.weight'] = P['lm_head.weight'] * 30
    assert abs(om.gpt_forward(P, x, y).item() - float(fx['fwd_loss_head30'])) < 2e-5


def test_oracle_population_matches_reference(fx, params):
    """population_loss (eggroll.py:66-103) with noise on all 60 parameters, head x30."""
    P = {k: v.float() for k, v in params.items()}
    P['lm_head.weight'] = P['lm_head.weight'] * 30
    shapes = {n: tuple(v.shape) for n, v in params.items()}
    flat, sign, idx = population_inputs(shapes)
    noise = {n: (tuple(t.repeat_interleave(2, 0) for t in rows.split(list(shapes[n]), dim=1))
                 if len(shapes[n]) == 2 else rows.repeat_interleave(2, 0)) for n, rows in flat.items()}
    assert torch.equal(sign, torch.from_numpy(fx['pop_sign'])) and torch.equal(idx, torch.from_numpy(fx['pop_idx']))
    got = om.population_loss(P, noise, sign, idx[:-1], idx[1:])
    ref = torch.from_numpy(fx['pop_losses'])
    assert (got - ref).abs().max() < 2e-5, (got, ref)
