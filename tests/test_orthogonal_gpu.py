"""Orthogonal draws on the device (noise_orthogonal_draws + OrthogonalDraws) and the population variant
with orthogonal antithetic pairs and the fp32 head (2048 members x 2048 tokens).

Bit-exact bar: the device draws equal (1) the reference's own algorithm (run.py:143-152, 218-238) run
with torch-ROCm's randint on cuda generators, and (2) the CPU oracle. Loss bar: per-member mean CE within
1e-3 of the fp32 CPU oracle."""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def torch_orthogonal(seed, rank, world, calls):
    """run.py:143-152, 218-238 restated with torch ops on the GPU's own generators (fp32 draws)."""
    gen = torch.Generator(DEV).manual_seed(seed + 3 + 7777 * rank)
    shared = torch.Generator(DEV).manual_seed(seed + 5)
    frames, outs = {}, []

    def hadamard(d):
        H = torch.ones(1, 1, device=DEV)
        while H.shape[0] < d:
            H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
        return H

    def signs(*shape, use_shared=False):
        g = shared if use_shared else gen
        return torch.randint(0, 2, shape, device=DEV, generator=g).to(torch.float32) * 2 - 1

    for site, draws, chunk, n, b, t, d in calls:
        if site not in frames:
            cycles = -(-world * draws // d)
            frames[site] = (signs(cycles, d, use_shared=True),
                            torch.randint(0, d, (b, t), device=DEV, generator=shared))
        patterns, offset = frames[site]
        index = rank * draws + chunk * n + torch.arange(n, device=DEV)
        rows = (offset.unsqueeze(0) + index[:, None, None]) % d
        outs.append(hadamard(d)[rows] * patterns[index // d][:, None, None, :] * signs(n, b, t, 1))
    return outs


# (site, draws, chunk, n, b, t, d); every call stays within its site's draws (chunk * n + n <= draws), as
# the reference's callers split a step's draws into chunks
# the calls cover both kernels (8 <= d <= 2048: eight coordinates per thread; d = 4: one per thread), frames longer
# than one workgroup's rows (300 x 8 positions at d = 512), draws across pattern cycles and d = 8, 16
CALLS = [('q', 2048, 0, 1024, 1, 1, 512), ('k', 4096, 0, 1024, 1, 1, 2048), ('q', 2048, 1, 1024, 1, 1, 512),
         ('tok', 48, 0, 16, 2, 64, 512), ('tok', 48, 1, 16, 2, 64, 512), ('small', 3, 0, 3, 1, 5, 4),
         ('wide', 4096, 1, 2048, 2, 3, 2048), ('frame', 64, 1, 32, 8, 300, 512), ('d8', 32, 0, 32, 3, 7, 8),
         ('d16', 48, 1, 24, 4, 40, 16)]


def test_calls_are_valid():
    for site, draws, chunk, n, b, t, d in CALLS:
        assert chunk * n + n <= draws, site


@pytest.mark.parametrize('seed,rank,world', [(0, 0, 1), (7, 1, 2)])
def test_device_draws_match_torch_generators(seed, rank, world):
    from noise_amd.noise import OrthogonalDraws
    ref = torch_orthogonal(seed, rank, world, CALLS)
    od = OrthogonalDraws(seed, rank, world, DEV)
    for call, r in zip(CALLS, ref):
        got = od(*call)
        assert torch.equal(got, r), f'call {call}'


def test_device_draws_match_oracle_and_bf16():
    from noise_amd.noise import OrthogonalDraws
    from oracle.orthogonal import OrthogonalDrawsOracle
    od, oo = OrthogonalDraws(3, 0, 1, DEV), OrthogonalDrawsOracle(3, 0, 1)
    for call in CALLS:
        got = od(*call, dtype=torch.bfloat16)
        assert got.dtype == torch.bfloat16
        assert np.array_equal(got.float().cpu().numpy(), oo(*call)), f'call {call}'


def test_invalid_width_and_cycles():
    from noise_amd import _lib
    from noise_amd.noise import OrthogonalDraws
    with pytest.raises(ValueError, match='power-of-two'):
        OrthogonalDraws(0, 0, 1, DEV)('x', 4, 0, 4, 1, 1, 96)
    with pytest.raises(ValueError, match='beyond'):
        OrthogonalDraws(0, 0, 1, DEV)('x', 4, 1, 4, 1, 1, 8)
    z = torch.zeros(8, dtype=torch.int64, device=DEV)
    out = torch.empty(8, device=DEV)
    with pytest.raises(RuntimeError, match='cycles'):
        _lib.call('noise_orthogonal_draws', _lib.ptr(out), 0, 2, 1, 4, 3, _lib.ptr(z), _lib.ptr(z), 1, _lib.ptr(z),
                  _lib.stream_ptr(DEV))


@pytest.fixture(scope='module')
def config5():
    """2048 members (1024 orthogonal antithetic pairs) x 2048 Zipf(1.1) tokens, seed-0 init with the head
    scaled x30 (logits of order 1, so the blocks move the loss), block matrices perturbed (sigma 0.002),
    fp32 head (split-bf16x3)."""
    from pathlib import Path
    from noise_amd.eggroll import Weights, block_matrix_shapes, orthogonal_directions, orthogonal_population
    from noise_amd.model import make_model
    P = {k: v.float() for k, v in make_model('cpu', 0).state_dict().items()}
    P['lm_head.weight'] = P['lm_head.weight'] * 30
    toks = torch.from_numpy(np.load(Path(__file__).resolve().parent / 'golden' / 'zipf_tokens_2049_seed0.npy')).long()
    x, y = toks[:-1].to(DEV), toks[1:].to(DEV)
    shapes = block_matrix_shapes(P)
    noise = orthogonal_directions(shapes, 1024, seed=0, device=DEV)
    W = Weights({k: v.to(DEV) for k, v in P.items()}, fp32_head=True)
    losses = orthogonal_population(W, noise, x, y, sigma=0.002, chunk=1024)
    return P, shapes, noise, W, x, y, losses


def test_config5_population_vs_oracle(config5):
    """Members 0, 1, 1022-1025 (the two sides of the 1024-member chunk boundary) and 2046, 2047 of the full
    2048-member run against the fp32 CPU oracle within 1e-3; the same members evaluated alone give
    bit-identical losses (members are independent)."""
    from noise_amd.eggroll import orthogonal_population
    from oracle import model as om
    from oracle.orthogonal import orthogonal_directions as oracle_dirs
    P, shapes, noise, W, x, y, losses = config5
    assert losses.shape == (2048,) and torch.isfinite(losses).all()
    dirs = torch.tensor([0, 511, 512, 1023])
    members = torch.tensor([0, 1, 1022, 1023, 1024, 1025, 2046, 2047])
    sub = orthogonal_population(W, noise, x, y, sigma=0.002, directions=dirs)
    assert torch.equal(sub, losses[members.to(DEV)])
    # the oracle draws its own directions (bit-exact twin), then the fp32 population loss
    on = oracle_dirs(shapes, 1024, seed=0)
    for name in shapes:
        assert np.array_equal(noise[name][0].cpu().numpy(), on[name][0])
    onoise = {n: (torch.from_numpy(a[dirs.numpy()]).repeat_interleave(2, 0),
                  torch.from_numpy(b[dirs.numpy()]).repeat_interleave(2, 0)) for n, (a, b) in on.items()}
    sign = torch.tensor([0.002, -0.002]).repeat(4)
    ref = om.population_loss(P, onoise, sign, x.cpu(), y.cpu(), members_per_chunk=2)
    err = (sub.cpu() - ref).abs().max().item()
    print(f'config 5 members {members.tolist()}: max |loss - oracle| = {err:.3e}, loss {ref.mean().item():.4f}')
    assert err <= 1e-3
    assert abs(ref.mean().item() - math.log(4096)) > 0.05, 'scaled head must move the loss off ln V'


def test_config5_antithetic_structure(config5):
    """Fitness L[2i+1] - L[2i] is nonzero and of both signs over the population; pairs differ only by the
    sign of sigma."""
    losses = config5[-1].cpu()
    fit = losses[1::2] - losses[0::2]
    assert (fit > 0).any() and (fit < 0).any()
    assert fit.abs().max() > 1e-4
