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


# ---- block_forward (run.py:102-117): the oracle pinned against the reference's Block and by the algebra
# of where each jitter enters

def _block_setup(layer, T=256, B=2):
    import torch
    from noise_amd.model import make_model
    from oracle.model import rotary_tables
    P = {k: v.float() for k, v in make_model('cpu', 0).state_dict().items()}
    pre = f'transformer.h.{layer}.'
    w = dict(q=P[pre + 'attn.c_q.weight'], k=P[pre + 'attn.c_k.weight'], v=P[pre + 'attn.c_v.weight'],
             gate=P.get(pre + 'attn.ve_gate.weight'), proj=P[pre + 'attn.c_proj.weight'],
             fc=P[pre + 'mlp.c_fc.weight'], out=P[pre + 'mlp.c_proj.weight'])
    # random residual-writer and gate weights: the pins below then do not depend on the init's values
    g = torch.Generator().manual_seed(layer)
    w['proj'] = torch.randn(512, 512, generator=g) * 0.02
    w['out'] = torch.randn(512, 2048, generator=g) * 0.02
    x = torch.randn(B, T, 512, generator=g)
    ve = torch.randn(B, T, 512, generator=g) if w['gate'] is not None else None
    if w['gate'] is not None:
        w['gate'] = torch.randn(8, 32, generator=g) * 0.3
    cos, sin = rotary_tables(T)
    return P, w, x, ve, cos, sin, g


def test_block_forward_without_jitter_is_the_models_block():
    import torch
    from oracle.model import _block
    for layer in (0, 1):
        P, w, x, ve, cos, sin, _ = _block_setup(layer)
        pre = f'transformer.h.{layer}.'
        P = dict(P)
        P[pre + 'attn.c_proj.weight'], P[pre + 'mlp.c_proj.weight'] = w['proj'], w['out']
        if ve is not None:
            P[pre + 'attn.ve_gate.weight'] = w['gate']
        ref = _block(P, layer, x, ve, cos, sin, 128)
        got = odust.block_forward(x, w, ve, cos, sin, 128)
        assert torch.allclose(got, ref, rtol=0, atol=1e-5)


def test_block_forward_jitter_placement():
    import torch
    P, w, x, ve, cos, sin, g = _block_setup(1)
    base = odust.block_forward(x, w, ve, cos, sin, 128)
    j = torch.randn(x.shape, generator=g) * 0.1
    # mlp: added to the block's last product, so to the output
    assert torch.allclose(odust.block_forward(x, w, ve, cos, sin, 128, mlp=j), base + j, rtol=0, atol=1e-5)
    # o: added before c_proj, so o = j Wproj^-T is attn = j
    o = torch.linalg.solve(w['proj'].double(), j.double().reshape(-1, 512).t()).t().reshape(x.shape).float()
    a1 = odust.block_forward(x, w, ve, cos, sin, 128, attn=j)
    a2 = odust.block_forward(x, w, ve, cos, sin, 128, o=o)
    assert torch.allclose(a1, a2, rtol=0, atol=2e-4)
    assert not torch.allclose(a1, base + j, rtol=0, atol=1e-3)  # the MLP sees the shifted residual
    # fc: added to the c_fc product, so fc = norm(x_mid) D^T is c_fc's weight + D
    w0 = dict(w, out=torch.zeros_like(w['out']))
    x_mid = odust.block_forward(x, w0, ve, cos, sin, 128)
    D = torch.randn(2048, 512, generator=g) * 0.01
    from oracle.model import norm
    f1 = odust.block_forward(x, w, ve, cos, sin, 128, fc=norm(x_mid) @ D.t())
    f2 = odust.block_forward(x, dict(w, fc=w['fc'] + D), ve, cos, sin, 128)
    assert torch.allclose(f1, f2, rtol=0, atol=1e-4)


def test_draw_errors_oracle_matches_the_reference_bf16_einsum():
    """oracle/dust.py:draw_errors against run.py:351-355 written as the reference writes it, with torch's own
    bf16 einsum on the CPU: errors[site] -= einsum('nbt,nbtd->btd', reward.to(bf16), a).float() / sigma.
    The einsum accumulates in fp32 and rounds its result to bf16, the oracle sums in float64 and rounds: the two
    agree exactly except where the sums straddle a bf16 rounding boundary (then by one ulp). Planting a
    dropped rounding (the reward left in fp32) breaks the agreement, so the check discriminates."""
    import torch
    rng = np.random.default_rng(7)
    n, b, t, d, sigma = 16, 2, 64, 32, 0.05
    reward = rng.normal(0, 0.3, size=(n, b, t)).astype(np.float32)
    a = torch.as_tensor(rng.choice([-1.0, 1.0], size=(n, b, t, d)).astype(np.float32)).bfloat16()
    errors = rng.normal(0, 1, size=(b, t, d))
    got = odust.draw_errors(errors, reward, a.float().numpy(), sigma)
    ref = torch.as_tensor(errors) - torch.einsum('nbt,nbtd->btd', torch.as_tensor(reward).bfloat16(),
                                                 a).double() / sigma
    e_got = (errors - got) * sigma
    e_ref = (errors - ref.numpy()) * sigma
    ulp = np.abs(e_ref) * 2.0 ** -7 + 1e-12
    assert (np.abs(e_got - e_ref) <= ulp).all()
    assert np.mean(np.abs(e_got - e_ref) <= 1e-9) > 0.99
    # mutation: without the reward's bf16 rounding the oracle would differ from the reference far more often
    e_fp32 = np.einsum('nbt,nbtd->btd', reward.astype(np.float64), a.float().numpy().astype(np.float64))
    e_fp32 = torch.as_tensor(e_fp32).float().bfloat16().double().numpy()
    assert np.mean(np.abs(e_fp32 - e_ref) > 1e-9) > 0.2


def test_rerun_oracle_reduces_to_the_clean_forward():
    """oracle/dust.py:capture + rerun (run.py:247-279) pinned against GPT.forward's own per-token losses
    (oracle/model.py:gpt_forward, itself pinned by the reference's outputs): with zero jitter every draw rerun
    from any entry -- the embedding or a cached block input -- reproduces the clean losses; a jitter at the
    entry block moves them."""
    import torch
    from noise_amd.model import make_model
    from oracle import model as om
    P = {k: v.float() for k, v in make_model('cpu', 0).state_dict().items()}
    P['lm_head.weight'] = P['lm_head.weight'] * 30
    g = torch.Generator().manual_seed(8)
    rows = torch.randint(0, 4096, (2, 257), generator=g)
    x, y = rows[:, :-1], rows[:, 1:]
    clean = om.gpt_forward(P, x, y, reduction='none').view(2, 256)
    cache = odust.capture(P, x)
    n = 2
    zero = {'transformer.wte': torch.zeros(n * 2, 256, 512)}
    for entry in (None, 0, 5, 7):
        got = odust.rerun(P, cache, y, n, entry, zero)
        assert got.shape == (n, 2, 256)
        assert (got - clean).abs().max().item() <= 1e-5, entry
    jit = {'o@5': 0.05 * torch.randn(n * 2, 256, 512, generator=g)}
    moved = odust.rerun(P, cache, y, n, 5, jit)
    assert (moved - clean).abs().max().item() > 1e-3


def test_chunk_size_is_the_largest_divisor():
    """run.py:76-78 by brute force: the largest n <= cap dividing draws; the product's and the oracle's agree."""
    from noise_amd.dust import chunk_size
    for draws in range(1, 65):
        for cap in range(1, 20):
            want = max(n for n in range(1, cap + 1) if draws % n == 0 and n <= draws)
            assert chunk_size(draws, cap) == want == odust.chunk_size(draws, cap), (draws, cap)
    with pytest.raises(ValueError):
        chunk_size(0, 4)


@pytest.mark.parametrize('gamma', [0.5, 0.9, 0.99])
def test_reward_to_go_closed_forms(gamma):
    """run.py:81-86: a unit impulse at token j gives gamma^(j - i) at every token i <= j within the lags (and 0
    elsewhere); a constant reward gives the truncated geometric sum (1 - gamma^m) / (1 - gamma),
    m = min(lags, t - i). The product's conv1d form (torch CPU) and the oracle's loop both match."""
    import math
    import torch
    from noise_amd.dust import reward_to_go
    t = 300
    lags = math.ceil(math.log(1e-6) / math.log(gamma))
    imp = np.zeros((2, 3, t))
    imp[1, 2, 250] = 1.0
    ones = np.ones((2, 3, t))
    i = np.arange(t)
    want_imp = np.where((i <= 250) & (250 - i < lags), gamma ** np.clip(250 - i, 0, None), 0.0)
    m = np.minimum(lags, t - i)
    want_ones = (1 - gamma ** m) / (1 - gamma)
    for fn, tol in ((odust.reward_to_go, 1e-12), (lambda r, g: reward_to_go(torch.from_numpy(r), g).numpy(), 1e-9)):
        got_imp, got_ones = fn(imp, gamma), fn(ones, gamma)
        assert np.abs(got_imp[1, 2] - want_imp).max() <= tol
        assert np.abs(got_imp[0]).max() == 0 and np.abs(got_imp[1, :2]).max() == 0
        assert np.abs(got_ones - want_ones).max() <= tol * lags


def _linear_case(d, draws, nrep, offset=0.0, prior_scale=None, mask=False, seed=0):
    """A loss that is linear in the jitter: loss_i = clean + sigma_bf a_i . g at every token (g per token), the
    oracle's direct_errors over its orthogonal draws (one site of width d). Returns (estimate, g, mask)."""
    import torch
    from oracle.orthogonal import OrthogonalDrawsOracle
    rng = np.random.default_rng(seed)
    b, t, sigma = 2, 8, 0.1
    g = rng.normal(size=(b, t, d))
    clean = rng.normal(size=(b, t)) + 8.0
    live = {}
    if mask:
        live['s'] = (rng.random((b, t, d)) > 0.5).astype(np.float64)
    draw = OrthogonalDrawsOracle(seed=seed)

    def rerun_fn(n, jitter):
        j = jitter['s'].double().numpy().reshape(n, b, t, d)
        return clean[None] + offset + np.einsum('nbtd,btd->nbt', j, g)

    priors = {'s': prior_scale * g} if prior_scale is not None else None
    est, _ = odust.direct_errors(draw, rerun_fn, clean, live, ['s'], {'s': d}, draws, sigma, nrep, priors=priors)
    return est['s'], g, live.get('s'), float(torch.tensor(sigma).bfloat16()) / sigma


def test_direct_errors_oracle_recovers_a_linear_gradient():
    """One full cycle of d orthogonal draws, one draw per rerun (no centring): sum_i a_i a_i^T = d I, so the
    estimate of a linear loss is its gradient g exactly, up to the bf16 rounding of each reward (2^-8 relative)
    and sigma's own bf16 rounding in the jitter (a fixed factor). With half of the units dead (masked), the dead
    units' estimates are exactly 0 and the live units' are the gradient of the masked loss."""
    for mask in (False, True):
        est, g, live, ratio = _linear_case(64, 64, 1, mask=mask)
        want = g * ratio * (live if mask else 1.0)
        err = np.abs(est - want).max()
        assert err <= 2 ** -7 * np.abs(g).sum(-1).max() / 8 + 1e-9, err
        if mask:
            assert np.all(est[live == 0] == 0)


def test_direct_errors_oracle_priors_and_centring():
    """A perfect prior (mu = g at sigma's bf16 ratio) leaves a zero residual reward, so the estimate is the prior
    itself; half a prior is completed by the draws. With n > 1 draws per rerun, a constant added to every
    perturbed loss cancels in the centring; with n = 1 it does not."""
    est, g, _, ratio = _linear_case(64, 64, 1, prior_scale=None)
    full, _, _, _ = _linear_case(64, 64, 1, prior_scale=ratio)
    assert np.abs(full - g * ratio).max() <= 2 ** -7 * np.abs(g).max() * 4
    half, _, _, _ = _linear_case(64, 64, 1, prior_scale=0.5 * ratio)
    assert np.abs(half - g * ratio).max() <= 2 ** -7 * np.abs(g).sum(-1).max() / 4 + 1e-9
    c0, _, _, _ = _linear_case(64, 64, 4)
    c1, _, _, _ = _linear_case(64, 64, 4, offset=0.37)
    assert np.abs(c1 - c0).max() <= 2 ** -6 * np.abs(c0).max()
    u0, _, _, _ = _linear_case(64, 64, 1)
    u1, _, _, _ = _linear_case(64, 64, 1, offset=0.37)
    assert np.abs(u1 - u0).max() > 0.01


def test_rerun_bf16_flow_reduces_to_the_fp32_rerun(monkeypatch):
    """The oracle's GPU-dtype-flow rerun (bf16 storage and stores, fp32 inside fused chains) is the fp32 rerun
    once its bf16 rounding is the identity; with rounding, every block output it produces is bf16-valued."""
    import torch
    import oracle.model as om
    from noise_amd.model import make_model
    P = {k: v.detach().float().clone() for k, v in make_model('cpu', 0).named_parameters()}
    P['lm_head.weight'] = P['lm_head.weight'] * 30
    g = torch.Generator().manual_seed(3)
    rows = torch.randint(0, 4096, (1, 257), generator=g)
    x, y = rows[:, :-1], rows[:, 1:]
    cache = odust.capture(P, x)
    jit = {'transformer.h.6.mlp.c_fc': (0.1 * (torch.randint(0, 2, (2, 256, 2048), generator=g) * 2 - 1)).bfloat16()}
    flow = odust.rerun_bf16_flow(P, cache, y, 2, 6, jit)
    with monkeypatch.context() as mp:
        mp.setattr(om, 'bf16', lambda t: t)
        ident = odust.rerun_bf16_flow(P, cache, y, 2, 6, jit)
    ref = odust.rerun(P, cache, y, 2, 6, jit)
    assert (ident - ref).abs().max().item() <= 1e-4
    assert (flow - ref).abs().max().item() > 1e-5        # the rounding matters
    from oracle.model import rotary_tables, window_sizes
    cos, sin = rotary_tables(256)
    out = odust.block_forward_bf16_flow(cache['blocks'][6].bfloat16().float(), odust.block_weights(P, 6), None, cos,
                                        sin, window_sizes()[6])
    assert torch.equal(out, out.bfloat16().float())


def test_rerun_batch_rows_are_cached_per_capture():
    # the tensors rerun derives from the captured batch (ids and targets repeated per draw, rotary tables, x0
    # repeated per draw) are built once per capture and n, and rebuilt when a source tensor is replaced or
    # changed in place, or n changes
    import torch
    from types import SimpleNamespace
    from noise_amd import dust as ndust
    T, b = 16, 2
    g = torch.Generator().manual_seed(0)
    model = SimpleNamespace(cos=torch.randn(1, 64, 1, 32, generator=g), sin=torch.randn(1, 64, 1, 32, generator=g))
    state = SimpleNamespace(model=model, length=T, x=torch.randint(0, 99, (b, T), generator=g),
                            y=torch.randint(0, 99, (b, T), generator=g), x0=torch.randn(b, T, 512, generator=g))
    r1 = ndust._batch_rows(state, 3, True)
    assert torch.equal(r1['idx'], state.x.repeat(3, 1)) and torch.equal(r1['targets'], state.y.repeat(3, 1))
    assert torch.equal(r1['x0'], state.x0.repeat(3, 1, 1))
    assert r1['rope'][0].shape == (T, 32) and r1['rope'][0].dtype == torch.bfloat16
    assert ndust._batch_rows(state, 3, True) is r1
    state.x0.mul_(2)  # in place: the version moves
    r2 = ndust._batch_rows(state, 3, True)
    assert r2 is not r1 and torch.equal(r2['x0'], state.x0.repeat(3, 1, 1))
    state.y = state.y.clone()  # another tensor with the same values
    r3 = ndust._batch_rows(state, 3, True)
    assert r3 is not r2
    r4 = ndust._batch_rows(state, 4, True)
    assert r4 is not r3 and r4['idx'].shape == (4 * b, T)
    assert ndust._batch_rows(state, 4, False)['x0'] is None
