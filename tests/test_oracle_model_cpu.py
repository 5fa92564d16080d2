"""Pins the fp32 oracle restatement (oracle/model.py) on the CPU, with checks a plausible mistake fails:
library routines (torch SDPA, F.cross_entropy, F.rms_norm), closed forms, brute force on tiny shapes and
the invariants of the population forward (sigma = 0 equality, antithetic second order, init loss)."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import model as om


def test_attention_full_window_is_causal_sdpa():
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 96, 3, 64, generator=g) for _ in range(3))
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True)
    assert torch.allclose(om.attention(q, k, v, 96), ref.transpose(1, 2), atol=1e-5)


def test_attention_window_is_banded_sdpa():
    """Window w: query s sees keys s-w .. s (model.py:20); the band mask via SDPA's attn_mask."""
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 80, 2, 64, generator=g) for _ in range(3))
    i, j = torch.arange(80)[:, None], torch.arange(80)[None, :]
    mask = (i >= j) & (i - j <= 7)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), attn_mask=mask)
    assert torch.allclose(om.attention(q, k, v, 7), ref.transpose(1, 2), atol=1e-5)
    assert torch.allclose(om.attention(q, k, v, 0), v, atol=1e-6)


def test_norm_is_rms_norm_with_fp32_eps():
    x = torch.randn(5, 512) * 3
    ref = x / torch.sqrt((x * x).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps)
    assert torch.allclose(om.norm(x), ref, rtol=1e-6, atol=1e-6)


def test_rotary_convention():
    """Position 0 is the identity; at position t the pair (x_i, x_{i+32}) = (1, 0) maps to
    (cos t w_i, -sin t w_i) (model.py:58's sign), with w_i = 10000^(-i/32); norms are preserved."""
    cos, sin = om.rotary_tables(8)
    x = torch.zeros(1, 8, 1, 64)
    x[..., 3] = 1.0
    y = om.apply_rotary_emb(x, cos, sin)
    assert torch.equal(y[0, 0, 0], x[0, 0, 0])
    w = 10000 ** (-3 / 32)
    t = 5
    assert abs(y[0, t, 0, 3] - math.cos(t * w)) < 1e-2 and abs(y[0, t, 0, 35] + math.sin(t * w)) < 1e-2
    z = torch.randn(2, 8, 4, 64)
    yz = om.apply_rotary_emb(z, cos, sin)
    pair = lambda a: (a[..., :32] ** 2 + a[..., 32:] ** 2)
    assert torch.allclose(pair(yz), pair(z) * (cos ** 2 + sin ** 2)[None, :, None, :], rtol=1e-5, atol=1e-6)
    # tables are the bf16 rounding of fp32 cos / sin
    assert torch.equal(cos, cos.bfloat16().float())


def test_lowrank_equals_materialised_perturbation():
    g = torch.Generator().manual_seed(2)
    m, T, n_in, n_out = 3, 7, 16, 12
    x = torch.randn(m, T, n_in, generator=g)
    W = torch.randn(n_out, n_in, generator=g)
    a, b = torch.randn(m, n_out, generator=g), torch.randn(m, n_in, generator=g)
    s = torch.tensor([0.3, -0.3, 0.7])
    y = om.lowrank(x, W, a, b, s)
    for i in range(m):
        Wi = W + s[i] * torch.outer(a[i], b[i])
        assert torch.allclose(y[i], x[i] @ Wi.t(), atol=1e-5)
    E = torch.randn(20, 16, generator=g)
    idx = torch.tensor([3, 0, 19, 3])
    ae, be = torch.randn(m, 20, generator=g), torch.randn(m, 16, generator=g)
    ye = om.lowrank_embed(E, ae, be, idx, s)
    for i in range(m):
        assert torch.allclose(ye[i], (E + s[i] * torch.outer(ae[i], be[i]))[idx], atol=1e-6)


def test_softcap_ce_is_cross_entropy_of_capped_logits():
    g = torch.Generator().manual_seed(3)
    z = torch.randn(10, 4096, generator=g) * 20
    y = torch.randint(0, 4096, (10,), generator=g)
    y[2] = -1
    capped = 15 * torch.tanh(z / 15)
    ref = F.cross_entropy(capped, y, ignore_index=-1, reduction='none')
    out = om.softcap_ce(z, y, 'none')
    assert torch.allclose(out, ref) and out[2] == 0
    # logits ~ 0 => CE ~ ln V
    assert abs(om.softcap_ce(torch.zeros(1, 4096), torch.tensor([5]), 'none').item() - math.log(4096)) < 1e-6


def test_hadamard_is_orthogonal_sylvester():
    H = om.hadamard(64)
    assert torch.equal(H @ H.t(), 64 * torch.eye(64))
    i, j = torch.arange(64)[:, None], torch.arange(64)[None, :]
    pop = torch.tensor([[bin(int(a) & int(b)).count('1') for b in range(64)] for a in range(64)])
    assert torch.equal(H, (1 - 2 * (pop % 2)).float())
    with pytest.raises(ValueError):
        om.hadamard(48)


@pytest.fixture(scope='module')
def params():
    from noise_amd.model import make_model
    return {k: v.float() for k, v in make_model('cpu', 0).state_dict().items()}


def test_make_model_shapes_and_distributions(params):
    """utils/model.py:123-175 + eggroll.py:45-49: 37,749,776 parameters; the drawn distributions."""
    assert sum(v.numel() for k, v in params.items()) == 37_749_776
    assert abs(params['transformer.wte.weight'].std().item() - 1.0) < 0.01
    assert abs(params['lm_head.weight'].std().item() - 0.001) < 1e-4
    s = 3 ** 0.5 * 512 ** -0.5
    assert params['transformer.h.0.attn.c_q.weight'].abs().max() <= s
    assert params['transformer.h.0.attn.c_proj.weight'].abs().max() <= 1.5 * (3 / 512) ** 0.5
    assert params['transformer.h.0.mlp.c_proj.weight'].abs().max() <= 1.5 * (3 / 2048) ** 0.5
    assert params['transformer.h.0.mlp.c_proj.weight'].abs().max() > 0.9 * 1.5 * (3 / 2048) ** 0.5  # re-drawn, not zero
    assert torch.equal(params['resid_lambdas'], torch.ones(8)) and torch.allclose(params['x0_lambdas'], torch.full((8,), 0.1))
    assert (params['transformer.h.1.attn.ve_gate.weight'] == 0).all()
    assert sorted(k for k in params if k.startswith('value_embeds')) == [f'value_embeds.{i}.weight' for i in (1, 3, 5, 7)]


def test_window_sizes():
    assert om.window_sizes() == [1024, 1024, 1024, 2048, 1024, 1024, 1024, 2048]
    assert [i for i in range(8) if om.has_ve(i)] == [1, 3, 5, 7]


def test_population_sigma_zero_equals_forward(params):
    """sigma = 0: every member's loss is GPT.forward's mean CE (eggroll.py:66-103 vs model.py:193-209)."""
    P = dict(params)
    P['lm_head.weight'] = params['lm_head.weight'] * 30
    g = torch.Generator().manual_seed(4)
    idx = torch.randint(0, 4096, (129,), generator=g)
    noise = {'transformer.h.2.mlp.c_fc.weight': (torch.randn(2, 2048, generator=g), torch.randn(2, 512, generator=g))}
    pop = om.population_loss(P, noise, torch.zeros(2), idx[:-1], idx[1:])
    ref = om.gpt_forward(P, idx[None, :-1], idx[None, 1:])
    assert torch.allclose(pop, ref.expand(2), atol=1e-5)
    assert abs(ref.item() - math.log(4096)) > 0.05


def test_population_antithetic_expansion(params):
    """L(+s) - L(-s) = 2 s L' + O(s^3): halving sigma halves it; the even part L(+s) + L(-s) - 2 L(0) = O(s^2)
    is negligible next to it at small sigma (a dropped or mis-signed rank-1 term breaks one of these)."""
    P = dict(params)
    P['lm_head.weight'] = params['lm_head.weight'] * 30
    g = torch.Generator().manual_seed(5)
    idx = torch.randint(0, 4096, (65,), generator=g)
    n = 'transformer.h.1.attn.c_v.weight'
    a, b = torch.randn(1, 512, generator=g), torch.randn(1, 512, generator=g)
    noise = {n: (a.repeat(3, 1), b.repeat(3, 1))}

    def terms(s):
        L = om.population_loss(P, noise, torch.tensor([s, -s, 0.0]), idx[:-1], idx[1:]).double()
        return (L[0] + L[1] - 2 * L[2]).item(), (L[0] - L[1]).item()

    c1, d1 = terms(0.008)
    c2, d2 = terms(0.004)
    assert abs(d1) > 1e-3
    assert abs(d2 / d1 - 0.5) < 0.03
    assert abs(c2) < 0.01 * abs(d2)


def test_init_loss_is_ln_vocab(params):
    """Seed-0 init: logits ~ 0 (head std 0.001), so every member's loss ~ ln 4096."""
    g = torch.Generator().manual_seed(6)
    idx = torch.randint(0, 4096, (65,), generator=g)
    L = om.population_loss(params, {}, torch.zeros(1), idx[:-1], idx[1:])
    assert abs(L.item() - math.log(4096)) < 5e-3


def test_head_loss_matches_forward_head(params):
    """run.py:89-94 on the final hidden state equals GPT.forward's per-token CE path."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 16, 512, generator=g)
    W = torch.randn(4096, 512, generator=g) * 0.1
    y = torch.randint(0, 4096, (2, 16), generator=g)
    ref = F.cross_entropy((15 * torch.tanh((om.norm(x) @ W.t()) / 15)).flatten(0, 1), y.flatten(), reduction='none')
    assert torch.allclose(om.head_loss(x, W, y), ref, atol=1e-5)
