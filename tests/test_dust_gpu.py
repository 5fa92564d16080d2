"""DUST's head error on the GPU (noise_coordinate_differences through the C ABI) against the float64
oracle (oracle/dust.py). The kernel computes in fp32 as the reference's torch ops do; the moved logits'
differences z' - z (about sigma) carry fp32 rounding of the capped values (~2e-6), so entries agree to
5e-5 absolute (entries are O(1))."""
import numpy as np
import pytest
import torch

from oracle import dust as odust

pytestmark = pytest.mark.gpu
ATOL = 5e-5


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_head_error_matches_oracle(dtype):
    from noise_amd.dust import head_error
    g = torch.Generator().manual_seed(0)
    logits = (torch.randn(2, 512, 4096, generator=g) * 5).to(dtype)
    y = torch.randint(0, 4000, (2, 512), generator=g)
    y[0, :7] = -1
    y[1, 100] = 3999
    got = head_error(logits.cuda(), y.cuda(), 4000, 0.1).cpu().numpy()
    ref = odust.head_error(logits.float().numpy(), y.numpy(), 4000, 0.1)
    err = float(np.abs(got - ref).max())
    print(dtype, 'max abs err', err, flush=True)
    assert got.shape == (2, 512, 4096)
    assert np.all(got[..., 4000:] == 0) and np.all(got[0, :7] == 0)
    assert err <= ATOL


def test_coordinate_differences_sum_rule():
    # sum_j of the exact derivative (softmax - onehot) * cap' has no closed form, but a token whose logits
    # are all equal has cap' equal everywhere and softmax uniform: the row sums to 0 up to O(sigma^2)
    from noise_amd.dust import coordinate_differences
    raw = torch.full((64, 4096), 2.5, dtype=torch.float32)
    y = torch.arange(64) * 61
    got = coordinate_differences(raw.cuda(), y.cuda(), 0.01).cpu().double()
    assert float(got.sum(-1).abs().max()) < 1e-4
    ref = odust.coordinate_differences(raw.numpy(), y.numpy(), 0.01)
    assert float(np.abs(got.numpy() - ref).max()) <= ATOL


def _block_case(layer, seed, B=2, T=2048):
    from noise_amd.model import make_model, window_sizes
    from oracle.model import rotary_tables
    P = {k: v.float() for k, v in make_model('cpu', 0).state_dict().items()}
    pre = f'transformer.h.{layer}.'
    g = torch.Generator().manual_seed(seed)
    w = dict(q=P[pre + 'attn.c_q.weight'], k=P[pre + 'attn.c_k.weight'], v=P[pre + 'attn.c_v.weight'],
             gate=P.get(pre + 'attn.ve_gate.weight'), proj=torch.randn(512, 512, generator=g) * 0.03,
             fc=P[pre + 'mlp.c_fc.weight'], out=torch.randn(512, 2048, generator=g) * 0.02)
    x = torch.randn(B, T, 512, generator=g)
    ve = None
    if w['gate'] is not None:
        w['gate'] = torch.randn(8, 32, generator=g) * 0.3
        ve = torch.randn(B, T, 512, generator=g).bfloat16()
    cos, sin = rotary_tables(T)
    return P, w, x, ve, cos, sin, window_sizes()[layer], g


@pytest.mark.parametrize('layer,site', [(0, None), (1, None), (1, 'o'), (3, 'attn'), (5, 'fc'), (7, 'mlp')])
def test_block_forward_matches_oracle(layer, site):
    """run.py:102-117 on the device vs the fp32 oracle at T = 2048 (the layer's real window): the block's
    increment x_out - x within 2e-2 relative (bf16 products and attention), and the fp32 head's per-sequence
    mean loss on x_out within 1e-3."""
    from noise_amd.dust import block_forward, head_loss
    from oracle.model import head_loss as o_head_loss
    P, w, x, ve, cos, sin, window, g = _block_case(layer, 10 + layer)
    jit = {}
    if site:
        width = 2048 if site == 'fc' else 512
        jit[site] = (0.1 * (torch.randint(0, 2, (2, 2048, width), generator=g) * 2 - 1)).bfloat16()
    dev = {k: (None if v is None else v.cuda()) for k, v in w.items()}
    got = block_forward(x.cuda(), dev, None if ve is None else ve.cuda(), cos.bfloat16().cuda(), sin.bfloat16().cuda(),
                        window, **{k: v.cuda() for k, v in jit.items()}).cpu()
    ref = odust.block_forward(x, w, None if ve is None else ve.float(), cos, sin, window,
                              **{k: v.float() for k, v in jit.items()})
    d_got, d_ref = got - x, ref - x
    rel = float((d_got - d_ref).norm() / d_ref.norm())
    y = torch.randint(0, 4096, (2, 2048), generator=g)
    head = P['lm_head.weight'] * 30
    l_got = head_loss(got.cuda(), head.cuda(), y.cuda(), 4096).view(2, 2048).mean(-1).cpu()
    l_ref = o_head_loss(ref, head, y, 4096).view(2, 2048).mean(-1)
    err = float((l_got - l_ref).abs().max())
    print(f'layer {layer} site {site}: increment rel {rel:.2e}, mean-loss err {err:.2e}', flush=True)
    assert rel <= 2e-2
    assert err <= 1e-3
    if site:
        # the jitter's own effect (jittered minus clean) against the oracle's: a difference of two runs whose
        # bf16 activations round independently (2^-9 of |y| ~ 1 against a 0.1 jitter), so 5e-2
        clean = block_forward(x.cuda(), dev, None if ve is None else ve.cuda(), cos.bfloat16().cuda(),
                              sin.bfloat16().cuda(), window).cpu()
        ref_clean = odust.block_forward(x, w, None if ve is None else ve.float(), cos, sin, window)
        eff, ref_eff = got - clean, ref - ref_clean
        rel_eff = float((eff - ref_eff).norm() / ref_eff.norm())
        print(f'    jitter effect rel {rel_eff:.2e} (|effect| {float(ref_eff.norm()):.3e})', flush=True)
        assert rel_eff <= 5e-2


def test_block_forward_chain_is_a_rerun():
    """Two blocks chained from a cached block input with the mixing scalars between them (the loop of
    run.py:256-272) stay within the same bars as one block."""
    from noise_amd.dust import block_forward
    P, w1, x, ve, cos, sin, win1, g = _block_case(1, 21)
    _, w2, _, _, _, _, win2, _ = _block_case(2, 22)
    x0 = torch.randn(x.shape, generator=g)
    lr, lx = 0.9, 0.1
    dev = lambda w: {k: (None if v is None else v.cuda()) for k, v in w.items()}
    cb, sb = cos.bfloat16().cuda(), sin.bfloat16().cuda()
    a = block_forward(x.cuda(), dev(w1), ve.cuda(), cb, sb, win1)
    a = lr * a + lx * x0.cuda()
    a = block_forward(a, dev(w2), None, cb, sb, win2).cpu()
    r = odust.block_forward(x, w1, ve.float(), cos, sin, win1)
    r = lr * r + lx * x0
    r = odust.block_forward(r, w2, None, cos, sin, win2)
    rel = float(((a - x) - (r - x)).norm() / (r - x).norm())
    print('chain rel', rel, flush=True)
    assert rel <= 2e-2


@pytest.mark.parametrize('d', [512, 2048])
def test_draw_errors_matches_oracle(d):
    """run.py:351-355: one chunk's estimate update against the float64 einsum of the oracle; both round the
    reward and the einsum's result to bf16, so entries agree to one bf16 step of the result."""
    from noise_amd.dust import draw_errors
    g = torch.Generator().manual_seed(d)
    n, b, t, sigma = 16, 8, 256, 0.1
    reward = torch.randn(n, b, t, generator=g) * 0.01
    a = (torch.randint(0, 2, (n * b, t, d), generator=g) * 2 - 1).bfloat16()
    errors = torch.randn(b, t, d, generator=g)
    got = draw_errors(errors.clone().cuda(), reward.cuda(), a.cuda(), sigma).cpu().double().numpy()
    ref = odust.draw_errors(errors.numpy(), reward.numpy(), a.float().numpy(), sigma)
    step = np.abs(ref - errors.double().numpy()) * 2 ** -7 + 1e-6
    print('max abs err', float(np.abs(got - ref).max()), flush=True)
    assert np.all(np.abs(got - ref) <= step)


FC, MLP, ATTN, O = 'transformer.h.{}.mlp.c_fc', 'transformer.h.{}.mlp.c_proj', 'transformer.h.{}.attn.c_proj', 'o@{}'
WIDTH = {FC: 2048, MLP: 512, ATTN: 512, O: 512, 'transformer.wte': 512}


@pytest.mark.parametrize('impl', ['rerun', 'rerun_tiled'])
@pytest.mark.parametrize('entry,sites', [(None, ['transformer.wte']), (3, [FC]), (6, [O]), (7, [MLP]), (0, [ATTN]),
                                         (2, [FC]), (7, [FC]), (4, [MLP]), (2, [O, ATTN, FC, MLP])],
                         ids=['embedding', 'fc-3', 'o-6', 'mlp-7', 'attn-0', 'fc-2', 'fc-7', 'mlp-4', 'all-2'])
def test_rerun_matches_oracle(entry, sites, impl):
    """DUST.rerun (run.py:256-279) end to end -- the cached input repeated n times (or the jittered embedding
    entry), the later blocks' mixing, block_forward with the entry's jitter, the final norm and fp32 head --
    against the oracle rerun composed from the pinned pieces (oracle/dust.py), per draw and per token. The
    capture cache comes from the oracle's clean forward. Head x30 so the losses depend on the blocks; sigma
    0.1 (+-1 draws in bf16 as the reference's) so the jitter moves them visibly. Each draw's mean loss stays
    within 1e-3 of the fp32 oracle, and so does the jitter's effect (rerun minus the unjittered rerun, the
    reward DUST forms) per draw. Per token, bf16 products and attention through up to 8 blocks (the
    reference's autocast numerics) put single tokens up to 2e-2 from fp32 (measured 1.95e-2 from the
    embedding): the per-token bound is 3e-2. Both forms: rerun (every block on the population kernels, the
    entry block's jitter in noise_block_entry, noise_add_bf16 and the jittered block kernels: mlp.c_fc jitter
    before a block with and without value embeddings and before the head, mlp.c_proj jitter alone, all four
    sites at once) and rerun_tiled (every block on noise_dust_block)."""
    from types import SimpleNamespace
    import noise_amd.dust as ndust
    rerun = getattr(ndust, impl)
    from noise_amd.model import make_model
    model = make_model('cpu', 0)
    with torch.no_grad():
        model.lm_head.weight.mul_(30)
    P = {k: v.detach().float().clone() for k, v in model.named_parameters()}
    g = torch.Generator().manual_seed(31)
    b, T, n = 2, 256, 3
    rows = torch.randint(0, 4096, (b, T + 1), generator=g)
    x, y = rows[:, :-1], rows[:, 1:]
    cache = odust.capture(P, x)
    names = [site.format(entry) if entry is not None else site for site in sites]
    jitter = {}
    for site, name in zip(sites, names):
        draws = (torch.randint(0, 2, (n * b, T, WIDTH[site]), generator=g) * 2 - 1).bfloat16()
        jitter[name] = (0.1 * draws.float()).bfloat16()
    print(f'rerun: entry {entry}, jitter at {names}, {n} draws x {b} sequences x {T} tokens', flush=True)
    ref = odust.rerun(P, cache, y, n, entry, jitter)
    zero = {name: torch.zeros_like(t) for name, t in jitter.items()}
    ref0 = odust.rerun(P, cache, y, n, entry, {} if entry is not None else zero)
    dev = torch.device('cuda', 0)
    m = model.to(dev)
    to = lambda d: {k: v.to(dev) for k, v in d.items()}
    dust = SimpleNamespace(model=m, length=T, batch=b, outputs=to(cache['outputs']),
                           blocks=to(cache['blocks']), x0=cache['x0'].to(dev), x=x.to(dev), y=y.to(dev),
                           weights=[{k: (None if v is None else v.to(dev)) for k, v in odust.block_weights(P, i).items()}
                                    for i in range(8)])
    got = rerun(dust, n, entry, to(jitter)).cpu()
    got0 = rerun(dust, n, entry, {} if entry is not None else to(zero)).cpu()
    assert got.shape == (n, b, T) and torch.isfinite(got).all()
    tok = (got - ref).abs().max().item()
    mean = (got.mean(-1) - ref.mean(-1)).abs().max().item()
    eff = ((got - got0).mean(-1) - (ref - ref0).mean(-1)).abs().max().item()
    print(f'rerun: per-token {tok:.2e}, per-draw mean {mean:.2e}, jitter effect {eff:.2e}, effect size '
          f'{(ref - ref0).mean(-1).abs().max().item():.2e}', flush=True)
    assert tok <= 3e-2
    assert mean <= 1e-3
    assert eff <= 1e-3
    effect = (ref - ref0).mean(-1).abs().max().item()
    assert effect > max(1e-4, 10 * eff), 'the jitter must move the losses well beyond the error'


@pytest.mark.parametrize('entry,sites,prior_sites,gamma', [
    (6, ['transformer.h.6.mlp.c_fc', 'o@6'], ['o@6'], 0.0),
    (3, ['transformer.h.3.mlp.c_fc', 'transformer.h.3.attn.c_proj'], ['transformer.h.3.mlp.c_fc'], 0.0),
    (None, ['transformer.wte'], [], 0.9)], ids=['late-fc-o-prior', 'fc-prior-attn', 'embedding-gamma'])
def test_direct_errors_matches_oracle(monkeypatch, entry, sites, prior_sites, gamma):
    """DUST.direct_errors (run.py:332-378) end to end on the device -- orthogonal draws per site, the live-unit
    mask of an mlp.c_fc site, 2 chunks of n = 4 draws (draws 8, nrep 4) rerun from block `entry`, the reward
    centred over each chunk (the clean loss is offset by 0.05 so that an uncentred reward would show), priors from
    a retrieval (alpha 0.5), reward-to-go, the bf16 estimate update -- against the oracle composition
    (oracle/dust.py direct_errors over OrthogonalDrawsOracle, the oracle's rerun and the bf16 roundings).

    Bounds. (1) The device draws equal the oracle's bit for bit. (2) Fed the device rerun's own losses, the
    oracle composition agrees with the device estimate to the rounding of the bf16 steps: per chunk a one-ulp
    flip (2^-7 relative) of each draw's bf16 reward and of the chunk sum, / (sigma draws). (3) The device rerun's
    losses are within the rerun's bar of the fp32 oracle's (per-draw mean 1e-3, per token 3e-2), and the
    end-to-end estimate differs from the oracle's by at most the propagated reward difference
    sum_i |delta r_i| |a_i| / (sigma draws) plus (2). (4) Dead units of an mlp.c_fc site without a prior are
    exactly 0; estimates of prior sites and the fits of retrieved sites are recorded as the reference does."""
    from types import SimpleNamespace
    import noise_amd.dust as ndust
    from noise_amd.model import make_model
    from noise_amd.noise import OrthogonalDraws
    from oracle.orthogonal import OrthogonalDrawsOracle
    model = make_model('cpu', 0)
    with torch.no_grad():
        model.lm_head.weight.mul_(30)
    P = {k: v.detach().float().clone() for k, v in model.named_parameters()}
    g = torch.Generator().manual_seed(41)
    b, T, draws, nrep, sigma = 2, 256, 8, 4, 0.1
    rows = torch.randint(0, 4096, (b, T + 1), generator=g)
    x, y = rows[:, :-1], rows[:, 1:]
    cache = odust.capture(P, x)
    clean = odust.rerun(P, cache, y, 1, 6, {})[0] + 0.05
    dev = torch.device('cuda', 0)
    to = lambda d: {k: v.to(dev) for k, v in d.items()}
    widths = {s: 512 if s.startswith('o@') else cache['outputs'][s].shape[-1] for s in sites}
    retrieved = {s: (torch.randn(b, T, widths[s], generator=g) * 0.2) for s in prior_sites}
    alpha = {s: 0.5 for s in prior_sites}
    print(f'direct_errors: entry {entry}, sites {sites}, priors {prior_sites}, gamma {gamma}, {draws} draws in '
          f'chunks of {nrep}, {b} x {T} tokens', flush=True)

    draws_dev = OrthogonalDraws(seed=0, device=dev)
    seen_draws, seen_losses = [], []

    def orthogonal_noise(site, draws_, chunk, n, b_, t_, d):
        a = draws_dev(site, draws_, chunk, n, b_, t_, d, dtype=torch.bfloat16)
        seen_draws.append((site, chunk, a.cpu()))
        return a

    real_rerun = ndust.rerun

    def recording_rerun(dust_, n, entry_, jitter):
        loss = real_rerun(dust_, n, entry_, jitter)
        seen_losses.append(loss.cpu().double().numpy())
        return loss

    monkeypatch.setattr(ndust, 'rerun', recording_rerun)
    m = model.to(dev)
    dust = SimpleNamespace(
        model=m, length=T, batch=b, outputs=to(cache['outputs']), blocks=to(cache['blocks']), x0=cache['x0'].to(dev),
        x=x.to(dev), y=y.to(dev), clean_loss=clean.to(dev), dtype=torch.bfloat16, recipe=SimpleNamespace(nrep=nrep),
        weights=[{k: (None if v is None else v.to(dev)) for k, v in odust.block_weights(P, i).items()} for i in range(8)],
        alpha=alpha, estimates={}, fits={}, prior_sites=list(prior_sites), orthogonal_noise=orthogonal_noise)
    got = ndust.direct_errors(dust, sites, draws, sigma, entry=entry, gamma=gamma, retrieved=to(retrieved))
    got = {s: e.cpu().double().numpy() for s, e in got.items()}

    live = {s: (cache['outputs'][s] > 0).double().numpy() for s in sites if s.endswith('mlp.c_fc')}
    priors = {s: 0.5 * retrieved[s].double().numpy() for s in prior_sites}
    oracle_draws = OrthogonalDrawsOracle(seed=0)
    draw = lambda *args: oracle_draws(*args)
    replay = iter(seen_losses)
    ref_g, rec_g = odust.direct_errors(draw, lambda n, j: next(replay), clean.numpy(), live, sites, widths, draws,
                                       sigma, nrep, gamma=gamma, priors=priors)
    oracle_draws = OrthogonalDrawsOracle(seed=0)
    ref, rec = odust.direct_errors(draw, lambda n, j: odust.rerun(P, cache, y, n, entry, j).numpy(), clean.numpy(),
                                   live, sites, widths, draws, sigma, nrep, gamma=gamma, priors=priors)

    # (1) the draws (the composition masks an mlp.c_fc site's draws by its live units)
    assert len(seen_draws) == len(sites) * (draws // nrep)
    for site, chunk, a in seen_draws:
        assert np.array_equal(a.double().numpy() * live.get(site, 1.0), rec_g[chunk]['a'][site]), (site, chunk)
    # (2) the composition over the device losses, to the bf16 steps' rounding
    ulp = 2.0 ** -7
    worst = {}
    for s in sites:
        bound = sum(ulp * (np.abs(r['sums'][s]) + np.einsum('nbt,nbtd->btd', np.abs(r['reward']), np.abs(r['a'][s])))
                    for r in rec_g) / (sigma * draws) + 1e-6
        diff = np.abs(got[s] - ref_g[s])
        worst[s] = float((diff / bound).max())
        assert np.all(diff <= bound), (s, worst[s])
    # (3) the end-to-end estimate against the fp32 oracle rerun
    dev_loss, ora_loss = np.stack(seen_losses), np.stack([r['loss'] for r in rec])
    tok = np.abs(dev_loss - ora_loss).max()
    mean = np.abs(dev_loss.mean(-1) - ora_loss.mean(-1)).max()
    assert tok <= 3e-2 and mean <= 1e-3, (tok, mean)
    for s in sites:
        prop = sum(np.einsum('nbt,nbtd->btd', np.abs(rg['reward'] - ro['reward']), np.abs(ro['a'][s]))
                   for rg, ro in zip(rec_g, rec)) / (sigma * draws)
        bound = prop + sum(ulp * (np.abs(r['sums'][s]) + np.einsum('nbt,nbtd->btd', np.abs(r['reward']),
                                                                   np.abs(r['a'][s]))) for r in rec_g + rec) \
            / (sigma * draws) + 1e-6
        rel = float(np.linalg.norm(got[s] - ref[s]) / np.linalg.norm(ref[s]))
        print(f'  {s}: composition {worst[s]:.2f} of its rounding bound; end to end rel {rel:.2e}, '
              f'|estimate| rms {float(np.sqrt((ref[s] ** 2).mean())):.3e}', flush=True)
        assert np.all(np.abs(got[s] - ref[s]) <= bound), s
    print(f'  rerun: per-token {tok:.2e}, per-draw mean {mean:.2e}', flush=True)
    # (4) dead units, recorded estimates and fits
    for s, mask in live.items():
        if s not in prior_sites:
            assert np.all(got[s][mask == 0] == 0)
    assert set(dust.estimates) == set(prior_sites)
    for s in prior_sites:
        kept = 1 - 1 / 4
        r = retrieved[s].double().numpy()
        dot, rr = dust.fits[s].cpu().double().numpy()
        assert abs(rr - (r * r).sum()) <= 1e-4 * (r * r).sum()
        assert abs(dot - (r * got[s] / kept).sum()) <= 1e-3 * np.abs(r * got[s] / kept).sum()



@pytest.mark.parametrize('entry,site,width', [(3, 'transformer.h.{}.mlp.c_fc', 2048), (6, 'o@{}', 512)],
                         ids=['fc-3', 'o-6'])
def test_rerun_fp32_stream_against_the_bf16_flow(entry, site, width):
    """The reference's DUST on a GPU keeps the model's embeddings in bf16 (utils/model.py:171-175), so its cached
    block inputs, x0 and value rows are bf16 and, under autocast, its residual stream is bf16 between blocks
    (oracle/dust.py rerun_bf16_flow). rerun keeps the stream in fp32 (the population kernels' residual). Measured
    here on the bf16-valued cache the reference would hold: the per-draw mean losses and the jitter's effect
    (rerun minus the unjittered rerun: the reward direct_errors forms, centred over draws) against that flow.
    Bounds: per-draw mean within 2e-3, the jitter's effect within 1e-3 (measured ~1e-3 and ~2e-4); the printed
    sizes are the deviation the fp32 stream brings against the reference's own GPU numerics."""
    from types import SimpleNamespace
    from noise_amd.dust import rerun
    from noise_amd.model import make_model
    model = make_model('cpu', 0)
    with torch.no_grad():
        model.lm_head.weight.mul_(30)
        for emb in [model.transformer.wte, *model.value_embeds.values()]:
            emb.weight.copy_(emb.weight.bfloat16().float())       # bf16 storage, as on a GPU
    P = {k: v.detach().float().clone() for k, v in model.named_parameters()}
    g = torch.Generator().manual_seed(51)
    b, T, n = 2, 256, 3
    rows = torch.randint(0, 4096, (b, T + 1), generator=g)
    x, y = rows[:, :-1], rows[:, 1:]
    cache = odust.capture(P, x)
    bf = lambda t: t.bfloat16()
    name = site.format(entry)
    jitter = {name: (0.1 * (torch.randint(0, 2, (n * b, T, width), generator=g) * 2 - 1)).bfloat16()}
    flow = odust.rerun_bf16_flow(P, cache, y, n, entry, jitter)
    flow0 = odust.rerun_bf16_flow(P, cache, y, n, entry, {})
    dev = torch.device('cuda', 0)
    m = model.to(dev)
    dust = SimpleNamespace(model=m, length=T, batch=b, x=x.to(dev), y=y.to(dev),
                           outputs={k: bf(v).to(dev) for k, v in cache['outputs'].items()},
                           blocks={k: bf(v).to(dev) for k, v in cache['blocks'].items()}, x0=bf(cache['x0']).to(dev),
                           weights=[{k: (None if v is None else v.to(dev)) for k, v in odust.block_weights(P, i).items()}
                                    for i in range(8)])
    got = rerun(dust, n, entry, {k: v.to(dev) for k, v in jitter.items()}).cpu()
    got0 = rerun(dust, n, entry, {}).cpu()
    mean = (got.mean(-1) - flow.mean(-1)).abs().max().item()
    eff = ((got - got0).mean(-1) - (flow - flow0).mean(-1)).abs().max().item()
    tok = (got - flow).abs().max().item()
    size = (flow - flow0).mean(-1).abs().max().item()
    print(f'fp32 stream vs the bf16 flow: per-draw mean {mean:.2e}, jitter effect {eff:.2e} (effect size '
          f'{size:.2e}), per token {tok:.2e}', flush=True)
    assert mean <= 2e-3 and eff <= 1e-3


@pytest.mark.parametrize('entry,sites', [(2, [FC, O]), (5, [MLP, ATTN]), (7, [FC, MLP])], ids=['fc-o-2', 'mlp-attn-5', 'fc-mlp-7'])
def test_rerun_full_length(entry, sites):
    """rerun at T = 2048 (the model's windows active: 1024 in blocks 0-2 and 4-6, 2048 in 3 and 7; 16 block-kernel
    tiles per sequence, every jitter row of a 2048-token row-set) against the fp32 oracle: per-draw mean loss and
    the jitter's effect within 1e-3, per token within 3e-2; and against rerun_tiled (the tiled kernels, another
    summation order of the same bf16 products) per-draw mean within 1e-3."""
    from types import SimpleNamespace
    from noise_amd.dust import rerun, rerun_tiled
    from noise_amd.model import make_model
    model = make_model('cpu', 0)
    with torch.no_grad():
        model.lm_head.weight.mul_(30)
    P = {k: v.detach().float().clone() for k, v in model.named_parameters()}
    g = torch.Generator().manual_seed(61 + entry)
    b, T, n = 1, 2048, 2
    rows = torch.randint(0, 4096, (b, T + 1), generator=g)
    x, y = rows[:, :-1], rows[:, 1:]
    cache = odust.capture(P, x)
    jitter = {}
    for site in sites:
        draws = (torch.randint(0, 2, (n * b, T, WIDTH[site]), generator=g) * 2 - 1).bfloat16()
        jitter[site.format(entry)] = (0.1 * draws.float()).bfloat16()
    print(f'rerun at T = {T}: entry {entry}, jitter at {list(jitter)}', flush=True)
    ref = odust.rerun(P, cache, y, n, entry, jitter)
    ref0 = odust.rerun(P, cache, y, n, entry, {})
    dev = torch.device('cuda', 0)
    to = lambda d: {k: v.to(dev) for k, v in d.items()}
    dust = SimpleNamespace(model=model.to(dev), length=T, batch=b, outputs=to(cache['outputs']),
                           blocks=to(cache['blocks']), x0=cache['x0'].to(dev), x=x.to(dev), y=y.to(dev),
                           weights=[{k: (None if v is None else v.to(dev)) for k, v in odust.block_weights(P, i).items()}
                                    for i in range(8)])
    got = rerun(dust, n, entry, to(jitter)).cpu()
    got0 = rerun(dust, n, entry, {}).cpu()
    tiled = rerun_tiled(dust, n, entry, to(jitter)).cpu()
    tok = (got - ref).abs().max().item()
    mean = (got.mean(-1) - ref.mean(-1)).abs().max().item()
    eff = ((got - got0).mean(-1) - (ref - ref0).mean(-1)).abs().max().item()
    vs_tiled = (got.mean(-1) - tiled.mean(-1)).abs().max().item()
    print(f'  per-token {tok:.2e}, per-draw mean {mean:.2e}, jitter effect {eff:.2e} (size '
          f'{(ref - ref0).mean(-1).abs().max().item():.2e}), vs rerun_tiled {vs_tiled:.2e}', flush=True)
    assert torch.isfinite(got).all()
    assert tok <= 3e-2 and mean <= 1e-3 and eff <= 1e-3 and vs_tiled <= 1e-3


def test_rerun_row_kernels():
    """The rerun's row kernels against torch on the same inputs: noise_mask_scale (a * mask in place and
    bf16(sigma * a), run.py:344-349) and noise_add_bf16 (y + o in bf16, run.py:114) bit for bit; noise_block_entry
    (x + attn jitter in fp32, bit for bit, and bf16(norm(x)) to one bf16 step; rows read modulo the cached rows)."""
    from noise_amd import _lib
    dev = torch.device('cuda', 0)
    g = torch.Generator(device=dev).manual_seed(71)
    n, b, t, d = 3, 2, 256, 2048
    a = (torch.randint(0, 2, (n, b, t, d), device=dev, generator=g) * 2 - 1).bfloat16()
    mask = (torch.rand(b, t, d, device=dev, generator=g) > 0.4).bfloat16()
    want_a, want_j = a * mask, 0.1 * (a * mask)
    scaled = torch.empty_like(a)
    _lib.call('noise_mask_scale', a.data_ptr(), mask.data_ptr(), n, b * t * d, 0.1, scaled.data_ptr(),
              _lib.stream_ptr(dev))
    assert torch.equal(a, want_a) and torch.equal(scaled, want_j)
    y = torch.randn(4, 256, 512, device=dev, generator=g).bfloat16()
    o = (0.1 * torch.randn(4, 256, 512, device=dev, generator=g)).bfloat16()
    want = y + o
    _lib.call('noise_add_bf16', y.data_ptr(), o.data_ptr(), y.numel(), _lib.stream_ptr(dev))
    assert torch.equal(y, want)
    x = torch.randn(2, 256, 512, device=dev, generator=g) * 3
    add = (0.1 * torch.randn(6, 256, 512, device=dev, generator=g)).bfloat16()
    out = torch.empty(6, 256, 512, device=dev)
    h = torch.empty(6, 256, 512, dtype=torch.bfloat16, device=dev)
    _lib.call('noise_block_entry', x.data_ptr(), 2 * 256, add.data_ptr(), 6 * 256, out.data_ptr(), h.data_ptr(),
              _lib.stream_ptr(dev))
    xr = x.repeat(3, 1, 1)
    assert torch.equal(out, xr + add.float())
    href = torch.nn.functional.rms_norm(xr, (512,))
    assert ((h.float() - href).abs() <= href.abs() * 2 ** -7 + 1e-6).all()
