"""noise_pop_block_qkv (a block's tail followed in the same kernel by the next block's value-embedding gates
and q/k/v, eggroll.py:92-94 then 81-90) against the launches it replaces: noise_pop_block writing h and the
next dots, then noise_pop_gate and noise_pop_qkv on that h (each pinned against the oracle by the population
and drop-in tests).

The residual rows come from the same code in both and must agree bit for bit; the gates are summed in the
gate kernel's order. The q/k/v products take h's k index in the permuted order the block kernel holds it in
(c_q, c_k, c_v permuted to match), so an fp32 sum can round differently; q, k, v agree to one bf16 ulp of
their scale, and the share of elements that differ at all is printed and bounded. Covered: value embeddings
with and without their gate and table noise, rank-1 noise on all of c_q, c_k, c_v or on c_k alone, none at
all, one token sequence shared by every member or one per member, a token id outside the value table (its V
rows are NaN in both), and the argument checks."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)
VOCAB = 300


def _case(m, T, seed, qkv_noise, ve, ve_noise, per_member_idx, block_noise=True):
    g = torch.Generator().manual_seed(seed)
    dirs = -(-m // 2)
    u = lambda *s, scale: ((torch.rand(*s, generator=g) * 2 - 1) * scale)
    c = dict(m=m, T=T)
    c['y'] = torch.randn(m, T, 512, generator=g).bfloat16()
    c['wo'] = u(512, 512, scale=1.5 * (3 / 512) ** 0.5).bfloat16()
    c['wfc'] = u(2048, 512, scale=(3 / 512) ** 0.5).bfloat16()
    c['wpj'] = u(512, 2048, scale=1.5 * (3 / 2048) ** 0.5).bfloat16()
    c['xres'] = torch.randn(m, T, 512, generator=g)
    c['x0'] = torch.randn(m, T, 512, generator=g)
    c['lam'] = torch.tensor([0.9, 0.15])
    if block_noise:
        c['ao'], c['odots'] = torch.randn(dirs, 512, generator=g), torch.randn(m * T, 8, generator=g)
        c['afc'], c['bfc'] = torch.randn(dirs, 2048, generator=g), torch.randn(dirs, 512, generator=g)
        c['apj'], c['bpj'] = torch.randn(dirs, 512, generator=g), torch.randn(dirs, 2048, generator=g)
        c['eps'] = torch.randn(dirs, 2, generator=g)
    else:
        for k in ('ao', 'odots', 'afc', 'bfc', 'apj', 'bpj', 'eps'):
            c[k] = None
    c['wq'] = [u(512, 512, scale=(3 / 512) ** 0.5).bfloat16() for _ in range(3)]
    c['rq'] = []
    for j in range(3):
        on = qkv_noise == 'all' or (qkv_noise == 'k' and j == 1)
        c['rq'].append((torch.randn(dirs, 512, generator=g), torch.randn(dirs, 512, generator=g)) if on else None)
    c['ve'] = torch.randn(VOCAB, 512, generator=g) if ve else None
    c['gate_w'] = (torch.randn(8, 32, generator=g) * 0.3).bfloat16().float() if ve else None
    if ve and ve_noise:
        c['rgate'] = (torch.randn(dirs, 8, generator=g), torch.randn(dirs, 32, generator=g))
        c['rve'] = (torch.randn(dirs, VOCAB, generator=g), torch.randn(dirs, 512, generator=g))
    else:
        c['rgate'] = c['rve'] = None
    idx = torch.randint(0, VOCAB, (m, T) if per_member_idx else (T,), generator=g)
    idx.view(-1)[7] = VOCAB + 5  # outside the table
    c['idx'] = idx
    c['sign'] = torch.tensor([0.05, -0.05]).repeat(dirs)[:m]

    def dev(v):
        if v is None:
            return None
        if isinstance(v, (list, tuple)):
            return type(v)(dev(t) for t in v)
        return v.to(DEV).contiguous() if torch.is_tensor(v) else v
    return {k: dev(v) for k, v in c.items()}


def _rank1(pair):
    from noise_amd import _lib
    if pair is None:
        return _lib.Rank1(None, None, 0, 0)
    a, b = pair
    return _lib.Rank1(a.data_ptr(), b.data_ptr(), a.stride(0), b.stride(0))


def _common(c):
    from noise_amd import _lib
    from noise_amd.eggroll import _rope_tables
    m, T = c['m'], c['T']
    stream = _lib.stream_ptr(DEV)
    pop = _lib.Population(m, T, c['sign'].data_ptr(), 2, _lib.ROUNDING_FUSED)
    V = lambda t, w: _lib.View(t.data_ptr(), T * w, w)
    r_o = _lib.Rank1(None, None, 0, 0) if c['ao'] is None else _lib.Rank1(c['ao'].data_ptr(), None,
                                                                          c['ao'].stride(0), 0)
    r_fc = _rank1(None if c['afc'] is None else (c['afc'], c['bfc']))
    r_pj = _rank1(None if c['apj'] is None else (c['apj'], c['bpj']))
    perm = {}
    for k in ('wfc', 'wpj'):
        perm[k] = torch.empty_like(c[k])
        _lib.call('noise_block_weight_layout', c[k].data_ptr(), perm[k].data_ptr(), c[k].shape[0], c[k].shape[1],
                  stream)
    eps = c['eps']
    mixargs = (1, c['lam'].data_ptr(), c['lam'].data_ptr() + 4, None if eps is None else eps[:, 0].data_ptr(),
               None if eps is None else eps[:, 1].data_ptr(), 0 if eps is None else eps.stride(0))
    xout = c['xres'].clone()
    head = (ctypes.byref(pop), V(c['y'], 512), c['wo'].data_ptr(), ctypes.byref(r_o), _lib.ptr(c['odots']), 8,
            V(xout, 512), perm['wfc'].data_ptr(), ctypes.byref(r_fc), perm['wpj'].data_ptr(), ctypes.byref(r_pj),
            xout.data_ptr(), *mixargs, V(c['x0'], 512))
    cos, sin = _rope_tables(T, DEV)
    outs = [torch.full((m, 8, T, 64), float('nan'), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    outs.append(torch.full((m, 8, 64, T), float('nan'), dtype=torch.bfloat16, device=DEV))
    r_q = (_lib.Rank1 * 3)(*[_rank1(p) for p in c['rq']])
    idx_sm = T if c['idx'].dim() == 2 else 0
    return pop, stream, V, head, xout, outs, r_q, cos, sin, idx_sm


def _separate(c):
    from noise_amd import _lib
    m, T = c['m'], c['T']
    pop, stream, V, head, xout, outs, r_q, cos, sin, idx_sm = _common(c)
    perturbed = any(p is not None for p in c['rq'])
    zero_b = torch.zeros(1, 512, device=DEV)
    nxt = (_lib.Rank1 * 3)(*[_rank1(p) if p is not None else _lib.Rank1(None, zero_b.data_ptr(), 0, 0)
                             for p in c['rq']])
    h = torch.full((m, T, 512), float('nan'), dtype=torch.bfloat16, device=DEV)
    dots = torch.full((m * T, 3), float('nan'), device=DEV)
    _lib.call('noise_pop_block', *head, h.data_ptr(), 0, nxt if perturbed else None, 3 if perturbed else 0,
              dots.data_ptr() if perturbed else None, stream)
    gates = torch.full((m * T, 8), float('nan'), device=DEV)
    ve = c['ve']
    if ve is not None:
        rg = _rank1(c['rgate'])
        _lib.call('noise_pop_gate', ctypes.byref(pop), V(h, 512), c['gate_w'].data_ptr(), ctypes.byref(rg),
                  gates.data_ptr(), stream)
    ws = (ctypes.c_void_p * 3)(*(w.data_ptr() for w in c['wq']))
    rve = _rank1(c['rve'])
    _lib.call('noise_pop_qkv', ctypes.byref(pop), V(h, 512), ws, r_q, dots.data_ptr(), cos.data_ptr(),
              sin.data_ptr(), _lib.ptr(ve), VOCAB if ve is not None else 0, c['idx'].data_ptr(), idx_sm,
              gates.data_ptr() if ve is not None else None, ctypes.byref(rve),
              (ctypes.c_void_p * 3)(*(o.data_ptr() for o in outs)), stream)
    torch.cuda.synchronize()
    return xout.cpu(), [o.float().cpu() for o in outs]


def _fused(c, **override):
    from noise_amd import _lib
    pop, stream, V, head, xout, outs, r_q, cos, sin, idx_sm = _common(c)
    wperm = []
    for w in c['wq']:
        p = torch.empty_like(w)
        _lib.call('noise_block_weight_layout', w.data_ptr(), p.data_ptr(), 512, 512, stream)
        wperm.append(p)
    ws = (ctypes.c_void_p * 3)(*(w.data_ptr() for w in wperm))
    ve = c['ve']
    rg, rve = _rank1(c['rgate']), _rank1(c['rve'])
    args = dict(head=head, ws=ws, r_q=r_q, cos=cos.data_ptr(), sin=sin.data_ptr(), ve=_lib.ptr(ve),
                vocab=VOCAB if ve is not None else 0, idx=c['idx'].data_ptr(), idx_sm=idx_sm,
                gate_w=_lib.ptr(c['gate_w']), rg=ctypes.byref(rg), rve=ctypes.byref(rve),
                out=(ctypes.c_void_p * 3)(*(o.data_ptr() for o in outs)))
    args.update(override)
    status = _lib.lib().noise_pop_block_qkv(*args['head'], args['ws'], args['r_q'], args['cos'], args['sin'],
                                            args['ve'], args['vocab'], args['idx'], args['idx_sm'], args['gate_w'],
                                            args['rg'], args['rve'], args['out'], stream)
    torch.cuda.synchronize()
    return status, xout.cpu(), [o.float().cpu() for o in outs]


CASES = {
    've-noisy': dict(qkv_noise='all', ve=True, ve_noise=True, per_member_idx=False),
    've-plain-gate': dict(qkv_noise='all', ve=True, ve_noise=False, per_member_idx=True),
    'no-ve': dict(qkv_noise='all', ve=False, ve_noise=False, per_member_idx=False),
    'k-only': dict(qkv_noise='k', ve=True, ve_noise=True, per_member_idx=False),
    'unperturbed': dict(qkv_noise='none', ve=True, ve_noise=False, per_member_idx=False, block_noise=False),
}


@pytest.mark.parametrize('name,m,T', [(n, 4, 256) for n in CASES] + [('ve-noisy', 3, 256)],
                         ids=list(CASES) + ['ve-noisy-3-members'])
def test_block_qkv_matches_separate_launches(name, m, T):
    """Every case at 4 members x 256 tokens, and an odd member count (the last direction has one member)."""
    print(f'block + next q/k/v: {m} members x {T} tokens, case {name}', flush=True)
    c = _case(m, T, 11, **CASES[name])
    xo_s, qkv_s = _separate(c)
    status, xo_f, qkv_f = _fused(c)
    assert status == 0
    assert torch.equal(xo_f, xo_s)
    for j, (f, s) in enumerate(zip(qkv_f, qkv_s)):
        nan_s, nan_f = torch.isnan(s), torch.isnan(f)
        assert torch.equal(nan_s, nan_f), f'matrix {j}: NaN positions differ'
        if j == 2 and c['ve'] is not None:
            # token 7 of the first sequence reads an id outside the table: its V is NaN in every head
            assert nan_s[0, :, :, 7].all()
        else:
            assert not nan_s.any()
        fs, ss = f[~nan_s], s[~nan_s]
        scale = ss.abs().max()
        diff = (fs - ss).abs()
        frac = (diff > 0).float().mean().item()
        print(f'  matrix {j}: max |diff| {diff.max().item():.3e} of scale {scale.item():.3e}, '
              f'{100 * frac:.3f}% of elements differ', flush=True)
        assert diff.max() <= 2.0 ** -7 * scale
        assert frac < 0.02
    again = _fused(c)
    assert torch.equal(again[1], xo_f)
    for f, a in zip(qkv_f, again[2]):
        assert torch.equal(torch.nan_to_num(f, nan=7.0), torch.nan_to_num(a, nan=7.0))


def test_block_qkv_rejects_bad_arguments():
    from noise_amd import _lib
    c = _case(4, 256, 5, qkv_noise='all', ve=True, ve_noise=True, per_member_idx=False)
    lib = _lib.lib()
    status, _, _ = _fused(c, gate_w=None)
    assert status != 0 and b'gate' in lib.noise_last_error()
    status, _, _ = _fused(c, out=None)
    assert status != 0
    status, _, _ = _fused(c, idx_sm=100)
    assert status != 0 and b'idx_sm' in lib.noise_last_error()
    _, _, _, head, _, _, _, _, _, _ = _common(c)
    no_xout = list(head)
    no_xout[11] = None
    status, _, _ = _fused(c, head=tuple(no_xout))
    assert status != 0 and b'xout' in lib.noise_last_error()
