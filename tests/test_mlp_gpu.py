"""The fused MLP (noise_pop_mlp: mlp.c_fc, ReLU^2, mlp.c_proj and the residual writer in one kernel,
eggroll.py:93 + 77-79) against the two-kernel path it replaces (noise_pop_fc then noise_pop_residual with
K = 2048, whose parity with the oracle the population tests pin) and against an fp32 restatement of the same
arithmetic on the CPU.

Both GPU paths round the hidden layer to bf16 from fp32 sums taken in different orders, so a hidden value
can round one bf16 ulp apart; outputs agree to 2e-3 of their scale (measured ~1e-5), next-matrix dots and the
bf16 norm output likewise. Every variant the population forward launches is covered: mixing on or off, 0, 1
or 3 next dots, the split-bf16x3 head input, perturbed or unperturbed matrices, with and without xout."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def _case(m, T, seed, perturbed):
    g = torch.Generator().manual_seed(seed)
    dirs = m // 2
    x = torch.randn(m, T, 512, generator=g)
    h = (x / x.pow(2).mean(-1, keepdim=True).sqrt()).bfloat16()
    wfc = ((torch.rand(2048, 512, generator=g) * 2 - 1) * (3 / 512) ** 0.5).bfloat16()
    wpj = ((torch.rand(512, 2048, generator=g) * 2 - 1) * 1.5 * (3 / 2048) ** 0.5).bfloat16()
    xres = torch.randn(m, T, 512, generator=g)
    x0 = torch.randn(m, T, 512, generator=g)
    nb = [torch.randn(dirs, 512, generator=g) for _ in range(3)]
    if perturbed:
        afc, bfc = torch.randn(dirs, 2048, generator=g), torch.randn(dirs, 512, generator=g)
        apj, bpj = torch.randn(dirs, 512, generator=g), torch.randn(dirs, 2048, generator=g)
        eps = torch.randn(dirs, 2, generator=g)
    else:
        afc = bfc = apj = bpj = eps = None
    sign = torch.tensor([0.05, -0.05]).repeat(dirs)
    lam = torch.tensor([0.9, 0.15])
    d = lambda t: None if t is None else t.to(DEV).contiguous()
    return dict(h=d(h), wfc=d(wfc), wpj=d(wpj), xres=d(xres), x0=d(x0), nb=[d(t) for t in nb], afc=d(afc), bfc=d(bfc),
                apj=d(apj), bpj=d(bpj), eps=d(eps), sign=d(sign), lam=d(lam), m=m, T=T)


def _run(c, fused, mix, nnext, split3, with_xout):
    from noise_amd import _lib
    m, T = c['m'], c['T']
    rows = m * T
    stream = _lib.stream_ptr(DEV)
    pop = _lib.Population(m, T, c['sign'].data_ptr(), 2, _lib.ROUNDING_FUSED)
    V = lambda t, w: _lib.View(t.data_ptr(), T * w, w)
    R = lambda a, b: _lib.Rank1(None, None, 0, 0) if a is None else _lib.Rank1(a.data_ptr(), b.data_ptr(),
                                                                               a.stride(0), b.stride(0))
    r_fc, r_pj = R(c['afc'], c['bfc']), R(c['apj'], c['bpj'])
    # x . b_fc, as the attn.c_proj residual writer leaves it
    dots = torch.zeros(rows, dtype=torch.float32, device=DEV)
    if c['afc'] is not None:
        _lib.call('noise_member_dots', ctypes.byref(pop), V(c['h'], 512), 512, ctypes.byref(_lib.Rank1(
            None, c['bfc'].data_ptr(), 0, c['bfc'].stride(0))), 1, dots.data_ptr(), stream)
    nxt = (_lib.Rank1 * 3)(*[_lib.Rank1(None, t.data_ptr(), 0, t.stride(0)) for t in c['nb']])
    ndots = torch.full((rows, max(nnext, 1)), float('nan'), device=DEV)
    xout = c['xres'].clone() if with_xout else None
    width = 1536 if split3 else 512
    hout = torch.full((m, T, width), float('nan'), dtype=torch.bfloat16, device=DEV)
    eps = c['eps']
    mixargs = (1, c['lam'].data_ptr(), c['lam'].data_ptr() + 4, None if eps is None else eps[:, 0].data_ptr(),
               None if eps is None else eps[:, 1].data_ptr(), 0 if eps is None else eps.stride(0)) if mix else \
        (0, None, None, None, None, 0)
    xres = xout if with_xout else c['xres']
    if fused:
        wperm = torch.empty_like(c['wpj'])
        _lib.call('noise_mlp_proj_layout', c['wpj'].data_ptr(), wperm.data_ptr(), 512, stream)
        _lib.call('noise_pop_mlp', ctypes.byref(pop), V(c['h'], 512), c['wfc'].data_ptr(), ctypes.byref(r_fc),
                  dots.data_ptr(), wperm.data_ptr(), ctypes.byref(r_pj), V(xres, 512), _lib.ptr(xout), *mixargs,
                  V(c['x0'], 512), hout.data_ptr(), int(split3), nxt, nnext, ndots.data_ptr(), stream)
    else:
        act = torch.empty(m, T, 2048, dtype=torch.bfloat16, device=DEV)
        pd = torch.empty(rows, 16, dtype=torch.float32, device=DEV)
        _lib.call('noise_pop_fc', ctypes.byref(pop), V(c['h'], 512), c['wfc'].data_ptr(), ctypes.byref(r_fc),
                  dots.data_ptr(), act.data_ptr(), ctypes.byref(r_pj) if c['apj'] is not None else None, pd.data_ptr(),
                  stream)
        _lib.call('noise_pop_residual', ctypes.byref(pop), V(act, 2048), c['wpj'].data_ptr(), 2048, ctypes.byref(r_pj),
                  pd.data_ptr(), 16, 16, V(xres, 512), _lib.ptr(xout), *mixargs, V(c['x0'], 512), hout.data_ptr(),
                  int(split3), nxt, nnext, ndots.data_ptr(), stream)
    torch.cuda.synchronize()
    return (None if xout is None else xout.cpu()), hout.float().cpu(), ndots[:, :nnext].cpu()


def _fp32_reference(c, mix, nnext):
    """The same arithmetic in fp32 on the CPU from the same bf16 operands (hidden layer rounded to bf16)."""
    m, T = c['m'], c['T']
    h = c['h'].float().cpu()
    sign = c['sign'].cpu()[:, None, None]
    rep = lambda t: None if t is None else t.cpu().repeat_interleave(2, 0)
    hid = h @ c['wfc'].float().cpu().t()
    if c['afc'] is not None:
        hid = hid + sign * (h @ rep(c['bfc']).unsqueeze(-1)) * rep(c['afc'])[:, None, :]
    hid = torch.relu(hid).square().bfloat16().float()
    y = c['xres'].cpu() + hid @ c['wpj'].float().cpu().t()
    if c['apj'] is not None:
        b = rep(c['bpj']).bfloat16().float()
        y = y + sign * (hid @ b.unsqueeze(-1)) * rep(c['apj'])[:, None, :]
    if mix:
        rl, ml = c['lam'][0].item(), c['lam'][1].item()
        if c['eps'] is not None:
            e = rep(c['eps'])
            rl = rl + sign * e[:, 0, None, None]
            ml = ml + sign * e[:, 1, None, None]
        y = rl * y + ml * c['x0'].cpu()
    rstd = torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps)
    nd = (torch.stack([(y * rep(c['nb'][k])[:, None, :]).sum(-1) for k in range(nnext)], -1) * rstd).reshape(m * T, nnext) \
        if nnext else None
    return y, y * rstd, nd


@pytest.mark.parametrize('perturbed', [False, True], ids=['plain', 'perturbed'])
@pytest.mark.parametrize('mix,nnext,split3,with_xout', [(True, 3, False, True), (True, 0, False, True),
                                                        (False, 1, False, False), (False, 0, True, False)],
                         ids=['mix-qkv-dots', 'mix-no-dots', 'last-head-dot', 'last-split3'])
def test_fused_mlp_matches_two_kernel_path(perturbed, mix, nnext, split3, with_xout):
    c = _case(4, 256, 1, perturbed)
    print(f'fused MLP: 4 members x 256 tokens, perturbed {perturbed}, mix {mix}, nnext {nnext}, split3 {split3}',
          flush=True)
    xo_f, ho_f, nd_f = _run(c, True, mix, nnext, split3, with_xout)
    xo_r, ho_r, nd_r = _run(c, False, mix, nnext, split3, with_xout)
    y, hn, nd = _fp32_reference(c, mix, nnext)
    assert torch.isfinite(ho_f).all() and torch.isfinite(nd_f).all()
    scale = y.abs().max()
    if with_xout:
        assert (xo_f - xo_r).abs().max() <= 2e-3 * scale
        assert (xo_f - y).abs().max() <= 2e-3 * scale
    hi_f = ho_f[..., :512]
    hscale = hn.abs().max()
    # bf16 norm output: one bf16 ulp (2^-7 of the largest value) plus the fp32 differences of y
    assert (hi_f - ho_r[..., :512]).abs().max() <= (2.0 ** -7 + 2e-3) * hscale
    assert (hi_f - hn).abs().max() <= (2.0 ** -7 + 2e-3) * hscale
    if split3:
        # [hi | lo | hi]: hi + lo carries the fp32 norm output
        assert torch.equal(ho_f[..., 1024:], hi_f)
        assert (hi_f + ho_f[..., 512:1024] - hn).abs().max() <= 2e-3 * hscale
    if nnext:
        assert (nd_f - nd_r).abs().max() <= 2e-3 * nd.abs().max()
        assert (nd_f - nd).abs().max() <= 2e-3 * nd.abs().max()


def test_fused_mlp_rejects_bad_arguments():
    from noise_amd import _lib
    pop = _lib.Population(2, 200, None, 1, _lib.ROUNDING_FUSED)
    with pytest.raises(RuntimeError, match='multiple of 128'):
        _lib.call('noise_pop_mlp', ctypes.byref(pop), _lib.View(16, 0, 512), 16, None, None, 16, None,
                  _lib.View(16, 0, 512), None, 0, None, None, None, None, 0, _lib.View(16, 0, 512), 16, 0, None, 0,
                  None, None)
    pop = _lib.Population(2, 256, None, 1, _lib.ROUNDING_EAGER)
    with pytest.raises(RuntimeError, match='fused rounding only'):
        _lib.call('noise_pop_mlp', ctypes.byref(pop), _lib.View(16, 0, 512), 16, None, None, 16, None,
                  _lib.View(16, 0, 512), None, 0, None, None, None, None, 0, _lib.View(16, 0, 512), 16, 0, None, 0,
                  None, None)


def _attn_case(m, T, seed, perturbed):
    c = _case(m, T, seed, perturbed)
    g = torch.Generator().manual_seed(seed + 100)
    dirs = m // 2
    c['y'] = torch.randn(m, T, 512, generator=g).bfloat16().to(DEV)
    c['wo'] = ((torch.rand(512, 512, generator=g) * 2 - 1) * 1.5 * (3 / 512) ** 0.5).bfloat16().to(DEV)
    if perturbed:
        c['ao'] = torch.randn(dirs, 512, generator=g).to(DEV)
        c['odots'] = torch.randn(m * T, 8, generator=g).to(DEV)
    else:
        c['ao'] = c['odots'] = None
    return c


def _run_attn(c, fused, mix, nnext, split3, with_xout):
    """noise_pop_attn_mlp (fused) or noise_pop_residual (K = 512, with the c_fc dot) then noise_pop_mlp."""
    from noise_amd import _lib
    m, T = c['m'], c['T']
    rows = m * T
    stream = _lib.stream_ptr(DEV)
    pop = _lib.Population(m, T, c['sign'].data_ptr(), 2, _lib.ROUNDING_FUSED)
    V = lambda t, w: _lib.View(t.data_ptr(), T * w, w)
    R = lambda a, b: _lib.Rank1(None, None, 0, 0) if a is None else _lib.Rank1(a.data_ptr(), _lib.ptr(b), a.stride(0),
                                                                               0 if b is None else b.stride(0))
    r_o, r_fc, r_pj = R(c['ao'], None), R(c['afc'], c['bfc']), R(c['apj'], c['bpj'])
    nxt = (_lib.Rank1 * 3)(*[_lib.Rank1(None, t.data_ptr(), 0, t.stride(0)) for t in c['nb']])
    ndots = torch.full((rows, max(nnext, 1)), float('nan'), device=DEV)
    xres = c['xres'].clone()  # the block's residual input (also its output when with_xout)
    width = 1536 if split3 else 512
    hout = torch.full((m, T, width), float('nan'), dtype=torch.bfloat16, device=DEV)
    eps = c['eps']
    mixargs = (1, c['lam'].data_ptr(), c['lam'].data_ptr() + 4, None if eps is None else eps[:, 0].data_ptr(),
               None if eps is None else eps[:, 1].data_ptr(), 0 if eps is None else eps.stride(0)) if mix else \
        (0, None, None, None, None, 0)
    xout = xres if with_xout else None
    perm = {}
    for k in ('wfc', 'wpj'):
        perm[k] = torch.empty_like(c[k])
        _lib.call('noise_mlp_proj_layout', c[k].data_ptr(), perm[k].data_ptr(), c[k].numel() // 2048, stream)
    if fused:
        _lib.call('noise_pop_attn_mlp', ctypes.byref(pop), V(c['y'], 512), c['wo'].data_ptr(), ctypes.byref(r_o),
                  _lib.ptr(c['odots']), 8, V(xres, 512), perm['wfc'].data_ptr(), ctypes.byref(r_fc),
                  perm['wpj'].data_ptr(), ctypes.byref(r_pj), _lib.ptr(xout), *mixargs, V(c['x0'], 512),
                  hout.data_ptr(), int(split3), nxt, nnext, ndots.data_ptr(), stream)
    else:
        xmid = torch.empty(m, T, 512, device=DEV)
        h = torch.empty(m, T, 512, dtype=torch.bfloat16, device=DEV)
        dfc = torch.zeros(rows, device=DEV)
        fcb = (_lib.Rank1 * 1)(_lib.Rank1(None, c['bfc'].data_ptr(), 0, c['bfc'].stride(0))) if c['bfc'] is not None \
            else None
        _lib.call('noise_pop_residual', ctypes.byref(pop), V(c['y'], 512), c['wo'].data_ptr(), 512, ctypes.byref(r_o),
                  _lib.ptr(c['odots']), 8, 8, V(xres, 512), xmid.data_ptr(), 0, None, None, None, None, 0,
                  V(c['x0'], 512), h.data_ptr(), 0, fcb, 1 if fcb is not None else 0, dfc.data_ptr(), stream)
        _lib.call('noise_pop_mlp', ctypes.byref(pop), V(h, 512), c['wfc'].data_ptr(), ctypes.byref(r_fc),
                  dfc.data_ptr(), perm['wpj'].data_ptr(), ctypes.byref(r_pj), V(xmid, 512), _lib.ptr(xout), *mixargs,
                  V(c['x0'], 512), hout.data_ptr(), int(split3), nxt, nnext, ndots.data_ptr(), stream)
    torch.cuda.synchronize()
    return (None if xout is None else xout.cpu()), hout.float().cpu(), ndots[:, :nnext].cpu()


@pytest.mark.parametrize('perturbed', [False, True], ids=['plain', 'perturbed'])
@pytest.mark.parametrize('mix,nnext,split3,with_xout', [(True, 3, False, True), (True, 0, False, True),
                                                        (False, 1, False, False), (False, 0, True, False)],
                         ids=['mix-qkv-dots', 'mix-no-dots', 'last-head-dot', 'last-split3'])
def test_attn_mlp_matches_residual_then_mlp(perturbed, mix, nnext, split3, with_xout):
    """noise_pop_attn_mlp (attention projection, residual, norm and the MLP in one kernel) against
    noise_pop_residual with K = 512 followed by noise_pop_mlp on the same inputs. The two round h to bf16 from
    fp32 values summed in different orders, so a hidden value can round one bf16 ulp apart: outputs agree to
    2e-3 of their scale, as the fused MLP does against its two-kernel form."""
    c = _attn_case(4, 256, 2, perturbed)
    print(f'attn+MLP: 4 members x 256 tokens, perturbed {perturbed}, mix {mix}, nnext {nnext}, split3 {split3}',
          flush=True)
    xo_f, ho_f, nd_f = _run_attn(c, True, mix, nnext, split3, with_xout)
    xo_r, ho_r, nd_r = _run_attn(c, False, mix, nnext, split3, with_xout)
    assert torch.isfinite(ho_f).all() and torch.isfinite(nd_f).all()
    if with_xout:
        scale = xo_r.abs().max()
        assert (xo_f - xo_r).abs().max() <= 2e-3 * scale
    hscale = ho_r[..., :512].abs().max()
    assert (ho_f[..., :512] - ho_r[..., :512]).abs().max() <= (2.0 ** -7 + 2e-3) * hscale
    if split3:
        assert torch.equal(ho_f[..., 1024:], ho_f[..., :512])
        assert (ho_f[..., :512] + ho_f[..., 512:1024] - ho_r[..., :512] - ho_r[..., 512:1024]).abs().max() <= 2e-3 * hscale
    if nnext:
        assert (nd_f - nd_r).abs().max() <= 2e-3 * nd_r.abs().max()


def test_attn_mlp_block0_shared_residual():
    """Block 0's residual input is shared by all members (member stride 0): every member reads the same rows."""
    from noise_amd import _lib
    c = _attn_case(2, 128, 5, True)
    shared = c['xres'][:1].contiguous()
    m, T = 2, 128
    pop = _lib.Population(m, T, c['sign'].data_ptr(), 2, _lib.ROUNDING_FUSED)
    copied = shared.expand(m, T, 512).contiguous()
    out = {}
    for name, xr in (('shared', _lib.View(shared.data_ptr(), 0, 512)),
                     ('copied', _lib.View(copied.data_ptr(), T * 512, 512))):
        perm = {}
        for k in ('wfc', 'wpj'):
            perm[k] = torch.empty_like(c[k])
            _lib.call('noise_mlp_proj_layout', c[k].data_ptr(), perm[k].data_ptr(), c[k].numel() // 2048,
                      _lib.stream_ptr(DEV))
        xo = torch.empty(m, T, 512, device=DEV)
        h = torch.empty(m, T, 512, dtype=torch.bfloat16, device=DEV)
        r_o = _lib.Rank1(c['ao'].data_ptr(), None, 512, 0)
        r_fc = _lib.Rank1(c['afc'].data_ptr(), c['bfc'].data_ptr(), 2048, 512)
        r_pj = _lib.Rank1(c['apj'].data_ptr(), c['bpj'].data_ptr(), 512, 2048)
        _lib.call('noise_pop_attn_mlp', ctypes.byref(pop), _lib.View(c['y'].data_ptr(), T * 512, 512),
                  c['wo'].data_ptr(), ctypes.byref(r_o), c['odots'].data_ptr(), 8, xr, perm['wfc'].data_ptr(),
                  ctypes.byref(r_fc), perm['wpj'].data_ptr(), ctypes.byref(r_pj), xo.data_ptr(), 0, None, None, None,
                  None, 0, _lib.View(c['x0'].data_ptr(), T * 512, 512), h.data_ptr(), 0, None, 0, None,
                  _lib.stream_ptr(DEV))
        torch.cuda.synchronize()
        out[name] = (xo.cpu(), h.cpu())
    assert torch.equal(out['shared'][0], out['copied'][0]) and torch.equal(out['shared'][1], out['copied'][1])


def _run_block(c, mix, nnext, split3, with_xout, kernel):
    """noise_pop_block (two waves per SIMD) or noise_pop_attn_mlp on the same inputs."""
    from noise_amd import _lib
    m, T = c['m'], c['T']
    rows = m * T
    stream = _lib.stream_ptr(DEV)
    pop = _lib.Population(m, T, c['sign'].data_ptr(), 2, _lib.ROUNDING_FUSED)
    V = lambda t, w: _lib.View(t.data_ptr(), T * w, w)
    R = lambda a, b: _lib.Rank1(None, None, 0, 0) if a is None else _lib.Rank1(a.data_ptr(), _lib.ptr(b), a.stride(0),
                                                                               0 if b is None else b.stride(0))
    r_o, r_fc, r_pj = R(c['ao'], None), R(c['afc'], c['bfc']), R(c['apj'], c['bpj'])
    nxt = (_lib.Rank1 * 3)(*[_lib.Rank1(None, t.data_ptr(), 0, t.stride(0)) for t in c['nb']])
    ndots = torch.full((rows, max(nnext, 1)), float('nan'), device=DEV)
    xres = c['xres'].clone()
    width = 1536 if split3 else 512
    hout = torch.full((m, T, width), float('nan'), dtype=torch.bfloat16, device=DEV)
    eps = c['eps']
    mixargs = (1, c['lam'].data_ptr(), c['lam'].data_ptr() + 4, None if eps is None else eps[:, 0].data_ptr(),
               None if eps is None else eps[:, 1].data_ptr(), 0 if eps is None else eps.stride(0)) if mix else \
        (0, None, None, None, None, 0)
    xout = xres if with_xout else None
    perm = {}
    for k in ('wfc', 'wpj'):
        perm[k] = torch.empty_like(c[k])
        if kernel == 'noise_pop_block':
            _lib.call('noise_block_weight_layout', c[k].data_ptr(), perm[k].data_ptr(), c[k].shape[0], c[k].shape[1],
                      stream)
        else:
            _lib.call('noise_mlp_proj_layout', c[k].data_ptr(), perm[k].data_ptr(), c[k].numel() // 2048, stream)
    _lib.call(kernel, ctypes.byref(pop), V(c['y'], 512), c['wo'].data_ptr(), ctypes.byref(r_o),
              _lib.ptr(c['odots']), 8, V(xres, 512), perm['wfc'].data_ptr(), ctypes.byref(r_fc),
              perm['wpj'].data_ptr(), ctypes.byref(r_pj), _lib.ptr(xout), *mixargs, V(c['x0'], 512),
              hout.data_ptr(), int(split3), nxt, nnext, ndots.data_ptr(), stream)
    torch.cuda.synchronize()
    return (None if xout is None else xout.cpu()), hout.float().cpu(), ndots[:, :nnext].cpu()


def test_block_weight_layout():
    """noise_block_weight_layout: within every 32 columns, position 8g + j holds column 4g + j (j < 4) or
    16 + 4g + j - 4 (j >= 4)."""
    from noise_amd import _lib
    w = torch.arange(3 * 64, dtype=torch.float32).view(3, 64).bfloat16().to(DEV)
    out = torch.empty_like(w)
    _lib.call('noise_block_weight_layout', w.data_ptr(), out.data_ptr(), 3, 64, _lib.stream_ptr(DEV))
    perm = [4 * (p // 8) + p % 8 if p % 8 < 4 else 16 + 4 * (p // 8) + p % 8 - 4 for p in range(32)]
    idx = torch.tensor(perm + [32 + q for q in perm])
    assert torch.equal(out.cpu(), w.cpu()[:, idx])


@pytest.mark.parametrize('perturbed', [False, True], ids=['plain', 'perturbed'])
@pytest.mark.parametrize('mix,nnext,split3,with_xout', [(True, 3, False, True), (True, 0, False, True),
                                                        (False, 1, False, False), (False, 0, True, False)],
                         ids=['mix-qkv-dots', 'mix-no-dots', 'last-head-dot', 'last-split3'])
def test_block_matches_attn_mlp(perturbed, mix, nnext, split3, with_xout):
    """noise_pop_block against noise_pop_attn_mlp (itself checked against the residual writer + fused MLP pair):
    the same arithmetic with fp32 sums in a different order, so h and the hidden layer can round one bf16 ulp
    apart; outputs agree to 2e-3 of their scale. Also bit-stable across two calls."""
    c = _attn_case(4, 256, 3, perturbed)
    print(f'block: 4 members x 256 tokens, perturbed {perturbed}, mix {mix}, nnext {nnext}, split3 {split3}', flush=True)
    xo_b, ho_b, nd_b = _run_block(c, mix, nnext, split3, with_xout, 'noise_pop_block')
    xo_r, ho_r, nd_r = _run_block(c, mix, nnext, split3, with_xout, 'noise_pop_attn_mlp')
    assert torch.isfinite(ho_b).all() and torch.isfinite(nd_b).all()
    if with_xout:
        assert (xo_b - xo_r).abs().max() <= 2e-3 * xo_r.abs().max()
    hscale = ho_r[..., :512].abs().max()
    assert (ho_b[..., :512] - ho_r[..., :512]).abs().max() <= (2.0 ** -7 + 2e-3) * hscale
    if split3:
        assert torch.equal(ho_b[..., 1024:], ho_b[..., :512])
        assert (ho_b[..., :512] + ho_b[..., 512:1024] - ho_r[..., :512] - ho_r[..., 512:1024]).abs().max() <= 2e-3 * hscale
    if nnext:
        assert (nd_b - nd_r).abs().max() <= 2e-3 * nd_r.abs().max()
    again = _run_block(c, mix, nnext, split3, with_xout, 'noise_pop_block')
    assert torch.equal(again[1], ho_b) and torch.equal(again[2], nd_b)
