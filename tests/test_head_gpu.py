"""noise_pop_head_ce at K = 512 (the bf16 head, eggroll.py:94-101 / model.py:202-209) against the same
arithmetic in fp32 on the CPU from the same bf16 operands: logits = x W^T (+ sign (x . b) a for a perturbed
head), z = 15 tanh(logits / 15), per-token CE = logsumexp(z) - z[target], 0 for target -1 and NaN for an id
outside [0, vocab). The kernel accumulates the products in fp32 in its own order: per-token losses agree to
5e-5 (measured ~1e-6). With eager rounding the logits are rounded to bf16 first; a logit whose fp32 sums
straddle a bf16 rounding boundary rounds one ulp apart, so there the per-token bound is loose and the row
mean carries the check."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def _reference(x, w, targets, sign=None, dots=None, a=None, eager=False):
    logits = x.float() @ w.float().t()
    if eager:
        logits = logits.bfloat16().float()
    if a is not None:
        logits = logits + (sign[:, None] * dots.view(sign.shape[0], -1))[..., None] * a.repeat_interleave(2, 0)[:, None, :]
    z = 15 * torch.tanh(logits / 15)
    lse = torch.logsumexp(z, -1)
    t = targets.clamp(0, w.shape[0] - 1)
    zt = z.gather(-1, t.expand(z.shape[0], -1)[..., None])[..., 0]
    ce = lse - zt
    ce = torch.where(targets == -1, torch.zeros_like(ce), ce)
    return torch.where((targets < -1) | (targets >= w.shape[0]), torch.full_like(ce, float('nan')), ce)


def _run(x, w, targets, sign=None, dots=None, a=None, b=None, eager=False):
    from noise_amd import _lib
    m, T, K = x.shape
    xd, wd, td = x.to(DEV), w.to(DEV), targets.to(DEV)
    loss = torch.full((m * T,), -7.0, device=DEV)
    rounding = _lib.ROUNDING_EAGER if eager else _lib.ROUNDING_FUSED
    sd = None if sign is None else sign.to(DEV)
    pop = _lib.Population(m, T, _lib.ptr(sd), 2, rounding)
    r1 = None
    if a is not None:
        ad, bd = a.to(DEV).contiguous(), b.to(DEV).contiguous()
        r1 = _lib.Rank1(ad.data_ptr(), bd.data_ptr(), ad.stride(0), bd.stride(0))
    dd = None if dots is None else dots.to(DEV)
    _lib.call('noise_pop_head_ce', ctypes.byref(pop), _lib.View(xd.data_ptr(), T * K, K), wd.data_ptr(), K, w.shape[0],
              None if r1 is None else ctypes.byref(r1), _lib.ptr(dd), td.data_ptr(), 0, loss.data_ptr(),
              _lib.stream_ptr(DEV))
    torch.cuda.synchronize()
    return loss.view(m, T).cpu()


def _case(seed, m=4, T=256):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, T, 512, generator=g).bfloat16()
    w = (torch.randn(4096, 512, generator=g) * 0.4).bfloat16()  # logits of a few tens: the soft cap is active
    targets = torch.randint(0, 4096, (T,), generator=g)
    targets[3], targets[10], targets[200] = -1, 4095, 0
    return g, x, w, targets


@pytest.mark.parametrize('perturbed', [False, True], ids=['plain', 'perturbed'])
def test_bf16_head_matches_fp32_reference(perturbed):
    g, x, w, targets = _case(11)
    print(f'head K=512: 4 members x 256 tokens, perturbed {perturbed}', flush=True)
    kw = {}
    if perturbed:
        a = torch.randn(2, 4096, generator=g)
        b = torch.randn(2, 512, generator=g)
        sign = torch.tensor([0.05, -0.05, 0.05, -0.05])
        dots = (x.float() @ b.repeat_interleave(2, 0)[:, :, None])[..., 0].reshape(-1)
        kw = dict(sign=sign, dots=dots, a=a)
        got = _run(x, w, targets, sign=sign, dots=dots, a=a, b=b)
    else:
        got = _run(x, w, targets)
    ref = _reference(x, w, targets, **kw)
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    ok = ~torch.isnan(ref)
    assert (got[ok] - ref[ok]).abs().max().item() <= 5e-5
    assert (got[:, 3] == 0).all()


def test_bf16_head_out_of_range_target_is_nan():
    g, x, w, targets = _case(12, m=2)
    targets[7], targets[8] = 4096, -2
    got = _run(x, w, targets)
    assert torch.isnan(got[:, 7]).all() and torch.isnan(got[:, 8]).all()
    ref = _reference(x, w, targets)
    ok = ~torch.isnan(ref)
    assert (got[ok] - ref[ok]).abs().max().item() <= 5e-5


def test_bf16_head_eager_rounding():
    g, x, w, targets = _case(13)
    got = _run(x, w, targets, eager=True)
    ref = _reference(x, w, targets, eager=True)
    ok = ~torch.isnan(ref)
    diff = (got[ok] - ref[ok]).abs()
    assert (diff <= 5e-5).float().mean().item() >= 0.99
    assert diff.max().item() <= 0.1
    assert (got - ref).nan_to_num().mean(-1).abs().max().item() <= 1e-4


def _split(v):
    hi = v.bfloat16()
    return hi, (v - hi.float()).bfloat16()


@pytest.mark.parametrize('perturbed', [False, True], ids=['plain', 'perturbed'])
def test_split3_head_matches_fp64_reference(perturbed):
    """K = 1536, the split-bf16x3 fp32 head: x rows [hi | lo | hi], w rows [hi | hi | lo] (noise_split3's layouts).
    Against the same three products summed in float64 on the CPU: per-token losses within 5e-5 (fp32
    accumulation in the kernel's own order); against the unsplit fp32 logits within 2e-4 (the split's own error,
    ~2^-16 relative per product). The third x segment repeats hi and is not read: it holds NaN here."""
    g = torch.Generator().manual_seed(23)
    m, T, V = 4, 256, 4096
    x = torch.randn(m, T, 512, generator=g)
    w = torch.randn(V, 512, generator=g) * 0.4
    targets = torch.randint(0, V, (T,), generator=g)
    targets[5], targets[77], targets[130] = -1, V - 1, V + 3
    xh, xl = _split(x)
    wh, wl = _split(w)
    x3 = torch.cat([xh, xl, torch.full_like(xh, float('nan'))], -1)
    w3 = torch.cat([wh, wh, wl], -1)
    logits = (xh.double() @ wh.double().t() + xl.double() @ wh.double().t() + xh.double() @ wl.double().t())
    exact = x.double() @ w.double().t()
    kw = {}
    if perturbed:
        a = torch.randn(2, V, generator=g)
        b = torch.randn(2, 512, generator=g)
        sign = torch.tensor([0.05, -0.05, 0.05, -0.05])
        dots = (x @ b.repeat_interleave(2, 0)[:, :, None])[..., 0].reshape(-1)
        r1 = (sign[:, None] * dots.view(m, -1))[..., None].double() * a.repeat_interleave(2, 0)[:, None, :].double()
        logits, exact = logits + r1, exact + r1
        kw = dict(sign=sign, dots=dots, a=a, b=b)
    print(f'head K=1536 (split-bf16x3): {m} members x {T} tokens, perturbed {perturbed}', flush=True)
    got = _run(x3, w3, targets, **kw)

    def ce(lg):
        z = 15 * torch.tanh(lg / 15)
        t = targets.clamp(0, V - 1)
        out = torch.logsumexp(z, -1) - z.gather(-1, t.expand(m, -1)[..., None])[..., 0]
        out = torch.where(targets == -1, torch.zeros_like(out), out)
        return torch.where((targets < -1) | (targets >= V), torch.full_like(out, float('nan')), out).float()

    ref, ref_exact = ce(logits), ce(exact)
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    ok = ~torch.isnan(ref)
    assert (got[ok] - ref[ok]).abs().max().item() <= 5e-5
    assert (got[ok] - ref_exact[ok]).abs().max().item() <= 2e-4
    assert (got[:, 5] == 0).all()
