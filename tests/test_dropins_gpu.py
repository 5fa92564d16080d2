"""The reference's call-site functions on the GPU vs the oracle / torch's own generators.

lowrank (eggroll.py:56-58), lowrank_embed (61-63), head_loss (run.py:89-94), Eggroll.offsets / noise
(eggroll.py:117-128).
"""
import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def bits(t):
    return t.contiguous().view(torch.int32)


@pytest.mark.parametrize('shared', [False, True])
def test_lowrank_vs_oracle(shared):
    """y = x W^T + sign (x b) a^T; bf16 operands, fp32 output. Tolerance: 1e-2 of the output's max
    magnitude (bf16 inputs), and the rank-1 term itself to 2e-2 of its scale."""
    from noise_amd.eggroll import lowrank
    g = torch.Generator().manual_seed(0)
    m, T, n_in, n_out = 4, 512, 512, 2048
    # per-member x, equal within each antithetic pair (as members of a pair see one sequence)
    x = torch.randn(1 if shared else m // 2, T, n_in, generator=g)
    x = x.expand(m, T, n_in) if shared else x.repeat_interleave(2, 0)
    w = torch.randn(n_out, n_in, generator=g) * 0.02
    a, b = torch.randn(m // 2, n_out, generator=g), torch.randn(m // 2, n_in, generator=g)
    sign = torch.tensor([1e-2, -1e-2] * (m // 2))
    xd = x.to(DEV) if not shared else x[:1].to(DEV).expand(m, T, n_in)
    y = lowrank(xd, w.to(DEV), a.to(DEV), b.to(DEV), sign.to(DEV), dir_div=2).cpu()
    xr = x.bfloat16().float()
    ref = om.lowrank(xr, w.bfloat16().float(), a.repeat_interleave(2, 0), b.repeat_interleave(2, 0), sign)
    scale = ref.abs().max()
    assert (y - ref).abs().max() <= 1e-2 * scale
    # antithetic: y+ + y- = 2 x W^T (the rank-1 terms cancel) and y+ - y- = 2 sigma (x b) a^T
    d = (y[0] - y[1]) / 2
    rank1 = 1e-2 * (xr[0] @ b[0])[:, None] * a[0][None, :]
    assert (d - rank1).abs().max() <= 2e-2 * rank1.abs().max()


@pytest.mark.parametrize('dir_div,y_fp32,T,width', [(1, 1, 10, 1028), (3, 0, 7, 2048), (2, 2, 9, 4), (2, 0, 12, 1040)])
def test_rank1_expand_generic(dir_div, y_fp32, T, width):
    """noise_rank1_expand against the formula on shapes off the population's: directions of 1 or 3 members
    (and a last direction with fewer), token counts that end inside a 4-row tile, widths that end inside a
    1024-column tile, bf16 output and the dot rounded to bf16 (y_fp32 = 2). fp32: exact up to the fma
    contraction (1e-6 relative); bf16: one bf16 ulp."""
    import ctypes
    from noise_amd import _lib
    g = torch.Generator().manual_seed(11)
    m = 7
    dirs = -(-m // dir_div)
    base = torch.randn(T, width, generator=g)
    a = torch.randn(dirs, width, generator=g)
    dots = torch.randn(T, dirs + 3, generator=g)  # row stride larger than the directions
    sign = torch.randn(m, generator=g)
    bd, ad, dd, sd = (t.to(DEV).contiguous() for t in (base, a, dots, sign))
    y = torch.empty(m, T, width, dtype=torch.float32 if y_fp32 else torch.bfloat16, device=DEV)
    pop = _lib.Population(m, T, sd.data_ptr(), dir_div)
    r1 = _lib.Rank1(ad.data_ptr(), None, width, 0)
    _lib.call('noise_rank1_expand', ctypes.byref(pop), bd.data_ptr(), width, dd.data_ptr(), dirs + 3,
              ctypes.byref(r1), y.data_ptr(), y_fp32, _lib.stream_ptr(DEV))
    dir_of = torch.arange(m) // dir_div
    dv = dots[:, dir_of].t()                       # [m, T]
    if y_fp32 == 2:
        dv = dv.bfloat16().float()
    ref = base[None] + (sign[:, None] * dv)[:, :, None] * a[dir_of][:, None, :]
    out = y.float().cpu()
    if y_fp32:
        assert torch.allclose(out, ref, rtol=1e-6, atol=1e-6)
    else:
        assert torch.equal(out, ref.bfloat16().float()) or (out - ref).abs().max() <= ref.abs().max() * 2.0 ** -8


def test_lowrank_embed_exact():
    from noise_amd.eggroll import lowrank_embed
    g = torch.Generator().manual_seed(1)
    W = torch.randn(4096, 512, generator=g)
    a, b = torch.randn(3, 4096, generator=g), torch.randn(3, 512, generator=g)
    idx = torch.randint(0, 4096, (300,), generator=g)
    sign = torch.tensor([0.1, -0.2, 0.3])
    out = lowrank_embed(W.to(DEV), a.to(DEV), b.to(DEV), idx.to(DEV), sign.to(DEV)).cpu()
    ref = om.lowrank_embed(W, a, b, idx, sign)
    assert torch.allclose(out, ref, rtol=1e-6, atol=1e-6)


def test_head_loss_fp32_precision():
    """Large logits (|z| up to the cap): split-bf16x3 matches the fp32 oracle to 2e-4 per token, where a
    plain bf16 head is off by far more (checked) -- the test discriminates the two."""
    from noise_amd.dust import head_loss
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, 512, 512, generator=g)
    w = torch.randn(4096, 512, generator=g) * 0.3
    y = torch.randint(0, 4096, (3, 512), generator=g)
    y[0, :7] = -1
    got = head_loss(x.to(DEV), w.to(DEV), y.to(DEV), 4096).cpu()
    ref = om.head_loss(x, w, y)
    assert got.shape == ref.shape == (3 * 512,)
    assert (got - ref).abs().max() <= 2e-4
    assert (got.view(3, 512)[0, :7] == 0).all()
    bf16_ref = om.softcap_ce((om.norm(x).bfloat16().float() @ w.bfloat16().float().t()), y, 'none')
    assert (bf16_ref - ref).abs().max() > 10 * 2e-4


def test_head_loss_ragged_rows():
    from noise_amd.dust import head_loss
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 100, 512, generator=g)
    w = torch.randn(4096, 512, generator=g) * 0.05
    y = torch.randint(0, 4096, (1, 100), generator=g)
    got = head_loss(x.to(DEV), w.to(DEV), y.to(DEV), 4096).cpu()
    assert (got - om.head_loss(x, w, y)).abs().max() <= 2e-4


def test_eggroll_offsets_and_noise_bit_exact():
    """Offsets = torch.randint on a cuda generator seeded 1_000_003*SEED + step, one draw per parameter in
    named_parameters order; noise rows = the reference buffer's slices. Checked against torch's own device
    draws (the buffer materialised here only as the reference)."""
    from noise_amd.eggroll import Eggroll
    from noise_amd.model import make_model
    model = make_model('cpu', 0).to(DEV)
    pairs = 512
    es = Eggroll(model, pairs)
    offs = es.offsets(3)
    g = torch.Generator(DEV).manual_seed(1_000_003 * 0 + 3)
    params = dict(model.named_parameters())
    NOISE = 2 ** 28
    for name, p in params.items():
        ref = torch.randint(0, NOISE - sum(p.shape), (pairs,), device=DEV, generator=g)
        assert torch.equal(offs[name], ref), name
    buffer = torch.randn(NOISE, device=DEV, generator=torch.Generator(DEV).manual_seed(0))
    directions = torch.arange(256, 256 + 64, 2, device=DEV) % (2 * pairs) // 2
    noise = es.noise(offs, directions)
    for name in ('resid_lambdas', 'transformer.wte.weight', 'transformer.h.3.mlp.c_fc.weight', 'lm_head.weight',
                 'value_embeds.7.weight', 'transformer.h.7.attn.ve_gate.weight'):
        p = params[name]
        rows = buffer[offs[name][directions, None] + torch.arange(sum(p.shape), device=DEV)]
        ref = rows.split(list(p.shape), dim=1) if p.dim() == 2 else (rows,)
        got = noise[name] if p.dim() == 2 else (noise[name],)
        for r, o in zip(ref, got):
            assert torch.equal(bits(o), bits(r)), name


def test_custom_ops_compile_without_graph_breaks():
    """torch.compile(fullgraph=True) over the registered ops (the reference compiles its callers)."""
    import noise_amd.ops  # noqa: F401

    def f(q, k, v):
        return torch.ops.noise_amd.attention(q, k, v, 64).float().sum(-1)

    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(1, 256, 8, 64, generator=g).bfloat16().to(DEV) for _ in range(3))
    compiled = torch.compile(f, fullgraph=True, backend='aot_eager')
    assert torch.equal(compiled(q, k, v), f(q, k, v))


def test_config3_antithetic_linear_full_size():
    """The antithetic perturbed linear at full size: X bf16 [2048, 512] ~ N(0, 1) and W bf16 [2048 out,
    512 in] ~ N(0, 0.02^2) from one CPU generator seeded 0 (X drawn first); 256 pairs (512 members),
    sigma = 1e-3; a [2048], b [512] per pair sliced from the seed-0 noise buffer at offsets drawn by
    torch.randint(0, 2^28 - 2560) on a cuda generator seeded 0 (eggroll.py:117-128 for one parameter of
    this shape). Output [512, 2048, 2048] fp32 (8.6 GB).

    lowrank returns autocast's form (the reference runs it under torch.autocast): y = bf16(x W^T) +
    sign * bf16(x . bf16(b)) * a. Size-independent checks: the slices are bit-exact against torch's own
    device draws; every pair's sum y+ + y- equals 2 bf16(x W^T) (the rank-1 terms cancel; the fp32 product
    of the same bf16 operands rounded to bf16, within one bf16 ulp where the two fp32 sums round apart);
    every pair's difference (y+ - y-) / 2 equals sigma bf16(x . b) a^T (within one bf16 ulp of the dot;
    both bounds also allow the fp32 sums' order-dependent error, 2^-20 of the sum of the terms' magnitudes);
    four members checked whole against the formula."""
    from noise_amd.eggroll import lowrank
    from noise_amd.noise import DeviceGenerator
    g = torch.Generator().manual_seed(0)
    X = torch.randn(2048, 512, generator=g).bfloat16()
    W = (torch.randn(2048, 512, generator=g) * 0.02).bfloat16()
    pairs, sigma, NOISE = 256, 1e-3, 2 ** 28
    offs = torch.randint(0, NOISE - 2560, (pairs,), device=DEV, generator=torch.Generator(DEV).manual_seed(0))
    rows = DeviceGenerator(0, DEV).take(NOISE).gather(offs, 2560)
    a, b = rows[:, :2048], rows[:, 2048:]
    ref_buffer = torch.randn(NOISE, device=DEV, generator=torch.Generator(DEV).manual_seed(0))
    ref_rows = ref_buffer[offs[:, None] + torch.arange(2560, device=DEV)]
    assert torch.equal(bits(rows), bits(ref_rows))
    del ref_buffer, ref_rows
    print('config 3: 512 members x 2048 tokens x 2048 features', flush=True)
    sign = torch.tensor([sigma, -sigma], device=DEV).repeat(pairs)
    xd = X.to(DEV)
    y = lowrank(xd[None].expand(2 * pairs, 2048, 512), W.to(DEV), a, b, sign, dir_div=2)
    assert y.shape == (512, 2048, 2048) and torch.isfinite(y).all()
    prod = xd.float() @ W.to(DEV).float().t()
    base = prod.bfloat16().float()
    scale = base.abs().max()
    xb32 = xd.float() @ b.bfloat16().float().t()  # [2048 tokens, 256 pairs], fp32 sums of the bf16 operands
    xb = xb32.bfloat16().float()
    # one bf16 ulp of each product (where two fp32 sums straddle a rounding boundary they round apart), plus
    # the fp32 sums' own order-dependent error, at most ~2^-20 of the sum of the terms' magnitudes
    ulp_prod = prod.abs() * 2.0 ** -7 + (xd.float().abs() @ W.to(DEV).float().abs().t()) * 2.0 ** -20 + 1e-30
    xb_abs = xd.float().abs() @ b.bfloat16().float().abs().t()
    worst_sum = worst_diff = 0.0
    for i in range(pairs):
        s = (y[2 * i] + y[2 * i + 1]) * 0.5
        d = (y[2 * i] - y[2 * i + 1]) * 0.5
        r1 = sigma * xb[:, i, None] * a[i][None, :]
        # (B + r) + (B - r) in fp32 also carries the fp32 rounding of the two sums, ~2^-23 |r| each
        worst_sum = max(worst_sum, ((s - base).abs() / (ulp_prod + r1.abs() * 2.0 ** -22)).max().item())
        ulp_r1 = sigma * (xb32[:, i, None].abs() * 2.0 ** -7 + xb_abs[:, i, None] * 2.0 ** -20) * a[i][None, :].abs()
        worst_diff = max(worst_diff, ((d - r1).abs() / (ulp_r1 + 1e-6 * r1.abs().max())).max().item())
    print(f'config 3: worst pair-sum error {worst_sum:.2f} ulp, worst rank-1 error {worst_diff:.2f} ulp', flush=True)
    assert worst_sum <= 1.01
    assert worst_diff <= 1.01
    for mbr in (0, 1, 255, 511):
        i = mbr // 2
        ref = base + sign[mbr] * xb[:, i, None] * a[i][None, :]
        assert ((y[mbr] - ref).abs().max() / scale).item() <= 2.0 ** -7, mbr


@pytest.mark.parametrize('members,tokens,dir_div,nk,width', [(1024, 256, 2, 3, 512), (7, 100, 2, 2, 1024),
                                                             (5, 64, 1, 1, 512)])
def test_member_dots_shared_rows(members, tokens, dir_div, nk, width):
    """noise_member_dots with rows every member shares (member stride 0: one dot per token and direction,
    written to each member of the direction) against float64 sums and against the per-member kernel on the
    same rows repeated per member; ragged token and direction counts included."""
    import ctypes
    from noise_amd import _lib
    print(f'member dots: {members} members x {tokens} tokens, dir_div {dir_div}, {nk} vectors, width {width}',
          flush=True)
    g = torch.Generator().manual_seed(members + tokens)
    dirs = -(-members // dir_div)
    x = torch.randn(tokens, width, generator=g).bfloat16()
    bs = [torch.randn(dirs, width + 4, generator=g)[:, :width] for _ in range(nk)]  # strided rows
    sign = torch.ones(members)
    xd, sd = x.to(DEV), sign.to(DEV)
    bd = [b.to(DEV) for b in bs]
    vecs = (_lib.Rank1 * 3)(*[_lib.Rank1(None, b.data_ptr(), 0, b.stride(0)) for b in bd])
    pop = _lib.Population(members, tokens, sd.data_ptr(), dir_div, _lib.ROUNDING_FUSED)
    stream = _lib.stream_ptr(DEV)
    out = torch.full((members * tokens, nk), float('nan'), device=DEV)
    _lib.call('noise_member_dots', ctypes.byref(pop), _lib.View(xd.data_ptr(), 0, width), width, vecs, nk,
              out.data_ptr(), stream)
    xr = xd.unsqueeze(0).expand(members, tokens, width).contiguous()
    ref_k = torch.full_like(out, float('nan'))
    _lib.call('noise_member_dots', ctypes.byref(pop), _lib.View(xr.data_ptr(), tokens * width, width), width, vecs, nk,
              ref_k.data_ptr(), stream)
    torch.cuda.synchronize()
    got = out.cpu().view(members, tokens, nk)
    mdir = torch.arange(members) // dir_div
    ref = torch.stack([x.double() @ b.double().t() for b in bs], -1)[:, mdir].permute(1, 0, 2)  # [m, T, nk]
    scale = ref.abs().max().item()
    assert torch.isfinite(got).all()
    assert (got.double() - ref).abs().max().item() <= 1e-5 * scale
    assert (got - ref_k.cpu().view(members, tokens, nk)).abs().max().item() <= 1e-5 * scale
