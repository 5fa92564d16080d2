"""The drop-in boundary at the reference's own call sites, on the GPU.

- A compiled caller of the reference's shape (eggroll.py:115, 133-146): a population evaluated chunk by chunk
  under torch.compile and bf16 autocast, per-member noise of all 60 parameters, member g on direction
  (g mod 2P) // 2 with sign +-sigma. Run twice: with the fused population_loss drop-in, and with a population
  forward composed from the lowrank / lowrank_embed / attention drop-ins (the oracle's composition, given the
  drop-ins as its ops), so every linear call site -- the value-embedding gate's lowrank on h[..., :32]
  included -- goes through this library. Both stay within 1e-3 of the fp32 oracle for every member.
- Eggroll.population's member -> direction, sign and sequence mapping (eggroll.py:134-146) with 8
  sequences, three chunks per rank and two rank slices, against the oracle on noise gathered per member
  from the mapping's closed form.
- lowrank in autocast's form for every shape (eggroll.py:56-58 under eggroll.py:144), block_forward and
  coordinate_differences behind torch.compile (run.py:102, 120), token ids outside the vocabulary, and
  the device make_model's bf16 embedding storage (utils/model.py:171-175).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import model as om

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)
TOL = 1e-3


def _bf(t):
    return t.bfloat16().float()


@pytest.fixture(scope='module')
def model():
    """Seed-0 model with the head scaled x30 (so losses depend on the hidden state) and non-zero value-embedding
    gates (so the gate path matters), on the GPU."""
    from noise_amd.model import make_model
    m = make_model('cpu', 0)
    with torch.no_grad():
        m.lm_head.weight.mul_(30)
        g = torch.Generator().manual_seed(11)
        for blk in m.transformer.h:
            if blk.attn.ve_gate is not None:
                blk.attn.ve_gate.weight.copy_(torch.randn(8, 32, generator=g) * 0.3)
    return m.to(DEV)


def _cpu_params(model):
    return {k: v.detach().float().cpu() for k, v in model.named_parameters()}


def _cpu_noise(noise):
    return {n: (tuple(t.cpu() for t in v) if isinstance(v, tuple) else v.cpu()) for n, v in noise.items()}


class DropIns:
    """The library's drop-ins in the roles the composed population forward gives its ops (oracle/model.py
    population_loss takes lowrank, lowrank_embed and attention as arguments): with these, every linear call
    site of a population forward -- the value-embedding gate's lowrank on h[..., :32] included -- and every
    attention runs through libnoise_amd, while the elementwise steps stay torch's, as in the reference."""

    @staticmethod
    def lowrank(x, weight, a, b, sign):
        from noise_amd.eggroll import lowrank
        return lowrank(x, weight, a, b, sign)

    @staticmethod
    def lowrank_embed(weight, a, b, idx, sign):
        from noise_amd.eggroll import lowrank_embed
        return lowrank_embed(weight, a, b, idx, sign)

    @staticmethod
    def attention(q, k, v, window):
        return torch.ops.noise_amd.attention(q, k, v, window)


def composed_population_loss(model, p, noise, sign, idx, targets):
    """A population_loss of the reference's signature composed from the drop-ins (the oracle's composition run
    with DropIns as its ops, on the device tensors)."""
    return om.population_loss(p, noise, sign, idx, targets, ops=DropIns)


def member_noise(es, offsets, members, pairs):
    """Per-member noise, signs and directions for the member ids `members` of a population of `pairs` antithetic
    pairs: member g perturbs along direction (g mod 2 pairs) // 2, by +sigma when g is even and -sigma when it
    is odd (eggroll.py:134-142). The rows are gathered per member directly (a direction drawn once per member
    that uses it), so no pair expansion is needed."""
    from noise_amd.eggroll import SIGMA
    direction = (members % (2 * pairs)) // 2
    sign = torch.where(members % 2 == 0, SIGMA, -SIGMA).float()
    return es.noise(offsets, direction), sign, direction


def run_population(model, loss_fn, pairs, chunk, x, y, step=0):
    """One rank's whole population through `loss_fn(model, params, noise, sign, idx, targets)` under bf16 autocast,
    `2 * chunk` members per call; each call's members score the sequence of their first member (per_seq members
    per sequence, eggroll.py:143). Returns the member losses and, per call, (first member, noise, sign, sequence)."""
    from noise_amd.eggroll import Eggroll
    es = Eggroll(model, pairs)
    total = max(2 * pairs, 2 * len(x))
    per_seq = total // len(x)
    offsets = es.offsets(step)
    parts, calls = [], []
    for first in range(0, total, 2 * chunk):
        noise, sign, _ = member_noise(es, offsets, torch.arange(first, first + 2 * chunk, device=DEV), pairs)
        seq = first // per_seq
        with torch.autocast('cuda', dtype=torch.bfloat16):
            parts.append(loss_fn(model, es.params, noise, sign, x[seq], y[seq]))
        calls.append((first, noise, sign, seq))
    return torch.cat(parts), calls


def _tokens(batch, T, seed):
    g = torch.Generator().manual_seed(seed)
    rows = torch.randint(0, 4096, (batch, T + 1), generator=g)
    return rows[:, :-1].to(DEV), rows[:, 1:].to(DEV)


def _check_against_oracle(model, losses, calls, x, y, chunk):
    P = _cpu_params(model)
    worst = 0.0
    for start, noise, sign, seq in calls:
        ref = om.population_loss(P, _cpu_noise(noise), sign.cpu(), x[seq].cpu(), y[seq].cpu(), members_per_chunk=4)
        got = losses[start:start + 2 * chunk].cpu()
        assert torch.isfinite(got).all()
        worst = max(worst, (got - ref).abs().max().item())
    return worst


@pytest.mark.parametrize('composed', [False, True], ids=['fused-population_loss', 'composed-from-drop-ins'])
def test_reference_chunk_loop_under_compile(model, composed):
    from noise_amd.eggroll import population_loss
    pairs, chunk = 8, 4                      # two chunks of 8 members
    x, y = _tokens(2, 256, 5)                # two sequences: members 0-7 on one, 8-15 on the other
    if composed:
        fn = torch.compile(composed_population_loss, backend='aot_eager', fullgraph=True)
    else:
        fn = torch.compile(population_loss, fullgraph=True)
    print(f'chunk loop under torch.compile ({"composed" if composed else "fused"}): 16 members x 256 tokens, '
          f'all 60 parameters perturbed', flush=True)
    losses, calls = run_population(model, fn, pairs, chunk, x, y)
    worst = _check_against_oracle(model, losses, calls, x, y, chunk)
    print(f'worst |loss - oracle| = {worst:.3e}', flush=True)
    assert worst <= TOL
    # the perturbations must matter at this tolerance: a pair's losses differ
    assert (losses[1::2] - losses[0::2]).abs().max().item() > 0


def test_fused_and_composed_agree(model):
    """The fused population_loss and the drop-in composition of the reference's body give the same member
    losses (both compiled, same noise), within the bar."""
    from noise_amd.eggroll import population_loss
    x, y = _tokens(1, 256, 6)
    fused, _ = run_population(model, torch.compile(population_loss), 4, 4, x, y, step=1)
    comp, _ = run_population(model, torch.compile(composed_population_loss, backend='aot_eager'), 4, 4, x, y, step=1)
    assert (fused - comp).abs().max().item() <= TOL


def test_population_member_mapping_ranks_and_chunks(model):
    """Eggroll.population (eggroll.py:134-146): 24 pairs = 48 members over 8 sequences (6 each), two ranks
    of 24 members, chunks of 8 members (three per rank; a chunk's sequence is its first member's,
    start // per_seq, as the reference takes it). Every member of both ranks is checked against the oracle
    on noise gathered member by member from the mapping's closed form (member_noise)."""
    from noise_amd.eggroll import Eggroll
    pairs, batch, world, chunk = 24, 8, 2, 8
    x, y = _tokens(batch, 256, 7)
    step = 2
    members = max(2 * pairs, 2 * batch)
    per_seq, per_rank = members // batch, members // world
    P = _cpu_params(model)
    worst = 0.0
    for rank in range(world):
        es = Eggroll(model, pairs, rank=rank, world=world)
        print(f'population mapping: rank {rank} of {world}, members {rank * per_rank}..{(rank + 1) * per_rank - 1}',
              flush=True)
        got = es.population(step, x, y, chunk=chunk).cpu()
        assert got.shape == (per_rank,)
        offsets = es.offsets(step)
        for start in range(rank * per_rank, (rank + 1) * per_rank, chunk):
            noise, sign, _ = member_noise(es, offsets, torch.arange(start, start + chunk, device=DEV), pairs)
            seq = start // per_seq
            ref = om.population_loss(P, _cpu_noise(noise), sign.cpu(), x[seq].cpu(), y[seq].cpu(),
                                     members_per_chunk=4)
            part = got[start - rank * per_rank:start - rank * per_rank + chunk]
            worst = max(worst, (part - ref).abs().max().item())
    print(f'population mapping: worst |loss - oracle| = {worst:.3e}', flush=True)
    assert worst <= TOL


@pytest.mark.parametrize('shape', [(4, 256, 32, 8), (4, 100, 48, 40), (2, 256, 512, 2048)],
                         ids=['ve_gate', 'ragged', 'mfma'])
def test_lowrank_autocast_form(shape):
    """lowrank in autocast's form for any shape: y = bf16(x W^T) + sign bf16(x . b) a, with bf16 x, W and b.
    Both products are rounded once from an fp32 sum, so the result is the fp32 formula up to a last-bit
    disagreement of that rounding (sums differ in order): within one bf16 ulp of each product."""
    from noise_amd.eggroll import lowrank
    m, T, n_in, n_out = shape
    g = torch.Generator().manual_seed(sum(shape))
    h = torch.randn(m // 2, T, 512 if n_in == 32 else n_in, generator=g).repeat_interleave(2, 0)
    w = torch.randn(n_out, n_in, generator=g) * 0.3
    a, b = torch.randn(m // 2, n_out, generator=g), torch.randn(m // 2, n_in, generator=g)
    sign = torch.tensor([0.05, -0.05]).repeat(m // 2)[:m]
    hd = h.to(DEV)
    x = hd[..., :32] if n_in == 32 else hd       # the gate's strided slice h[..., :32] (eggroll.py:88)
    got = lowrank(x, w.to(DEV), a.to(DEV), b.to(DEV), sign.to(DEV), dir_div=2).cpu()
    xr = _bf(x.cpu())
    prod = xr @ _bf(w).t()
    dot = (xr * _bf(b).repeat_interleave(2, 0)[:m, None, :]).sum(-1, keepdim=True)
    ref = _bf(prod) + sign[:, None, None] * _bf(dot) * a.repeat_interleave(2, 0)[:m, None, :]
    ulp = prod.abs() * 2.0 ** -7 + (sign.abs()[:, None, None] * dot.abs() * 2.0 ** -7) * a.abs().max() + 1e-6
    assert got.shape == (m, T, n_out)
    assert ((got - ref).abs() <= ulp).all()


def test_lowrank_gate_call_site_compiled():
    """The gate call site itself, 2 sigmoid(lowrank(h[..., :32], W_gate, a, b, sign)) (eggroll.py:88), behind
    torch.compile with no graph break, equal to the eager call."""
    from noise_amd.eggroll import lowrank
    g = torch.Generator().manual_seed(21)
    h = torch.randn(4, 256, 512, generator=g).to(DEV)
    w = (torch.randn(8, 32, generator=g) * 0.3).to(DEV)
    a, b = torch.randn(4, 8, generator=g).to(DEV), torch.randn(4, 32, generator=g).to(DEV)
    sign = torch.tensor([0.01, -0.01, 0.01, -0.01], device=DEV)

    def gate(h, w, a, b, sign):
        return 2 * torch.sigmoid(lowrank(h[..., :32], w, a, b, sign))

    compiled = torch.compile(gate, fullgraph=True, backend='aot_eager')
    assert torch.equal(compiled(h, w, a, b, sign), gate(h, w, a, b, sign))


def test_block_forward_and_coordinate_differences_compiled():
    """run.py:89, :102 and :120 compile head_loss, block_forward and coordinate_differences: all three trace
    through the registered ops (fullgraph) and equal the eager drop-ins bit for bit."""
    from noise_amd.dust import block_forward, coordinate_differences, head_loss, head_loss_eager
    from noise_amd.model import make_model, rotary_tables
    P = {k: v.to(DEV) for k, v in make_model('cpu', 0).state_dict().items()}
    pre = 'transformer.h.1.'
    w = dict(q=P[pre + 'attn.c_q.weight'], k=P[pre + 'attn.c_k.weight'], v=P[pre + 'attn.c_v.weight'],
             gate=P[pre + 'attn.ve_gate.weight'], proj=P[pre + 'attn.c_proj.weight'], fc=P[pre + 'mlp.c_fc.weight'],
             out=P[pre + 'mlp.c_proj.weight'])
    g = torch.Generator().manual_seed(22)
    x = torch.randn(2, 256, 512, generator=g).to(DEV)
    ve = torch.randn(2, 256, 512, generator=g).to(DEV)
    jit = (torch.randn(2, 256, 2048, generator=g) * 0.01).to(DEV)
    cos, sin = (t[None, :, None, :].bfloat16().to(DEV) for t in rotary_tables(256))

    def blk(x, ve, jit):
        return block_forward(x, w, ve, cos, sin, 128, fc=jit)

    eager = blk(x, ve, jit)
    assert torch.equal(torch.compile(blk, fullgraph=True, backend='aot_eager')(x, ve, jit), eager)
    raw = (torch.randn(2, 256, 4096, generator=g) * 3).bfloat16().to(DEV)
    yy = torch.randint(-1, 4096, (2, 256), generator=g).to(DEV)
    cd = torch.compile(lambda r, t: coordinate_differences(r, t, 0.1), fullgraph=True, backend='aot_eager')
    assert torch.equal(cd(raw, yy), coordinate_differences(raw, yy, 0.1))
    # run.py:89 compiles head_loss too: the fp32 head traces through torch.ops.noise_amd.head_loss
    xs = torch.randn(2, 256, 512, generator=g).to(DEV)
    head = P['lm_head.weight'].float() * 30
    hl = torch.compile(lambda x_, w_, t_: head_loss(x_, w_, t_, 4096), fullgraph=True, backend='aot_eager')
    got = hl(xs, head, yy)
    assert got.shape == (2 * 256,) and torch.equal(got, head_loss_eager(xs, head, yy, 4096))


def test_out_of_range_token_ids_give_nan():
    """Ids outside [0, vocab) read nothing outside the tables and show up as NaN (the reference raises):
    in the embedding entry, the value-embedding rows, lowrank_embed and the head's targets. In-range
    members and tokens stay finite, and -1 targets are ignored (0)."""
    from noise_amd.eggroll import Weights, lowrank_embed, population_forward
    from noise_amd.model import make_model
    P = {k: v.float().to(DEV) for k, v in make_model('cpu', 0).state_dict().items()}
    W = Weights(P)
    g = torch.Generator().manual_seed(23)
    sign = torch.zeros(2, device=DEV)
    idx = torch.randint(0, 4096, (256,), generator=g).to(DEV)
    tgt = torch.randint(0, 4096, (256,), generator=g).to(DEV)
    ok = population_forward(W, {}, sign, idx, tgt, per_token=True).clone()
    assert torch.isfinite(ok).all()
    bad_idx = idx.clone()
    bad_idx[7] = 4096
    out = population_forward(W, {}, sign, bad_idx, tgt, per_token=True)
    assert torch.isnan(out[:, 7]).all()
    bad_t = tgt.clone()
    bad_t[3], bad_t[4], bad_t[5] = 4096, -1, -7
    out = population_forward(W, {}, sign, idx, bad_t, per_token=True)
    assert torch.isnan(out[:, 3]).all() and (out[:, 4] == 0).all() and torch.isnan(out[:, 5]).all()
    assert torch.isfinite(out[:, 6:]).all()
    e = lowrank_embed(P['transformer.wte.weight'], torch.zeros(2, 4096, device=DEV), torch.zeros(2, 512, device=DEV),
                      bad_idx, sign)
    assert torch.isnan(e[:, 7]).all() and torch.isfinite(e[:, 8:]).all()


def test_device_make_model_bf16_embeddings():
    """make_model('cuda', 0): the embeddings hold init_weights' bf16-rounded values (utils/model.py:171-175
    stores them in bf16 on a GPU; eggroll.py:50-52 casts back to fp32). The token embedding is the first
    draw of the device generator seeded 0, rounded; DUST's variant keeps the bf16 storage."""
    from noise_amd.model import make_model
    m = make_model('cuda', 0)
    for name, t in m.named_parameters():
        assert t.dtype == torch.float32, name
    for emb in [m.transformer.wte, *m.value_embeds.values()]:
        wt = emb.weight
        assert torch.equal(wt, wt.bfloat16().float())
    torch.manual_seed(0)
    first = torch.empty(4096, 512, device=DEV).normal_()
    assert torch.equal(m.transformer.wte.weight, first.bfloat16().float())
    d = make_model('cuda', 0, fp32_embeddings=False)
    assert d.transformer.wte.weight.dtype == torch.bfloat16
    assert d.lm_head.weight.dtype == torch.float32
    assert torch.equal(d.transformer.wte.weight.float(), m.transformer.wte.weight)
