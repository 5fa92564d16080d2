"""EGGROLL's update reassembly on the GPU (noise_update_weights / noise_update_gradients through the C ABI)
against the oracle (oracle/update.py) and against a float64 contraction over Eggroll.noise's device slices
(the update of eggroll.py:151-165: -(1/F) sum_d w_d a_d b_d^T per matrix, -(1/F) sum_d w_d eps_d per 1-D scalar).

Tolerance: the gradients are fp32 sums over the directions; the device forms the matrices' products as
split-bf16x3 MFMA GEMMs (each value hi + lo to 2^-16), so entries agree with the float64 oracle to 1e-4 of
the largest entry (the reference's own products are TF32 under set_float32_matmul_precision('high'),
about 2^-11 per factor)."""
import numpy as np
import pytest
import torch

from oracle import update as oupdate

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _rel(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _losses(members, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (8.3 + 0.01 * torch.randn(members, generator=g)).cuda()


class _Params(torch.nn.Module):
    """A handful of parameters of the model's shapes (both update paths, several chunks)."""

    def __init__(self):
        super().__init__()
        self.q = torch.nn.Parameter(torch.zeros(512, 512))
        self.fc = torch.nn.Parameter(torch.zeros(2048, 512))
        self.proj = torch.nn.Parameter(torch.zeros(512, 2048))
        self.gate = torch.nn.Parameter(torch.zeros(8, 32))
        self.lam = torch.nn.Parameter(torch.zeros(8))


def _direction_weights(losses, pairs):
    """Per-direction weights of the update, float64: member pair i holds losses (L[2i], L[2i+1]) and scores
    L[2i+1] - L[2i]; the scores are divided by their sample standard deviation (+1e-8) and summed per direction
    i mod pairs."""
    L = losses.double().cpu().numpy().reshape(-1, 2)
    score = L[:, 1] - L[:, 0]
    score = score / (score.std(ddof=1) + 1e-8)
    return score.reshape(-1, pairs).sum(0)


def _oracle(es, losses, offsets):
    d = es.buffer
    shapes = {n: tuple(p.shape) for n, p in es.params.items()}
    return oupdate.update_gradients(losses.cpu().numpy(), es.pairs, {n: o.cpu().numpy() for n, o in offsets.items()},
                                    shapes, (d.seed, d.offset, d.threads))


def test_weights_match_torch():
    from noise_amd import _lib
    for members, pairs in ((128, 64), (256, 64), (1024, 512)):
        losses = _losses(members, seed=members)
        w = torch.empty(pairs, device='cuda')
        _lib.call('noise_update_weights', _lib.ptr(losses), members, pairs, _lib.ptr(w), _lib.stream_ptr())
        ref = torch.from_numpy(_direction_weights(losses, pairs)).float().cuda()
        torch.cuda.synchronize()
        print(f'weights members {members} pairs {pairs}', flush=True)
        assert torch.allclose(w, ref, rtol=1e-5, atol=1e-6)


def test_full_model_matches_oracle():
    from noise_amd.eggroll import Eggroll
    from noise_amd.model import make_model
    model = make_model('cpu', 0).cuda()
    es = Eggroll(model, 64)
    offsets = es.offsets(3)
    losses = _losses(128)
    grads = es.update(losses, offsets)
    torch.cuda.synchronize()
    ref = _oracle(es, losses, offsets)
    assert set(grads) == set(ref) and len(grads) == 60
    worst = max((_rel(grads[n].cpu().numpy(), ref[n]), n) for n in grads)
    print('full model worst', worst, flush=True)
    assert worst[0] <= TOL


def test_chunks_accumulate_and_match_the_contraction():
    # pairs 600 in chunks of 256: three GEMM passes (the last partial), 1-D and small parameters alongside
    from noise_amd.eggroll import Eggroll
    es = Eggroll(_Params().cuda(), 600)
    offsets = es.offsets(11)
    losses = _losses(1200, seed=1)
    grads = es.update(losses, offsets, chunk=256)
    # the same gradients as one float64 contraction over all directions at once, on the device slices
    w = _direction_weights(losses, 600)
    n_pairs = losses.numel() // 2
    drawn = es.noise(offsets, torch.arange(600, device='cuda'))
    torch_grads = {}
    for name, n in drawn.items():
        if isinstance(n, tuple):
            A, B = (t.double().cpu().numpy() for t in n)
            torch_grads[name] = -((A * w[:, None]).T @ B) / n_pairs
        else:
            torch_grads[name] = -(w @ n.double().cpu().numpy()) / n_pairs
    ref = _oracle(es, losses, offsets)
    for name in es.params:
        got = grads[name].cpu().numpy()
        torch_ref = torch_grads[name]
        print(name, _rel(got, ref[name]), _rel(got, torch_ref), flush=True)
        assert got.shape == tuple(es.params[name].shape)
        assert _rel(got, ref[name]) <= TOL
        assert _rel(got, torch_ref) <= TOL


def test_update_is_deterministic_and_linear_in_fitness():
    from noise_amd.eggroll import Eggroll
    es = Eggroll(_Params().cuda(), 64)
    offsets = es.offsets(0)
    losses = _losses(128, seed=2)
    g1 = es.update(losses, offsets)
    g2 = es.update(losses, offsets)
    # shifting every loss leaves the antithetic differences (and so the update) unchanged: the losses lie in
    # [8, 16), where adding 0.5 is exact in fp32
    g3 = es.update(losses + 0.5, offsets)
    for n in g1:
        assert torch.equal(g1[n], g2[n])
        assert torch.equal(g3[n], g1[n])


def test_step_applies_the_update_with_the_optimizer():
    from noise_amd.eggroll import Eggroll
    from noise_amd.model import make_model
    model = make_model('cpu', 0).cuda()
    es = Eggroll(model, 8)
    g = torch.Generator().manual_seed(0)
    x = torch.randint(0, 4096, (1, 2048), generator=g).cuda()
    y = torch.randint(0, 4096, (1, 2048), generator=g).cuda()
    before = {n: p.detach().clone() for n, p in es.params.items()}
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    mean = es.step(x, y, opt, 0)
    after = {n: p.detach().clone() for n, p in es.params.items()}
    # replay from the old parameters: the same losses and offsets give the same gradients, and SGD moved
    # each parameter by -lr * grad
    for n, p in es.params.items():
        p.data.copy_(before[n])
    losses = es.population(0, x, y)
    assert abs(losses.mean().item() - mean) < 1e-6
    grads = es.update(losses, es.offsets(0))
    for n in es.params:
        assert not torch.equal(after[n], before[n]), n
        assert torch.allclose(after[n], before[n] - 0.1 * grads[n], rtol=0, atol=1e-6), n


@pytest.mark.parametrize('pairs', [600, 20])
def test_materialised_buffer_gives_the_same_gradients(pairs):
    # reading the materialised draw (noise_normal_fill) instead of regenerating it changes nothing: the
    # GEMM splits the same values into the same hi / lo halves, so it produces the same bits. 600 pairs: three
    # chunks of 256, the last 88 valid; 20 pairs: one chunk whose stages are padding past direction 20
    from noise_amd.eggroll import Eggroll
    es = Eggroll(_Params().cuda(), pairs)
    offsets = es.offsets(5)
    losses = _losses(2 * pairs, seed=3)
    g_regen = es.update(losses, offsets, chunk=256, materialise=False)
    g_buf = es.update(losses, offsets, chunk=256, materialise=True)
    for n in g_regen:
        print(n, float((g_regen[n] - g_buf[n]).abs().max()), flush=True)
        assert torch.equal(g_regen[n], g_buf[n]), n


def test_slices_leaving_the_draw_give_nan_rows_and_columns():
    # an element of a slice outside the draw reads as NaN: a slice starting before it makes the first rows of
    # that matrix's gradient NaN, one running past its end the last columns. The GEMM reading the materialised
    # draw and the regenerating path mark the same entries and agree bitwise on the others (the second slice
    # lies in the second chunk of directions; the third chunk is padded)
    from noise_amd.eggroll import Eggroll
    es = Eggroll(_Params().cuda(), 600, noise_numel=1 << 22)
    offsets = {n: o.clone() for n, o in es.offsets(9).items()}
    numel = es.noise_numel
    offsets['q'][0] = -100                   # a[0 .. 99] before the draw
    offsets['fc'][300] = numel - 2048 - 200  # a inside, b[200 ..] past the end
    losses = _losses(1200, seed=5)
    g_regen = es.update(losses, offsets, chunk=256, materialise=False)
    g_buf = es.update(losses, offsets, chunk=256, materialise=True)
    for n in g_regen:
        a, b = g_regen[n], g_buf[n]
        assert torch.equal(torch.isnan(a), torch.isnan(b)), n
        assert torch.equal(torch.nan_to_num(a, nan=0.0), torch.nan_to_num(b, nan=0.0)), n
    q, fc = g_buf['q'], g_buf['fc']
    assert torch.isnan(q[:100]).all() and torch.isfinite(q[100:]).all()
    assert torch.isnan(fc[:, 200:]).all() and torch.isfinite(fc[:, :200]).all()
    for n in ('proj', 'gate', 'lam'):
        assert torch.isfinite(g_buf[n]).all(), n


def test_workspace_without_partial_tiles_gives_the_same_gradients(monkeypatch):
    # a workspace that holds only the tables: the GEMM then runs whole tiles over every direction instead of
    # splitting the last round's tiles into partial tiles summed in order. The same products, summed in another
    # order: equal to fp32 rounding of the sums, and both within the oracle's bar
    from noise_amd import _lib
    from noise_amd.eggroll import Eggroll
    es = Eggroll(_Params().cuda(), 600)
    offsets = es.offsets(7)
    losses = _losses(1200, seed=4)
    lib = _lib.lib()
    full_bytes = lib.noise_update_workspace_bytes

    def tables_only(table, n, pairs, chunk):
        np_ = (min(chunk, pairs) + 255) // 256 * 256
        big = [table[i] for i in range(n) if table[i].cols > 0 and table[i].rows % 256 == 0 and table[i].cols % 256 == 0]
        need = sum((t.rows + t.cols) * 2 * np_ * 2 for t in big)
        assert full_bytes(table, n, pairs, chunk) > need  # the default leaves room for partial tiles
        return need

    split = es.update(losses, offsets, chunk=256)
    monkeypatch.setattr(lib, 'noise_update_workspace_bytes', tables_only)
    whole = es.update(losses, offsets, chunk=256)
    ref = _oracle(es, losses, offsets)
    for n in es.params:
        a, b = split[n].cpu().numpy(), whole[n].cpu().numpy()
        print(n, _rel(a, b), flush=True)
        assert _rel(a, b) <= 1e-6, n
        assert _rel(b, ref[n]) <= TOL, n
