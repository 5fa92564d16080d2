"""The scorer (utils/eval.py:34-53) on the GPU: one validation row per member, no noise, the eager bf16
autocast forward (ROUNDING_EAGER), summed per-token CE over float64.

Bar: each row's mean CE within 1e-3 absolute of the oracle's eager forward (oracle/model.py
gpt_forward_eager, pinned bit-exactly on the CPU against torch's bf16 dtype flow), and the score within
1e-3 of torch's own eager autocast forward run on the GPU. The head is scaled x30 so the loss depends on
the hidden state (at the seed-0 init every loss sits at ln 4096). The eager and fp32-stream forwards
differ by ~3e-4 in row means, inside the bar, so the rounding mode itself is checked where its effect is
deterministic (block 0's entry, bf16 values in the residual stream).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import model as om

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)
TOL = 1e-3


@pytest.fixture(scope='module')
def params():
    from noise_amd.model import make_model
    P = {k: v.float() for k, v in make_model('cpu', 0).state_dict().items()}
    P['lm_head.weight'] = P['lm_head.weight'] * 30
    return P


def _rows(n, T, seed):
    return torch.randint(0, 4096, (n, T + 1), generator=torch.Generator().manual_seed(seed))


def _attention_fp32(q, k, v, window):
    """model.py:17-31 in fp32 on the device: [B, T, H, D], scale 1/sqrt(D), mask q >= k and q - k <= window."""
    T, D = q.shape[1], q.shape[3]
    i = torch.arange(T, device=q.device)
    mask = (i[:, None] >= i[None, :]) & (i[:, None] - i[None, :] <= window)
    q, k, v = (t.transpose(1, 2) for t in (q, k, v))
    s = (q @ k.transpose(-1, -2).contiguous()) / math.sqrt(D)
    p = s.masked_fill(~mask, float('-inf')).softmax(-1)
    return (p @ v).transpose(1, 2)


def _autocast_forward(P, idx, targets):
    """model.py:193-209 under torch.autocast('cuda', bf16) with the bf16 embeddings of model.py:170-174,
    as eval.py:43-46 runs it. Attention is computed in fp32 from the bf16 q, k, v and returned in bf16
    (flex attention's output dtype), avoiding bf16 batched products."""
    B, T = idx.shape
    cos, sin = (t.to(DEV, torch.bfloat16)[None, :, None, :] for t in om.rotary_tables(T))
    W = {k: v.to(DEV) for k, v in P.items()}
    for k in W:
        if k == 'transformer.wte.weight' or k.startswith('value_embeds.'):
            W[k] = W[k].to(torch.bfloat16)
    norm = lambda x: F.rms_norm(x, (x.size(-1),))

    def rot(u):
        u1, u2 = u[..., :32], u[..., 32:]
        return torch.cat([u1 * cos + u2 * sin, u1 * -sin + u2 * cos], 3)

    with torch.autocast('cuda', dtype=torch.bfloat16):
        x = x0 = norm(F.embedding(idx, W['transformer.wte.weight']))
        for i in range(8):
            pre = f'transformer.h.{i}.'
            x = W['resid_lambdas'][i] * x + W['x0_lambdas'][i] * x0
            h = norm(x)
            q, k, v = (F.linear(h, W[pre + f'attn.c_{n}.weight']).view(B, T, 8, 64) for n in 'qkv')
            if om.has_ve(i):
                ve = F.embedding(idx, W[f'value_embeds.{i}.weight']).view(B, T, 8, 64)
                gate = 2 * torch.sigmoid(F.linear(h[..., :32], W[pre + 'attn.ve_gate.weight']))
                v = v + gate.unsqueeze(-1) * ve
            q, k = norm(rot(q)), norm(rot(k))
            with torch.autocast('cuda', enabled=False):
                y = _attention_fp32(q.float(), k.float(), v.float(), om.window_sizes()[i]).to(torch.bfloat16)
            x = x + F.linear(y.reshape(B, T, 512), W[pre + 'attn.c_proj.weight'])
            x = x + F.linear(F.relu(F.linear(norm(x), W[pre + 'mlp.c_fc.weight'])).square(),
                             W[pre + 'mlp.c_proj.weight'])
        logits = F.linear(norm(x), W['lm_head.weight'])[..., :4096].float()
        logits = 15 * torch.tanh(logits / 15)
        return F.cross_entropy(logits.view(-1, 4096), targets.reshape(-1), ignore_index=-1, reduction='sum')


def test_eager_rows_match_oracle(params):
    from noise_amd import _lib
    from noise_amd.eggroll import Weights, _Buffers, population_forward
    from noise_amd.eval import load_model
    rows = _rows(3, 512, 11)
    idx, tgt = rows[:, :-1], rows[:, 1:].clone()
    tgt[1, 100:140] = -1  # ignored targets contribute 0
    print('eval: 3 rows x 512 tokens, eager rounding', flush=True)
    W = load_model(params, DEV)
    B = _Buffers(3, 512, DEV, False, True, eager=True)
    got = population_forward(W, {}, torch.zeros(3, device=DEV), idx.to(DEV), tgt.to(DEV), buffers=B,
                             per_token=True, rounding=_lib.ROUNDING_EAGER).cpu()
    want = om.gpt_forward_eager(params, idx, tgt, 'none').view(3, 512)
    assert torch.all(got[tgt < 0] == 0)
    err = (got.mean(1) - want.mean(1)).abs().max().item()
    assert err < TOL, err
    # The roundings themselves. A bf16 stream is chaotic at the one-ulp level (a single flipped rounding
    # in an early block moves a token's loss by ~1e-2 eight blocks later), so the end-to-end losses of the
    # two rounding modes are equally close to either oracle per token; the mode is checked where its
    # effect is deterministic. Block 0's entry: x0 = bf16(norm(bf16 wte[idx])) and the mix
    # bf16(bf16(rl x0) + bf16(ml x0)) with bf16 lambdas, equal to the oracle's but for rare one-ulp
    # differences of rsqrt; and the residual stream out of the last block holds bf16 values.
    bf = lambda t: t.bfloat16().float()
    x0 = bf(om.norm(bf(params['transformer.wte.weight'])[idx]))
    rl, ml = bf(params['resid_lambdas'][0]), bf(params['x0_lambdas'][0])
    xin = bf(bf(rl * x0) + bf(ml * x0))
    for name, dev_t, ref in (('x0', B.x0, x0), ('x after the mix', B.xin0, xin)):
        d = dev_t.cpu().view_as(ref)
        assert torch.equal(d, bf(d)), name
        ulp = (ref.abs() * 2.0 ** -7).clamp_min(1e-30)
        assert ((d - ref).abs() <= ulp).all(), name
        assert (d != ref).float().mean().item() < 1e-3, name
    resid = B.resid.cpu()
    assert torch.equal(resid, bf(resid))
    # the fused (fp32-stream) forward keeps those values in fp32, and matches the fp32 oracle
    B2 = _Buffers(3, 512, DEV, False, True)
    fused = population_forward(Weights({k: v.to(DEV) for k, v in params.items()}), {}, torch.zeros(3, device=DEV),
                               idx.to(DEV), tgt.to(DEV), buffers=B2, per_token=True).cpu()
    fp32 = om.gpt_forward(params, idx, tgt, 'none').view(3, 512)
    assert (fused.mean(1) - fp32.mean(1)).abs().max().item() < TOL
    assert not torch.equal(B2.resid.cpu(), bf(B2.resid.cpu()))


def test_score_matches_torch_autocast_forward(params):
    from noise_amd.eval import load_model, score_rows
    rows = _rows(5, 1024, 12)
    print('eval: 5 rows x 1024 tokens, batches of 2', flush=True)
    W = load_model(params, DEV)
    total, count = score_rows(W, rows, batch_size=2)
    assert count == 5 * 1024
    want = _autocast_forward(params, rows[:, :-1].to(DEV), rows[:, 1:].to(DEV)).double().item()
    assert abs(total.item() / count - want / count) < TOL, (total.item() / count, want / count)
    # deterministic: the same rows in another batching give the same per-row losses summed in float64
    again, _ = score_rows(W, rows, batch_size=5)
    assert abs(again.item() - total.item()) < 1e-9 * abs(total.item()) + 1e-6


def test_evaluate_end_to_end(params, tmp_path, monkeypatch):
    from noise_amd import prepare_data as pd
    from noise_amd.eval import evaluate, load_model, score_rows
    rows = torch.randint(0, 4096, (pd.VAL_ROWS, pd.SEQ), generator=torch.Generator().manual_seed(13),
                         dtype=torch.int32)
    monkeypatch.setitem(pd.EXPECTED, 'val.pt', pd.token_hash(rows))
    torch.save(rows, tmp_path / 'val.pt')
    print('eval: evaluate() over 544 synthetic rows x 2048 tokens', flush=True)
    value = evaluate(params, tmp_path, batch_size=16)
    assert math.isfinite(value) and 7.0 < value < 9.5
    # the same rows scored through score_rows in a few slices agree with the whole (float64 sums)
    W = load_model(params, DEV)
    part = sum(score_rows(W, rows[s].long(), 16)[0].item()
               for s in (slice(0, 100), slice(100, 544)))
    assert abs(part / (pd.VAL_ROWS * 2048) - value) < 1e-9
    with pytest.raises(RuntimeError, match='missing keys'):
        evaluate({k: v for k, v in params.items() if k != 'lm_head.weight'}, tmp_path)
