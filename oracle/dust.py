"""ORACLE (test infrastructure only): DUST's head error, block_forward, capture cache, rerun and direct errors
on the CPU.

Restates train/val/run.py:121-137 (coordinate_differences) and run.py:380-389 (head_error) in float64
numpy: z = 15 tanh(raw / 15), the moved logits z' = cap(raw +- sigma), w = softmax(z), and
    change_j = log1p(w_j expm1(up_j - z_j)) - log1p(w_j expm1(down_j - z_j)) - [j = y] (up_j - down_j)
divided by 2 sigma, zero where y < 0. run.py:102-117 (block_forward), 247-254 (capture), 256-279 (rerun) in fp32
torch CPU ops; run.py:76-86 (chunk_size, reward_to_go) and 332-378 (direct_errors) in float64 numpy with the
reference's bf16 roundings (the reward and each chunk's estimate sum, the priors' predicted drop).
"""
import numpy as np


def softcap(v):
    return 15.0 * np.tanh(v / 15.0)


def coordinate_differences(raw, y, sigma):
    raw = np.asarray(raw, dtype=np.float64)
    y = np.asarray(y, dtype=np.int64)
    z, up, down = softcap(raw), softcap(raw + sigma), softcap(raw - sigma)
    e = np.exp(z - z.max(-1, keepdims=True))
    w = e / e.sum(-1, keepdims=True)
    change = np.log1p(w * np.expm1(up - z)) - np.log1p(w * np.expm1(down - z))
    t = np.clip(y, 0, None)[..., None]
    np.put_along_axis(change, t, np.take_along_axis(change, t, -1) - np.take_along_axis(up - down, t, -1), -1)
    return change / (2.0 * sigma) * (y >= 0)[..., None]


def head_error(logits, y, vocab, sigma=0.1):
    logits = np.asarray(logits, dtype=np.float64)
    out = np.zeros(logits.shape, dtype=np.float64)
    out[..., :vocab] = coordinate_differences(logits[..., :vocab], y, sigma)
    return out


def block_forward(x, w, ve, cos, sin, window, o=None, attn=None, fc=None, mlp=None, taps=None):
    """run.py:102-117 in the dtype of x (fp32 or fp64 torch, CPU): Block.forward with the jitter added at o
    (attention output), attn (c_proj product), fc (c_fc product, before ReLU^2) and mlp (mlp.c_proj product).
    w: q, k, v, gate (or None), proj, fc, out; cos, sin [T, 32]. taps: a dict that, when given, receives the
    three products 'attn' (attn.c_proj), 'fc' (mlp.c_fc) and 'mlp' (mlp.c_proj) as the module outputs a
    forward hook sees (run.py:196-200)."""
    import torch
    import torch.nn.functional as F
    from .model import norm, apply_rotary_emb, attention, N_HEAD, HEAD_DIM
    add = lambda t, j: t if j is None else t + j.to(t.dtype)
    B, T, C = x.shape
    dt = x.dtype
    W = {k: (None if v is None else v.to(dt)) for k, v in w.items()}
    h = norm(x)
    q, k, v = ((h @ W[n].t()).view(B, T, N_HEAD, HEAD_DIM) for n in ('q', 'k', 'v'))
    if ve is not None:
        gate = 2 * torch.sigmoid(h[..., :W['gate'].shape[1]] @ W['gate'].t())
        v = v + gate.unsqueeze(-1) * ve.to(dt).view(B, T, N_HEAD, HEAD_DIM)
    q, k = norm(apply_rotary_emb(q, cos.to(dt), sin.to(dt))), norm(apply_rotary_emb(k, cos.to(dt), sin.to(dt)))
    y = add(attention(q, k, v, window).to(dt).reshape(B, T, C), o)
    proj = y @ W['proj'].t()
    x = x + add(proj, attn)
    hidden = norm(x) @ W['fc'].t()
    out = F.relu(add(hidden, fc)).square() @ W['out'].t()
    if taps is not None:
        taps.update(attn=proj, fc=hidden, mlp=out)
    return x + add(out, mlp)


def draw_errors(errors, reward, a, sigma):
    """run.py:351-355: errors - einsum('nbt,nbtd->btd', bf16(reward), a) rounded to bf16, / sigma (float64
    sums; bf16 rounding of the reward and of the einsum's result as the reference's bf16 einsum)."""
    import torch
    bf = lambda v: torch.as_tensor(np.asarray(v, dtype=np.float32)).bfloat16().double().numpy()
    n = reward.shape[0]
    e = np.einsum('nbt,nbtd->btd', bf(reward), np.asarray(a, dtype=np.float64).reshape(n, *errors.shape))
    return np.asarray(errors, dtype=np.float64) - bf(e) / sigma


def capture(P, idx):
    """What DUST.capture (run.py:247-254) caches from the clean forward of GPT.forward (utils/model.py:193-209),
    in fp32 on the CPU: the embedding output, every block's input (after its mixing), x0 = norm(embedding), the
    value-embedding outputs and each block's attn.c_proj, mlp.c_fc and mlp.c_proj outputs (by module name, as
    the output hooks record them). idx [b, T]."""
    from .model import norm, has_ve, rotary_tables, window_sizes, N_LAYER
    T = idx.shape[1]
    cos, sin = rotary_tables(T)
    wins = window_sizes()   # the model's windows (sequence_len 2048), whatever T is
    emb = P['transformer.wte.weight'][idx].float()
    outputs = {'transformer.wte': emb}
    x = x0 = norm(emb)
    blocks = {}
    for i in range(N_LAYER):
        x = P['resid_lambdas'][i] * x + P['x0_lambdas'][i] * x0
        blocks[i] = x
        ve = P[f'value_embeds.{i}.weight'][idx].float() if has_ve(i) else None
        if ve is not None:
            outputs[f'value_embeds.{i}'] = ve
        taps = {}
        x = block_forward(x, block_weights(P, i), ve, cos, sin, wins[i], taps=taps)
        for key, site in SITES.items():
            if key in taps:
                outputs[site.format(i)] = taps[key]
    return dict(outputs=outputs, blocks=blocks, x0=x0)


def block_weights(P, i):
    """run.py:172-175's per-block dict of the fixed model's weights."""
    pre = f'transformer.h.{i}.'
    return dict(q=P[pre + 'attn.c_q.weight'], k=P[pre + 'attn.c_k.weight'], v=P[pre + 'attn.c_v.weight'],
                gate=P.get(pre + 'attn.ve_gate.weight'), proj=P[pre + 'attn.c_proj.weight'],
                fc=P[pre + 'mlp.c_fc.weight'], out=P[pre + 'mlp.c_proj.weight'])


SITES = {'o': 'o@{}', 'attn': 'transformer.h.{}.attn.c_proj', 'fc': 'transformer.h.{}.mlp.c_fc',
         'mlp': 'transformer.h.{}.mlp.c_proj'}


def rerun(P, cache, y, n, entry, jitter):
    """DUST.rerun (run.py:256-279) in fp32 on the CPU: per-token losses [n, b, T] of n jittered draws rerun
    from block `entry` (None: from the embedding) over the captured cache, jitter: site -> [n*b, T, width]."""
    from .model import norm, rotary_tables, window_sizes, head_loss, N_LAYER
    b, T = y.shape
    cos, sin = rotary_tables(T)
    wins = window_sizes()
    if entry is None:
        x = x0 = norm(cache['outputs']['transformer.wte'].repeat(n, 1, 1) + jitter['transformer.wte'].float())
    else:
        x, x0 = cache['blocks'][entry].repeat(n, 1, 1), cache['x0'].repeat(n, 1, 1)
    for i in range(entry or 0, N_LAYER):
        if entry is None or i > entry:
            x = P['resid_lambdas'][i] * x + P['x0_lambdas'][i] * x0
        ve = cache['outputs'].get(f'value_embeds.{i}')
        sites = {k: jitter.get(s.format(i)) for k, s in SITES.items()} if i == entry else {}
        sites = {k: (None if v is None else v.float()) for k, v in sites.items()}
        x = block_forward(x, block_weights(P, i), None if ve is None else ve.repeat(n, 1, 1), cos, sin, wins[i],
                          **sites)
    return head_loss(x, P['lm_head.weight'], y.repeat(n, 1)).view(n, b, T)


def chunk_size(draws, cap):
    """run.py:76-78: largest divisor of draws that does not exceed cap."""
    n = min(cap, draws)
    while draws % n:
        n -= 1
    return n


def reward_to_go(reward, gamma):
    """run.py:81-86 by its definition: out[..., i] = sum_{k < lags, i + k < t} gamma^k reward[..., i + k],
    lags = ceil(log(1e-6) / log(gamma)); float64."""
    r = np.asarray(reward, dtype=np.float64)
    lags = int(np.ceil(np.log(1e-6) / np.log(gamma)))
    t = r.shape[-1]
    out = np.zeros_like(r)
    for k in range(min(lags, t)):
        out[..., :t - k] += gamma ** k * r[..., k:]
    return out


def _bf16(v):
    import torch
    return torch.as_tensor(np.asarray(v, dtype=np.float32)).bfloat16().double().numpy()


def direct_errors(draw, rerun_fn, clean_loss, live, sites, widths, draws, sigma, nrep, gamma=0.0, priors=None):
    """DUST.direct_errors (run.py:332-378) in float64 with the reference's bf16 roundings.

    draw(site, draws, chunk, n, b, t, d) -> [n, b, t, d] of +-1 (OrthogonalDrawsOracle); rerun_fn(n, jitter) ->
    per-token losses [n, b, t] with jitter site -> bf16 torch tensor [n * b, t, d] holding bf16(sigma) * draw;
    clean_loss [b, t]; live: site -> 0/1 mask [b, t, d] (the mlp.c_fc sites); widths: site -> d; priors: site ->
    alpha * retrieval [b, t, d] or None.

    Per chunk of n = chunk_size(draws, nrep) draws: reward = clean_loss - loss, centred over the draws when n > 1,
    discounted when gamma > 0, plus sigma * sum_s bf16(a_s . bf16(prior_s)) (bf16 sums over sites; centred when
    n > 1), then each site's estimate -= bf16(sum_i bf16(reward_i) a_i) / sigma. Returns (estimates, record):
    estimates site -> error / draws + (1 - 1/n) prior, record per chunk the rewards, predicted drops and the
    chunk sums (for rounding bounds)."""
    import torch
    priors = {s: np.asarray(p, dtype=np.float64) * live.get(s, 1.0) for s, p in (priors or {}).items()}
    clean_loss = np.asarray(clean_loss, dtype=np.float64)
    b, t = clean_loss.shape
    n = chunk_size(draws, nrep)
    est = {s: np.zeros((b, t, widths[s])) for s in sites}
    record = []
    sig_bf = float(torch.tensor(sigma).bfloat16())   # the jitter sigma * a rounds sigma to bf16
    for chunk in range(draws // n):
        a = {s: np.asarray(draw(s, draws, chunk, n, b, t, widths[s]), dtype=np.float64) * live.get(s, 1.0)
             for s in sites}
        jitter = {s: torch.from_numpy((sig_bf * v).reshape(n * b, t, -1).astype(np.float32)).bfloat16()
                  for s, v in a.items()}
        loss = np.asarray(rerun_fn(n, jitter), dtype=np.float64)
        reward = clean_loss[None] - loss
        if n > 1:
            reward = reward - reward.mean(0, keepdims=True)
        if gamma:
            reward = reward_to_go(reward, gamma)
        predicted = None
        if priors:
            total = None
            for s, p in priors.items():
                dot = _bf16(np.einsum('nbtd,btd->nbt', a[s], _bf16(p)))
                total = dot if total is None else _bf16(total + dot)
            predicted = sigma * total
            reward = reward + (predicted - predicted.mean(0, keepdims=True) if n > 1 else predicted)
        sums = {}
        for s in sites:
            sums[s] = _bf16(np.einsum('nbt,nbtd->btd', _bf16(reward), a[s]))
            est[s] = est[s] - sums[s] / sigma
        record.append(dict(loss=loss, reward=reward, predicted=predicted, sums=sums, a=a))
    kept = 1 - 1 / n if n > 1 else 1.0
    return {s: e / draws + kept * priors.get(s, 0.0) for s, e in est.items()}, record


def block_forward_bf16_flow(x, w, ve, cos, sin, window, o=None, attn=None, fc=None, mlp=None):
    """run.py:102-117 with the dtype flow the reference's compiled block_forward has on a GPU under bf16 autocast,
    for bf16-valued x: fp32 inside every fused elementwise chain, bf16 at every linear output (weights rounded to
    bf16) and at every tensor the graph stores (norm outputs, q and k after rotary and norm, v with its gated
    value embedding, the attention output, x_mid, ReLU^2, the block output). fp32 CPU tensors holding bf16 values."""
    import torch
    import torch.nn.functional as F
    from .model import norm, apply_rotary_emb, attention, bf16, N_HEAD, HEAD_DIM
    add = lambda t, j: t if j is None else t + j.float()
    B, T, C = x.shape
    W = {k: (None if v is None else bf16(v.float())) for k, v in w.items()}
    lin = lambda u, name: bf16(u @ W[name].t())
    h = bf16(norm(x))
    q, k, v = (lin(h, n).view(B, T, N_HEAD, HEAD_DIM) for n in ('q', 'k', 'v'))
    if ve is not None:
        gate = 2 * torch.sigmoid(lin(h[..., :W['gate'].shape[1]], 'gate'))
        v = bf16(v + gate.unsqueeze(-1) * ve.float().view(B, T, N_HEAD, HEAD_DIM))
    q, k = bf16(norm(apply_rotary_emb(q, cos, sin))), bf16(norm(apply_rotary_emb(k, cos, sin)))
    y = bf16(add(bf16(attention(q, k, v, window)).reshape(B, T, C), o))
    x = bf16(x + add(lin(y, 'proj'), attn))
    act = bf16(F.relu(add(lin(bf16(norm(x)), 'fc'), fc)).square())
    return bf16(x + add(lin(act, 'out'), mlp))


def rerun_bf16_flow(P, cache, y, n, entry, jitter):
    """DUST.rerun (run.py:256-279) with the dtype flow it has on a GPU: the model's embeddings stored in bf16
    (utils/model.py:171-175), so the captured embedding, block inputs, x0 and value-embedding outputs are bf16;
    the mixing between blocks in bf16 (a 0-dim fp32 lambda times a bf16 tensor rounds the lambda and each
    product, then the sum); block_forward_bf16_flow; the final norm, head and loss in fp32. cache: capture() of
    the model with bf16-rounded embedding tables. Per-token losses [n, b, T]."""
    from .model import norm, bf16, rotary_tables, window_sizes, head_loss, N_LAYER
    b, T = y.shape
    cos, sin = rotary_tables(T)
    wins = window_sizes()
    mix = lambda i, u, u0: bf16(bf16(bf16(P['resid_lambdas'][i]) * u) + bf16(bf16(P['x0_lambdas'][i]) * u0))
    if entry is None:
        x = x0 = bf16(norm(bf16(bf16(cache['outputs']['transformer.wte']).repeat(n, 1, 1)
                                + jitter['transformer.wte'].float())))
    else:
        x, x0 = bf16(cache['blocks'][entry]).repeat(n, 1, 1), bf16(cache['x0']).repeat(n, 1, 1)
    for i in range(entry or 0, N_LAYER):
        if entry is None or i > entry:
            x = mix(i, x, x0)
        ve = cache['outputs'].get(f'value_embeds.{i}')
        sites = {k: jitter.get(s.format(i)) for k, s in SITES.items()} if i == entry else {}
        x = block_forward_bf16_flow(x, block_weights(P, i), None if ve is None else bf16(ve).repeat(n, 1, 1), cos,
                                    sin, wins[i], **sites)
    return head_loss(x, P['lm_head.weight'], y.repeat(n, 1)).view(n, b, T)
