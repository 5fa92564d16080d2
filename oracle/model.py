"""ORACLE (test infrastructure only): fp32 CPU restatement of the reference's population forward.

Follows, in plain fp32 torch CPU ops (no autocast, no flex_attention):
  utils/model.py:17-31   attention with the window mask q >= k & q - k <= window (dense masked softmax)
  utils/model.py:46-58   norm (rms_norm, eps = finfo(fp32).eps), has_ve, apply_rotary_emb
  utils/model.py:177-191 rotary tables (fp32 freqs -> cos/sin rounded to bf16), window sizes
  utils/model.py:193-209 GPT.forward (mix scalars, blocks, final norm, head, softcap 15, cross-entropy)
  utils/eval.py:43-46    the scorer's forward: GPT.forward run eagerly under bf16 autocast with the bf16
                         embeddings of model.py:170-174 (gpt_forward_eager: every op's result rounded)
  utils/model.py:81-120  CausalSelfAttention / MLP / Block forward
  train/val/eggroll.py:56-103 lowrank, lowrank_embed, population_loss
  train/val/run.py:89-94  head_loss (final norm, fp32 head, softcap, per-token CE)
  train/val/run.py:143-152 hadamard
Parameters are a dict name -> tensor using the reference's state-dict names.
"""
import math

import torch
import torch.nn.functional as F

N_LAYER, N_HEAD, HEAD_DIM, N_EMBD, VOCAB, SEQ = 8, 8, 64, 512, 4096, 2048
SOFTCAP = 15.0


def has_ve(i, n_layer=N_LAYER):
    return i % 2 == (n_layer - 1) % 2


def window_sizes(n_layer=N_LAYER, seq=SEQ, pattern='SSSL'):
    """model.py:185-191: S = seq // 2, L = seq, last block always L."""
    sizes = [seq if pattern[i % len(pattern)] == 'L' else seq // 2 for i in range(n_layer)]
    sizes[-1] = seq
    return sizes


def norm(x):
    return F.rms_norm(x, (x.size(-1),))


def rotary_tables(length, head_dim=HEAD_DIM, base=10000):
    """cos, sin [length, head_dim/2] as fp32 holding the bf16-rounded values of model.py:177-183."""
    inv_freq = 1.0 / base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)
    t = torch.arange(length, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().bfloat16().float(), freqs.sin().bfloat16().float()


def apply_rotary_emb(x, cos, sin):
    """x [B, T, H, D]; cos/sin [T, D/2]."""
    d = x.shape[3] // 2
    x1, x2 = x[..., :d], x[..., d:]
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    return torch.cat([x1 * c + x2 * s, x1 * -s + x2 * c], 3)


def attention(q, k, v, window, chunk=4):
    """softmax(q k^T / sqrt(D) masked) v for [B, T, H, D] inputs, in fp32, batches in chunks."""
    B, T, H, D = q.shape
    i = torch.arange(T)[:, None]
    j = torch.arange(T)[None, :]
    visible = (i >= j) & (i - j <= window)
    out = torch.empty(B, T, H, D, dtype=torch.float32)
    for b0 in range(0, B, chunk):
        qh = q[b0:b0 + chunk].float().transpose(1, 2)
        kh = k[b0:b0 + chunk].float().transpose(1, 2)
        vh = v[b0:b0 + chunk].float().transpose(1, 2)
        s = (qh @ kh.transpose(-1, -2)) / math.sqrt(D)
        s = s.masked_fill(~visible, float('-inf'))
        out[b0:b0 + chunk] = (torch.softmax(s, -1) @ vh).transpose(1, 2)
    return out


def softcap_ce(logits, targets, reduction='mean'):
    logits = SOFTCAP * torch.tanh(logits.float() / SOFTCAP)
    return F.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1), ignore_index=-1,
                           reduction=reduction)


def _block(P, i, x, ve, cos, sin, window):
    """Block.forward (model.py:116-120) with CausalSelfAttention (81-97) and MLP (105-107)."""
    B, T, C = x.shape
    pre = f'transformer.h.{i}.'
    h = norm(x)
    q = (h @ P[pre + 'attn.c_q.weight'].t()).view(B, T, N_HEAD, HEAD_DIM)
    k = (h @ P[pre + 'attn.c_k.weight'].t()).view(B, T, N_HEAD, HEAD_DIM)
    v = (h @ P[pre + 'attn.c_v.weight'].t()).view(B, T, N_HEAD, HEAD_DIM)
    if ve is not None:
        gate = 2 * torch.sigmoid(h[..., :32] @ P[pre + 'attn.ve_gate.weight'].t())
        v = v + gate.unsqueeze(-1) * ve.view(B, T, N_HEAD, HEAD_DIM)
    q, k = norm(apply_rotary_emb(q, cos, sin)), norm(apply_rotary_emb(k, cos, sin))
    y = attention(q, k, v, window).reshape(B, T, C)
    x = x + y @ P[pre + 'attn.c_proj.weight'].t()
    x = x + F.relu(norm(x) @ P[pre + 'mlp.c_fc.weight'].t()).square() @ P[pre + 'mlp.c_proj.weight'].t()
    return x


def gpt_forward(P, idx, targets=None, reduction='mean'):
    """GPT.forward (model.py:193-209) in fp32: logits, or the softcapped cross-entropy."""
    B, T = idx.shape
    cos, sin = rotary_tables(T)
    windows = window_sizes()
    x = x0 = norm(P['transformer.wte.weight'][idx].float())
    for i in range(N_LAYER):
        x = P['resid_lambdas'][i] * x + P['x0_lambdas'][i] * x0
        ve = P[f'value_embeds.{i}.weight'][idx].float() if has_ve(i) else None
        x = _block(P, i, x, ve, cos, sin, windows[i])
    x = norm(x)
    logits = (x @ P['lm_head.weight'].t())[..., :VOCAB].float()
    if targets is None:
        return SOFTCAP * torch.tanh(logits / SOFTCAP)
    return softcap_ce(logits, targets, reduction)


def bf16(t):
    """t rounded to the nearest bf16 (ties to even), as fp32."""
    return t.bfloat16().float()


def gpt_forward_eager(P, idx, targets=None, reduction='mean'):
    """The scorer's forward (eval.py:43-46 over model.py:193-209, 81-120): eager, under bf16 autocast, with
    the token and value embeddings stored in bf16. Every op's result is rounded to bf16 as eager autocast
    does: linear outputs (weights cast to bf16, fp32 sums), rms_norm of a bf16 input (fp32 inside), each
    product and sum of the mix (model.py:197, the fp32 lambdas entering as bf16), the rotary products and sums (model.py:55-58), the value
    gate's sigmoid and products (model.py:90-92), attention's output (fp32 inside), the residual adds
    (model.py:119-120) and ReLU's square (model.py:107). The logits leave the head as bf16 and are capped
    and scored in fp32 (model.py:203-209). Computation in fp32 with explicit rounding."""
    B, T = idx.shape
    cos, sin = rotary_tables(T)
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    windows = window_sizes()
    lin = lambda x, name: bf16(x @ bf16(P[name]).t())

    def rotary(u):
        u1, u2 = u[..., :HEAD_DIM // 2], u[..., HEAD_DIM // 2:]
        return torch.cat([bf16(bf16(u1 * c) + bf16(u2 * s)), bf16(bf16(u1 * -s) + bf16(u2 * c))], 3)

    x = x0 = bf16(norm(bf16(P['transformer.wte.weight'])[idx]))
    for i in range(N_LAYER):
        pre = f'transformer.h.{i}.'
        # a 0-dim fp32 tensor times a bf16 tensor computes in bf16: the scalar is rounded first
        rl, ml = bf16(P['resid_lambdas'][i]), bf16(P['x0_lambdas'][i])
        x = bf16(bf16(rl * x) + bf16(ml * x0))
        h = bf16(norm(x))
        q, k, v = (lin(h, pre + f'attn.c_{n}.weight').view(B, T, N_HEAD, HEAD_DIM) for n in 'qkv')
        if has_ve(i):
            ve = bf16(P[f'value_embeds.{i}.weight'])[idx].view(B, T, N_HEAD, HEAD_DIM)
            gate = bf16(2 * bf16(torch.sigmoid(lin(h[..., :32], pre + 'attn.ve_gate.weight'))))
            v = bf16(v + bf16(gate.unsqueeze(-1) * ve))
        q, k = bf16(norm(rotary(q))), bf16(norm(rotary(k)))
        y = bf16(attention(q, k, v, windows[i])).reshape(B, T, N_EMBD)
        x = bf16(x + lin(y, pre + 'attn.c_proj.weight'))
        hidden = lin(bf16(norm(x)), pre + 'mlp.c_fc.weight')
        x = bf16(x + lin(bf16(F.relu(hidden).square()), pre + 'mlp.c_proj.weight'))
    logits = lin(bf16(norm(x)), 'lm_head.weight')[..., :VOCAB]
    if targets is None:
        return SOFTCAP * torch.tanh(logits / SOFTCAP)
    return softcap_ce(logits, targets, reduction)


def lowrank(x, weight, a, b, sign):
    """eggroll.py:56-58 in fp32: x [m, T, in] through W [out, in] + sign * a b^T per member."""
    return x @ weight.t() + sign[:, None, None] * (x @ b.unsqueeze(-1)) * a[:, None, :]


def lowrank_embed(weight, a, b, idx, sign):
    """eggroll.py:61-63: embedding rows of W + sign * a b^T for token ids idx [T]."""
    return weight[idx].unsqueeze(0) + sign[:, None, None] * a[:, idx].unsqueeze(-1) * b[:, None, :]


class CpuOps:
    """The perturbed-linear, perturbed-embedding and attention ops population_loss composes; these are the
    oracle's own fp32 CPU forms. A caller may pass another set with the same signatures (the drop-ins), so the
    composition below doubles as a caller of the reference's shape: every weight matrix through lowrank, every
    table through lowrank_embed, attention on [B, T, H, D] views."""
    lowrank = staticmethod(lowrank)
    lowrank_embed = staticmethod(lowrank_embed)
    attention = staticmethod(attention)


def population_loss(P, noise, sign, idx, targets, members_per_chunk=None, ops=CpuOps):
    """eggroll.py:66-103 in fp32: mean CE [m] of m perturbed models on one sequence.

    noise: name -> (a [m, out], b [m, in]) for perturbed matrices/embeddings, or eps [m, L] for the mixing
    scalars; names absent from `noise` are unperturbed. members_per_chunk splits m to bound memory. ops: the
    lowrank / lowrank_embed / attention implementations (CpuOps: the oracle's)."""
    m = sign.shape[0]
    if members_per_chunk and m > members_per_chunk:
        parts = []
        for c in range(0, m, members_per_chunk):
            sl = slice(c, c + members_per_chunk)
            sub = {n: (tuple(t[sl] for t in v) if isinstance(v, tuple) else v[sl]) for n, v in noise.items()}
            parts.append(population_loss(P, sub, sign[sl], idx, targets, ops=ops))
        return torch.cat(parts)
    length = idx.shape[0]
    cos, sin = (t.to(idx.device) for t in rotary_tables(length))
    windows = window_sizes()
    s = sign[:, None, None]

    def lin(name, inp):
        if name in noise:
            return ops.lowrank(inp, P[name], *noise[name], sign)
        return inp @ P[name].t()

    def emb(name):
        if name in noise:
            return ops.lowrank_embed(P[name].float(), *noise[name], idx, sign)
        return P[name][idx].float().unsqueeze(0).expand(m, length, -1)

    def scalar(name, i):
        base = P[name][i]
        if name in noise:
            return base + s * noise[name][:, i, None, None]
        return base

    x = x0 = norm(emb('transformer.wte.weight'))
    for i in range(N_LAYER):
        pre = f'transformer.h.{i}.'
        x = scalar('resid_lambdas', i) * x + scalar('x0_lambdas', i) * x0
        h = norm(x)
        q = lin(pre + 'attn.c_q.weight', h).view(m, length, N_HEAD, HEAD_DIM)
        k = lin(pre + 'attn.c_k.weight', h).view(m, length, N_HEAD, HEAD_DIM)
        v = lin(pre + 'attn.c_v.weight', h).view(m, length, N_HEAD, HEAD_DIM)
        if has_ve(i):
            ve = emb(f'value_embeds.{i}.weight').reshape(m, length, N_HEAD, HEAD_DIM)
            gate = 2 * torch.sigmoid(lin(pre + 'attn.ve_gate.weight', h[..., :32]))
            v = v + gate.unsqueeze(-1) * ve
        q, k = norm(apply_rotary_emb(q, cos, sin)), norm(apply_rotary_emb(k, cos, sin))
        y = ops.attention(q, k, v, windows[i]).reshape(m, length, -1)
        x = x + lin(pre + 'attn.c_proj.weight', y)
        x = x + lin(pre + 'mlp.c_proj.weight', F.relu(lin(pre + 'mlp.c_fc.weight', norm(x))).square())
    h = norm(x)
    logits = lin('lm_head.weight', h)[..., :VOCAB]
    ce = softcap_ce(logits, targets.repeat(m), reduction='none')
    return ce.view(m, length).mean(-1)


def head_loss(x, weight, targets, vocab=VOCAB):
    """run.py:89-94 in fp32: final norm, head, softcap, per-token CE (ignore_index -1), reduction none."""
    logits = (norm(x.float()) @ weight.float().t())[..., :vocab]
    return softcap_ce(logits, targets, reduction='none')


def hadamard(d):
    """run.py:143-152: Sylvester Hadamard matrix of order d (power of two), entries +-1."""
    if d & (d - 1):
        raise ValueError(f'Orthogonal draws need a power-of-two width, not {d}.')
    H = torch.ones(1, 1)
    while H.shape[0] < d:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H
