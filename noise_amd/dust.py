"""DUST pieces on the population-forward path (train/val/run.py):

  head_loss(x, weight, targets, vocab)      run.py:89-94, the fp32 head of rerun (run.py:273-278)
  block_forward(x, w, ve, cos, sin, window, o, attn, fc, mlp)   run.py:102-117
  rerun(dust, n, entry, jitter)             run.py:256-279 (DUST.rerun)
  draw_errors(errors, reward, a, sigma)     run.py:351-355 (direct_errors' estimate update)
  direct_errors(dust, sites, draws, sigma, entry, gamma, retrieved)   run.py:332-378 (DUST.direct_errors)
  chunk_size(draws, cap), reward_to_go(reward, gamma)                 run.py:76-86
  coordinate_differences(raw, y, sigma)     run.py:121-137
  head_error(logits, y, vocab, sigma)       run.py:380-389
  hadamard(d, device, dtype)                run.py:143-152
  OrthogonalDraws                           run.py:218-238 (signs, orthogonal_noise)
"""
import ctypes
import math

import torch
import torch.nn.functional as F

from . import _lib
from .noise import DeviceGenerator

F32, BF16 = torch.float32, torch.bfloat16


def head_loss(x, weight, targets, vocab):
    """run.py:89-94 `head_loss(x, weight, targets, vocab)` through the registered op torch.ops.noise_amd.head_loss
    (the reference compiles it, run.py:89): per-token soft-capped cross-entropy of the fp32 head, [numel(targets)]."""
    return torch.ops.noise_amd.head_loss(x, weight, targets, int(vocab))


def head_loss_eager(x, weight, targets, vocab):
    """Final norm, fp32 head, soft cap and per-token cross-entropy (ignore_index -1), reduction none.

    x [..., T, 512] fp32, weight [V, 512], targets [..., T] -> [numel(targets)]. The reference runs the
    fp32 GEMM as TF32 on H100 (run.py:676); here it is split-bf16x3 on MFMA (x = hi + lo, w = hi + lo,
    logits = hi.hi + hi.lo + lo.hi), which is more accurate than TF32."""
    dev = x.device
    d = x.shape[-1]
    if d != 512 or weight.shape[1] != 512 or vocab % 256 or weight.shape[0] < vocab:
        raise ValueError('head_loss: width 512 and vocab a multiple of 256 are supported')
    rows = x.numel() // d
    pad = -rows % 256
    xs = x.reshape(rows, d).to(F32)
    if pad:
        xs = torch.cat([xs, torch.zeros(pad, d, dtype=F32, device=dev)])
    xs = xs.contiguous()
    tg = targets.reshape(rows).to(device=dev, dtype=torch.int64)
    if pad:
        tg = torch.cat([tg, torch.full((pad,), -1, dtype=torch.int64, device=dev)])
    tg = tg.contiguous()
    stream = _lib.stream_ptr(dev)
    n = rows + pad
    x3 = torch.empty(n, 3 * d, dtype=BF16, device=dev)
    _lib.call('noise_split3', xs.data_ptr(), n, d, 1, 0, x3.data_ptr(), stream)
    w = weight[:vocab].to(device=dev, dtype=F32).contiguous()
    w3 = torch.empty(vocab, 3 * d, dtype=BF16, device=dev)
    _lib.call('noise_split3', w.data_ptr(), vocab, d, 0, 1, w3.data_ptr(), stream)
    loss = torch.empty(n, dtype=F32, device=dev)
    pop = _lib.Population(1, n, None, 1)
    none = _lib.Rank1(None, None, 0, 0)
    _lib.call('noise_pop_head_ce', ctypes.byref(pop), _lib.View(x3.data_ptr(), 0, 3 * d), w3.data_ptr(), 3 * d, vocab,
              ctypes.byref(none), None, tg.data_ptr(), 0, loss.data_ptr(), stream)
    return loss[:rows]


def coordinate_differences(raw, y, sigma):
    """run.py:121-137: per token and logit, (loss(raw_j + sigma) - loss(raw_j - sigma)) / (2 sigma) of the
    soft-capped cross-entropy, in closed form; zero at ignored tokens (y < 0). raw [..., V] bf16 or fp32
    (unit inner stride), y [...] int64 -> fp32 [..., V]. Runs as torch.ops.noise_amd.coordinate_differences,
    so the reference's @torch.compile caller (run.py:120) traces it."""
    return torch.ops.noise_amd.coordinate_differences(raw, y, float(sigma))


def head_error(logits, y, vocab, sigma=0.1):
    """DUST.head_error (run.py:380-389): coordinate differences of the first `vocab` logits, the padding
    columns zero. logits [..., Vpad] bf16 or fp32 (unit inner stride), y [...] -> fp32 [..., Vpad]."""
    if logits.dtype not in (F32, BF16) or logits.stride(-1) != 1:
        raise ValueError('logits must be bf16 or fp32 with unit inner stride')
    width = logits.shape[-1]
    raw = logits.reshape(-1, width)
    if raw.data_ptr() != logits.data_ptr():
        raw = raw.contiguous()
    rows = raw.shape[0]
    tg = y.reshape(rows).to(device=logits.device, dtype=torch.int64).contiguous()
    out = torch.empty(*logits.shape[:-1], width, dtype=F32, device=logits.device)
    _lib.call('noise_coordinate_differences', raw.data_ptr(), 1 if raw.dtype == BF16 else 0, rows, vocab,
              raw.stride(0), tg.data_ptr(), float(sigma), out.data_ptr(), width, width,
              _lib.stream_ptr(logits.device))
    return out


def _bf16_weight(t):
    """bf16 contiguous copy of a weight (the reference's autocast casts it at every call too)."""
    return t.detach().to(BF16).contiguous()


def block_forward(x, w, ve, cos, sin, window, o=None, attn=None, fc=None, mlp=None):
    """run.py:102-117 `block_forward(x, w, ve, cos, sin, window, o, attn, fc, mlp)` through the registered op
    torch.ops.noise_amd.block_forward (the reference compiles it, run.py:102): w is the reference's dict
    q, k, v, gate, proj, fc, out."""
    ws = [w.get(k) if k == 'gate' else w[k] for k in ('q', 'k', 'v', 'gate', 'proj', 'fc', 'out')]
    return torch.ops.noise_amd.block_forward(x, ws, ve, cos, sin, int(window), o, attn, fc, mlp)


def block_forward_eager(x, w, ve, cos, sin, window, o=None, attn=None, fc=None, mlp=None):
    """run.py:102-117: Block.forward on x [B, T, 512] with optional jitter at o (attention output), attn
    (attn.c_proj product), fc (mlp.c_fc product, before ReLU^2) or mlp (mlp.c_proj product), each
    [B, T, width]. w: the reference's dict q, k, v, gate (None without value embeddings), proj, fc, out.
    ve: [B, T, 512] value-embedding rows or None. cos, sin: the model's rotary tables (bf16, T x 32 values).
    Returns x_out fp32 [B, T, 512]. One HIP chain (noise_dust_block): bf16 products with fp32 accumulation,
    bf16 attention, fp32 residual stream, as the reference's autocast."""
    dev = x.device
    B, T, C = x.shape
    if C != 512 or T % 256:
        raise ValueError('block_forward: width 512 and a multiple of 256 tokens are supported')
    xs = x.to(F32).contiguous()
    out = torch.empty(B, T, C, dtype=F32, device=dev)
    gate = w.get('gate')
    ws = [_bf16_weight(w['q']), _bf16_weight(w['k']), _bf16_weight(w['v']),
          None if gate is None else _bf16_weight(gate).to(F32).contiguous(),  # autocast rounds it to bf16 too
          _bf16_weight(w['proj']), _bf16_weight(w['fc']), _bf16_weight(w['out'])]
    wp = (ctypes.c_void_p * 7)(*[None if t is None else t.data_ptr() for t in ws])
    if ve is not None:
        if gate is None:
            raise ValueError('block_forward: value embeddings need the ve_gate weight')
        ve = ve.reshape(B, T, C).to(BF16).contiguous()
    cs = cos.reshape(-1)[:T * 32].view(T, 32).to(BF16).contiguous()
    sn = sin.reshape(-1)[:T * 32].view(T, 32).to(BF16).contiguous()
    jit = []
    for t, width in ((o, C), (attn, C), (fc, 4 * C), (mlp, C)):
        jit.append(None if t is None else t.reshape(B, T, width).to(BF16).contiguous())
    need = _lib.lib().noise_dust_block_workspace_bytes(B, T, 1 if ve is not None else 0)
    work = torch.empty(need, dtype=torch.uint8, device=dev)
    _lib.call('noise_dust_block', xs.data_ptr(), out.data_ptr(), B, T, wp, _lib.ptr(ve), cs.data_ptr(), sn.data_ptr(),
              int(window), *[_lib.ptr(t) for t in jit], work.data_ptr(), need, _lib.stream_ptr(dev))
    return out


def draw_errors(errors, reward, a, sigma):
    """run.py:351-355 in place: errors -= einsum('nbt,nbtd->btd', reward.to(bf16), a).float() / sigma.
    errors fp32 [b, t, d] (contiguous), reward [n, b, t], a bf16 [n * b, t, d] or [n, b, t, d]."""
    n = reward.shape[0]
    rows = errors.numel() // errors.shape[-1]
    d = errors.shape[-1]
    if errors.dtype != F32 or not errors.is_contiguous():
        raise ValueError('errors must be a contiguous fp32 tensor')
    r = reward.to(device=errors.device, dtype=F32).reshape(n, rows).contiguous()
    av = a.to(BF16).reshape(n, rows, d).contiguous()
    _lib.call('noise_draw_errors', r.data_ptr(), av.data_ptr(), n, rows, d, -1.0 / float(sigma), errors.data_ptr(),
              _lib.stream_ptr(errors.device))
    return errors


# jitter sites of a block (run.py:97-98): block_forward keyword -> the reference's site name
SITES = {'o': 'o@{}', 'attn': 'transformer.h.{}.attn.c_proj', 'fc': 'transformer.h.{}.mlp.c_fc',
         'mlp': 'transformer.h.{}.mlp.c_proj'}


def _rotary(model, T, dev):
    """The model's bf16 rotary tables for T tokens (utils/model.py:144-147 buffers when the model has them, else the
    device tables built once per length: a copy from host memory per call would wait for the stream)."""
    if hasattr(model, 'cos'):
        return model.cos[:, :T], model.sin[:, :T]
    from .eggroll import _rope_tables
    return _rope_tables(T, dev)


def _weights(dust):
    """The population kernels' weights of dust.model (bf16 matrices in the block kernel's layouts, the fp32 head
    as split-bf16x3), built on first use and rebuilt when a parameter has changed since (an in-place optimizer
    step bumps the tensor's version)."""
    from .eggroll import Weights
    params = dict(dust.model.named_parameters())
    # keyed on the parameter objects themselves (identity) and their versions: a tensor allocated later at a
    # freed parameter's address cannot pass for it
    key = tuple((name, p._version) for name, p in params.items())
    cached = getattr(dust, '_noise_amd_weights', None)
    if (cached is None or cached[0] != key or len(cached[1]) != len(params)
            or not all(a is b for a, b in zip(cached[1], params.values()))):
        dev = dust.y.device
        W = Weights({name: p.detach() for name, p in params.items()}, device=dev, n_layer=dust.model.config.n_layer,
                    fp32_head=True)
        dust._noise_amd_weights = cached = (key, list(params.values()), W)
    return cached[2]


def _batch_rows(dust, n, with_x0):
    """The batch's tensors that rerun reads for n draws: token ids and targets repeated n times (int64
    [n * batch, length]), the bf16 rotary tables [length, 32], and (with_x0) the normed embedding x0 repeated
    n times (fp32 [n * batch, length, 512]: the blocks' mixing reads x0 per member). Built on first use for this
    capture and n, and rebuilt when dust.x, dust.y or dust.x0 is another tensor or was changed in place: the
    reference's direct_errors reruns one capture over many sites and chunks of draws."""
    T = dust.length
    dev = dust.y.device
    # the cache holds the source tensors themselves: compared by identity and version, a tensor allocated later
    # at a freed one's address cannot pass for it
    src = (dust.x, dust.y, dust.x0 if with_x0 else None)
    versions = tuple(t._version if t is not None else None for t in src)
    cached = getattr(dust, '_noise_amd_rows', None)
    if (cached is not None and cached[0] == (n, T, with_x0, versions)
            and all(a is b for a, b in zip(cached[1], src))):
        return cached[2]
    cos, sin = _rotary(dust.model, T, dev)
    rows = dict(
        idx=dust.x.to(device=dev, dtype=torch.int64).repeat(n, 1).contiguous(),
        targets=dust.y.to(device=dev, dtype=torch.int64).repeat(n, 1).contiguous(),
        rope=(cos.reshape(-1)[:T * 32].view(T, 32).to(BF16).contiguous(),
              sin.reshape(-1)[:T * 32].view(T, 32).to(BF16).contiguous()),
        x0=dust.x0.detach().to(F32).repeat(n, 1, 1).contiguous() if with_x0 else None)
    dust._noise_amd_rows = ((n, T, with_x0, versions), src, rows)
    return rows


def rerun(dust, n, entry, jitter):
    """DUST.rerun (run.py:256-279) with the same arguments and state: the per-token losses [n, batch, length]
    of n jittered draws, rerun from block `entry` (None: from the embedding).

    `dust` carries what the reference's DUST object holds after capture: model (resid_lambdas, x0_lambdas,
    window_sizes, lm_head, config, parameters), length, batch, outputs ('transformer.wte' and 'value_embeds.{i}'
    outputs), blocks (block inputs by layer), x0 (the normed embedding), x and y (the batch's token ids and
    targets, [batch, length]) and weights (the per-block dicts of run.py:172-175). jitter: site name ->
    [n * batch, length, width] (sigma * draws).

    The chain, on the population kernels with n * batch members of one token row each and no rank-1 terms
    (blocks_forward): the cached input of block `entry` read for every draw with its attn.c_proj jitter folded
    into the residual (noise_block_entry), or the jittered embedding entry normed and mixed; block `entry` with
    its attention-output jitter (noise_add_bf16) and its mlp.c_fc / mlp.c_proj jitter in the block kernel's
    MLP (noise_pop_block_qkv_jit, noise_pop_block_jit); every later block with its mixing; the final norm and
    the fp32 head (split-bf16x3) with the soft cap and per-token CE."""
    from .eggroll import blocks_forward
    model = dust.model
    T, b = dust.length, dust.batch
    dev = dust.y.device
    stream = _lib.stream_ptr(dev)
    rows = n * b * T
    L = model.config.n_layer
    W = _weights(dust)
    batch = _batch_rows(dust, n, entry is not None)
    idx, targets, rope = batch['idx'], batch['targets'], batch['rope']
    x_in = torch.empty(n * b, T, 512, dtype=F32, device=dev)
    h_in = torch.empty(n * b, T, 512, dtype=BF16, device=dev)
    sites = {}
    if entry is None:
        # the jittered embedding entry x = x0 = norm(embedding + jitter), then block 0's mixing and norm
        emb = dust.outputs['transformer.wte'].detach().to(F32).contiguous()
        add = jitter.get('transformer.wte')
        add = None if add is None else add.reshape(n * b, T, -1).to(BF16).contiguous()
        x0 = torch.empty(n * b, T, 512, dtype=F32, device=dev)
        _lib.call('noise_rerun_rows', emb.data_ptr(), b * T, _lib.ptr(add), None, 0, None, None, rows, x0.data_ptr(),
                  stream)
        _lib.call('noise_rerun_mix_norm', x0.data_ptr(), rows, x0.data_ptr(), rows, W.lam_r(0), W.lam_x(0), rows,
                  x_in.data_ptr(), h_in.data_ptr(), stream)
        first = 0
    else:
        # the cached input of block `entry` for every draw (row r reads row r mod batch * length), its norm, and the
        # residual with the attn.c_proj jitter folded in; the block's other jitter sites go to blocks_forward
        x = dust.blocks[entry].detach().to(F32).contiguous()
        width = {'o': 512, 'attn': 512, 'fc': 2048, 'mlp': 512}
        for key, site in SITES.items():
            t = jitter.get(site.format(entry))
            if t is not None:
                sites[key] = t.reshape(n * b, T, width[key]).to(BF16).contiguous()
        attn = sites.pop('attn', None)
        _lib.call('noise_block_entry', x.data_ptr(), b * T, _lib.ptr(attn), rows, x_in.data_ptr(), h_in.data_ptr(),
                  stream)
        x0 = batch['x0']
        first = entry
    loss = blocks_forward(W, first, x_in, h_in, x0, idx, targets, rope=rope, jitter=sites)
    return loss.view(n, b, T)


def rerun_tiled(dust, n, entry, jitter):
    """DUST.rerun (run.py:256-279) with every block on noise_dust_block (the tiled kernels): the form `rerun`
    replaced, kept as its cross-check and as the baseline the rerun benchmark times it against. Same arguments,
    state and result as rerun.

    `dust` carries what the reference's DUST object holds after capture: model (resid_lambdas, x0_lambdas,
    window_sizes, lm_head, config), length, batch, outputs ('transformer.wte' and 'value_embeds.{i}' outputs),
    blocks (block inputs by layer), x0 (the normed embedding), y (targets) and weights (the per-block dicts of
    run.py:172-175). jitter: site name -> [n * batch, length, width] (sigma * draws). The chain: the cached
    input repeated n times (or the jittered embedding entry, normed), each later block's mixing, block_forward
    with the entry block's jitter sites, then the final norm and the fp32 head (head_loss, split-bf16x3)."""
    model = dust.model
    T, b = dust.length, dust.batch
    dev = dust.y.device
    stream = _lib.stream_ptr(dev)
    rows = n * b * T
    L = model.config.n_layer
    lam_r = model.resid_lambdas.detach().to(F32).contiguous()
    lam_x = model.x0_lambdas.detach().to(F32).contiguous()
    if entry is None:
        emb = dust.outputs['transformer.wte'].detach().to(F32).contiguous()
        add = jitter.get('transformer.wte')
        add = None if add is None else add.reshape(n * b, T, -1).to(BF16).contiguous()
        x = torch.empty(n * b, T, 512, dtype=F32, device=dev)
        _lib.call('noise_rerun_rows', emb.data_ptr(), b * T, _lib.ptr(add), None, 0, None, None, rows, x.data_ptr(),
                  stream)
        x0, x0_rows = x, rows
    else:
        x = dust.blocks[entry].detach().to(F32).repeat(n, 1, 1).contiguous()
        x0 = dust.x0.detach().to(F32).contiguous()
        x0_rows = b * T
    cos, sin = _rotary(model, T, dev)
    for i in range(entry or 0, L):
        if entry is None or i > entry:
            xm = torch.empty_like(x)
            _lib.call('noise_rerun_rows', x.data_ptr(), rows, None, x0.data_ptr(), x0_rows, lam_r.data_ptr() + 4 * i,
                      lam_x.data_ptr() + 4 * i, rows, xm.data_ptr(), stream)
            x = xm
        ve = dust.outputs.get(f'value_embeds.{i}')
        ve = None if ve is None else ve.detach().repeat(n, 1, 1)
        sites = {key: jitter.get(site.format(i)) for key, site in SITES.items()} if i == entry else {}
        x = block_forward_eager(x, dust.weights[i], ve, cos, sin, model.window_sizes[i][0], **sites)
    loss = head_loss_eager(x, model.lm_head.weight.detach().float(), dust.y.repeat(n, 1), model.config.vocab_size)
    return loss.view(n, b, T)


def chunk_size(draws, cap):
    """run.py:76-78: the draws per rerun, the largest divisor of `draws` that is at most `cap`."""
    if draws < 1 or cap < 1:
        raise ValueError(f'chunk_size needs positive draws and cap, not {draws} and {cap}')
    return max(n for n in range(1, min(cap, draws) + 1) if draws % n == 0)


def reward_to_go(reward, gamma):
    """run.py:81-86: each token's reward plus the rewards of the later tokens of its sequence, the token k places
    later weighted gamma^k, over the lags whose weight reaches 1e-6. reward [..., t] (the last dim is the
    sequence). A correlation with the weight row gamma^0 .. gamma^(lags - 1) over the right-padded rows."""
    lags = math.ceil(math.log(1e-6) / math.log(gamma))
    weight = torch.pow(torch.tensor(gamma, dtype=reward.dtype, device=reward.device),
                       torch.arange(lags, device=reward.device, dtype=reward.dtype))
    rows = reward.reshape(-1, 1, reward.shape[-1])
    return F.conv1d(F.pad(rows, (0, lags - 1)), weight.view(1, 1, lags)).view(reward.shape)


def _site_width(dust, site):
    """run.py:338: an attention-output site o@i is n_embd wide; any other site as wide as its captured output."""
    return dust.model.config.n_embd if site.startswith('o@') else dust.outputs[site].shape[-1]


def direct_errors(dust, sites, draws, sigma, entry=None, gamma=0.0, retrieved=None):
    """DUST.direct_errors (run.py:332-378) over this library's rerun: each site's output error per token,
    estimated from n orthogonal draws per rerun (n = chunk_size(draws, dust.recipe.nrep)), returned as
    {site: fp32 [batch, length, width]}.

    Per chunk of n draws: the draws a of every site in the draw dtype (dust.orthogonal_noise, run.py:223-238;
    an mlp.c_fc site keeps only its live units, those whose captured output is > 0), the rerun of n jittered
    copies of the batch from block `entry` with sigma * a added at every site (rerun, run.py:256-279), the
    reward clean_loss - perturbed loss per draw and token, centred over the chunk's draws when n > 1, discounted
    over later tokens when gamma > 0 (reward_to_go), corrected by the priors' predicted loss drop when
    `retrieved` holds memory retrievals (prior = alpha[site] * retrieval, masked like the draws), and folded
    into the estimates by noise_draw_errors (bf16 reward times the draws, summed over the chunk's draws, / sigma).
    Finally each estimate is divided by `draws` and the prior, scaled by the centring's 1 - 1/n, added back.

    `dust` carries the reference DUST's state: model, batch, length, outputs, blocks, x0, y, weights, clean_loss
    [batch, length] fp32, dtype (the draws' dtype: bf16 on a GPU), recipe.nrep, alpha, estimates, fits,
    prior_sites and orthogonal_noise(site, draws, chunk, n, b, t, d). Like the reference, it records the
    estimates of prior sites in dust.estimates and, per retrieved site, the least-squares fit statistics
    (<retrieval, unshrunk estimate>, |retrieval|^2) in dust.fits."""
    retrieved = retrieved or {}
    dtype = dust.dtype
    priors = {s: dust.alpha[s] * r for s, r in retrieved.items() if s in dust.alpha}
    n, b, t = chunk_size(draws, dust.recipe.nrep), dust.batch, dust.length
    dev = dust.clean_loss.device
    width = {s: _site_width(dust, s) for s in sites}
    errors = {s: torch.zeros(b, t, width[s], dtype=F32, device=dev) for s in sites}
    # an mlp.c_fc site is jittered at its live units only (ReLU is flat below 0); its prior is masked alike
    live = {s: (dust.outputs[s] > 0).to(BF16).contiguous() for s in sites if s.endswith('mlp.c_fc')}
    for s, mask in live.items():
        if s in priors:
            priors[s] = priors[s] * mask.float()
    mu = {s: p.to(dtype).float() for s, p in priors.items()}  # the priors as the draws' bf16 products see them

    for chunk in range(draws // n):
        a, jitter = {}, {}
        for s in sites:
            draw = dust.orthogonal_noise(s, draws, chunk, n, b, t, width[s])
            if draw.dtype != BF16 or draw.device != dev or draw.shape != (n, b, t, width[s]):
                raise ValueError(f'direct_errors: the draws of {s!r} must be bf16 [{n}, {b}, {t}, {width[s]}] on '
                                 f'{dev} (the reference draws in bf16 on a GPU), got {draw.dtype} {tuple(draw.shape)}')
            # the live-unit mask in place and the jitter sigma * a in one pass (noise_mask_scale)
            draw = draw.contiguous()
            scaled = torch.empty_like(draw)
            _lib.call('noise_mask_scale', draw.data_ptr(), _lib.ptr(live.get(s)), n, b * t * width[s], float(sigma),
                      scaled.data_ptr(), _lib.stream_ptr(dev))
            a[s] = draw.reshape(n * b, t, width[s])
            jitter[s] = scaled.reshape(n * b, t, width[s])
        loss = rerun(dust, n, entry, jitter)
        reward = dust.clean_loss.unsqueeze(0) - loss
        if n > 1:
            reward = reward - reward.mean(0, keepdim=True)
        if gamma:
            reward = reward_to_go(reward, gamma)
        if priors:
            # the loss drop the priors predict, sigma a.mu summed over sites: each site's product rounded to the
            # draw dtype, the sum over sites in it too, then fp32 (run.py:359-363)
            predicted = None
            for s, m in mu.items():
                dot = (a[s].view(n, b, t, -1).float() * m).sum(-1).to(dtype)
                predicted = dot if predicted is None else predicted + dot
            predicted = sigma * predicted.float()
            reward = reward + (predicted - predicted.mean(0, keepdim=True) if n > 1 else predicted)
        for s in sites:
            draw_errors(errors[s], reward, a[s], sigma)

    kept = 1 - 1 / n if n > 1 else 1.0
    out = {}
    for s, e in errors.items():
        out[s] = e / draws + kept * priors[s] if s in priors else e / draws
    dust.estimates.update({s: e for s, e in out.items() if s in dust.prior_sites})
    for s, r in retrieved.items():
        unshrunk = out[s] / kept
        dust.fits[s] = torch.stack([(r * unshrunk).sum(), (r * r).sum()])
    return out
