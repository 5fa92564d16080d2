"""EGGROLL's population forward on libnoise_amd (train/val/eggroll.py:56-168 call sites).

  lowrank(x, weight, a, b, sign)            eggroll.py:56-58
  lowrank_embed(weight, a, b, idx, sign)    eggroll.py:61-63
  population_loss(model, p, noise, sign, idx, targets)   eggroll.py:66-103
  Eggroll(model, pairs).offsets(step) / .noise(offsets, directions)   eggroll.py:106-128

The forward runs as one chain of fused HIP kernels per block (noise_pop_* in include/noise_amd.h):
  qkv (+rank-1, ve gate, rotary, q/k norm) -> attention (+ x.b dots of c_proj) ->
  residual (c_proj, + norm, + c_fc dot) -> fc (ReLU^2, + mlp.c_proj partial dots) ->
  residual (mlp.c_proj, + next block's mix, norm and q/k/v dots) ... -> head + softcap + CE -> mean.
Noise enters as per-direction rows: member m uses row m // dir_div (2 for antithetic pairs) of every
[dirs, out + in] table, never repeated per member.
"""
import ctypes
import math

import torch

from . import _lib
from ._lib import ATTN_QK_NORMED, ATTN_V_TRANSPOSED
from .model import rotary_tables, window_sizes, has_ve, N_EMBD, N_HEAD, HEAD_DIM, VOCAB
from .noise import DeviceGenerator, OrthogonalDraws

BF16 = torch.bfloat16
F32 = torch.float32

BUFFER_NUMEL = 2 ** 28   # eggroll.py:35 NOISE
SEED = 0                 # eggroll.py:29


def _view(t, sm, st):
    return _lib.View(t.data_ptr(), sm, st)


class KernelTimer:
    """Records HIP events around every library launch of the forward on torch's current stream (the
    stream the kernels run on): name -> list of (start, end) event pairs, tagged with a caller label."""

    def __init__(self):
        self.events = []
        self.label = None

    def call(self, name, *args):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        _lib.call(name, *args)
        e.record()
        self.events.append((name, self.label, s, e))

    def totals(self):
        """(name, label) -> (launches, total ms), after a synchronize."""
        out = {}
        for name, label, s, e in self.events:
            n, t = out.get((name, label), (0, 0.0))
            out[(name, label)] = (n + 1, t + s.elapsed_time(e))
        return out


_TIMER = None
_ROPE = {}


def _rope_tables(T, dev):
    """bf16 rotary tables of length T on dev, built once per (T, device): the copy from host memory waits for
    the stream, so a per-call copy would stall the launch queue (the reference keeps them as model buffers,
    model.py:177-183)."""
    key = (T, dev.type, dev.index)
    if key not in _ROPE:
        cos, sin = rotary_tables(T)
        _ROPE[key] = (cos.to(dev).bfloat16().contiguous(), sin.to(dev).bfloat16().contiguous())
    return _ROPE[key]


def _pair_signs(pairs, sigma, device):
    """[+sigma, -sigma] * pairs built on the device (no host copy that would wait for the stream)."""
    sign = torch.full((2 * pairs,), float(sigma), device=device)
    sign[1::2] = -float(sigma)
    return sign


def set_timer(timer):
    """Install (or clear, with None) a KernelTimer for subsequent population_forward calls."""
    global _TIMER
    _TIMER = timer


def _call(name, *args, label=None):
    if _TIMER is None:
        return _lib.call(name, *args)
    _TIMER.label = label
    return _TIMER.call(name, *args)


def _rank1(pair):
    """noise_rank1_t of an (a, b) pair of [dirs, out] / [dirs, in] fp32 row views (None: unperturbed)."""
    if pair is None:
        return _lib.Rank1(None, None, 0, 0)
    a, b = pair
    for t in (a, b):
        if t.dtype != F32 or t.stride(-1) != 1 or t.data_ptr() % 16 or t.stride(0) % 4:
            raise ValueError('noise rows must be fp32, 16 B aligned, unit inner stride')
    return _lib.Rank1(a.data_ptr(), b.data_ptr(), a.stride(0), b.stride(0))


def _rank1_array(pairs):
    arr = (_lib.Rank1 * len(pairs))()
    for i, pr in enumerate(pairs):
        arr[i] = _rank1(pr)
    return arr


class Weights:
    """Device copies of a parameter dict in the layouts the kernels read (bf16 matrices, fp32 tables),
    built once per parameter update. Names are the reference's state-dict names (utils/model.py)."""

    def __init__(self, p, device=None, n_layer=8, fp32_head=False):
        dev = torch.device(device) if device is not None else p['lm_head.weight'].device
        if dev.type != 'cuda':
            raise ValueError('population_loss runs on the GPU')
        self.device, self.n_layer = dev, n_layer
        g = lambda n: p[n].detach().to(dev)
        bf = lambda n: g(n).to(BF16).contiguous()
        # fp32 tables and scalars are copied even when the parameter is already fp32 on the device: a Weights
        # is a snapshot of one update's parameters, never a view of the live ones
        snap = lambda n: g(n).to(F32, copy=True).contiguous()
        self.wte = snap('transformer.wte.weight')
        self.lm_head = bf('lm_head.weight')
        self.fp32_head = fp32_head
        if fp32_head:
            w = g('lm_head.weight').to(F32).contiguous()
            self.lm_head3 = torch.empty(w.shape[0], 3 * w.shape[1], dtype=BF16, device=dev)
            _lib.call('noise_split3', w.data_ptr(), w.shape[0], w.shape[1], 0, 1, self.lm_head3.data_ptr(),
                      _lib.stream_ptr(dev))
        # the mixing scalars stay on the device: the kernels read them there (a host copy would wait for the
        # stream at every update)
        self.resid_lambdas = snap('resid_lambdas')
        self.x0_lambdas = snap('x0_lambdas')
        self.blocks = []
        for i in range(n_layer):
            pre = f'transformer.h.{i}.'
            blk = dict(q=bf(pre + 'attn.c_q.weight'), k=bf(pre + 'attn.c_k.weight'), v=bf(pre + 'attn.c_v.weight'),
                       o=bf(pre + 'attn.c_proj.weight'), fc=bf(pre + 'mlp.c_fc.weight'),
                       mp=bf(pre + 'mlp.c_proj.weight'))
            # mlp.c_fc and mlp.c_proj in the block kernel's column order (within every 32 columns); so are c_q, c_k
            # and c_v of the blocks whose q/k/v the previous block's kernel forms
            perm = [('mp', 'mp_blk'), ('fc', 'fc_blk')]
            if i:
                perm += [('q', 'q_blk'), ('k', 'k_blk'), ('v', 'v_blk')]
            for src, dst in perm:
                blk[dst] = torch.empty_like(blk[src])
                _lib.call('noise_block_weight_layout', blk[src].data_ptr(), blk[dst].data_ptr(), blk[src].shape[0],
                          blk[src].shape[1], _lib.stream_ptr(dev))
            if has_ve(i, n_layer):
                # the gate's product runs under autocast: its weights enter rounded to bf16
                blk['gate'] = bf(pre + 'attn.ve_gate.weight').to(F32).contiguous()
                blk['ve'] = snap(f'value_embeds.{i}.weight')
            self.blocks.append(blk)
        self.windows = window_sizes(n_layer)

    def lam_r(self, i):
        """Device address of resid_lambdas[i] (fp32)."""
        return self.resid_lambdas.data_ptr() + 4 * i

    def lam_x(self, i):
        """Device address of x0_lambdas[i] (fp32)."""
        return self.x0_lambdas.data_ptr() + 4 * i


class _Buffers:
    def __init__(self, m, T, dev, fp32_head, per_member, eager=False):
        rows = m * T
        e = m if per_member else 1
        self.x0 = torch.empty(e, T, N_EMBD, dtype=F32, device=dev)
        self.xin0 = torch.empty(e, T, N_EMBD, dtype=F32, device=dev)
        self.h0 = torch.empty(e, T, N_EMBD, dtype=BF16, device=dev)
        self.resid = torch.empty(m, T, N_EMBD, dtype=F32, device=dev)
        self.h = torch.empty(m, T, N_EMBD, dtype=BF16, device=dev)
        self.qkv = torch.empty(3, m, N_HEAD, T, HEAD_DIM, dtype=BF16, device=dev)
        self.y = torch.empty(m, T, N_EMBD, dtype=BF16, device=dev)
        # the MLP hidden layer: materialised only by the eager-rounding path (the fused MLP keeps it on chip)
        self.act = torch.empty(m, T, 4 * N_EMBD, dtype=BF16, device=dev) if eager else None
        self.h3 = torch.empty(m, T, 3 * N_EMBD, dtype=BF16, device=dev) if fp32_head else None
        # block 0's shared q/k/v product when every member reads the same block input
        self.qkv_base = None if per_member else torch.empty(T, 3 * N_EMBD, dtype=F32, device=dev)
        self.d_qkv = torch.empty(rows, 3, dtype=F32, device=dev)
        self.d_attn = torch.empty(rows, N_HEAD, dtype=F32, device=dev)
        self.d_fc = torch.empty(rows, dtype=F32, device=dev)
        self.d_mp = torch.empty(rows, 16, dtype=F32, device=dev) if eager else None
        self.d_head = torch.empty(rows, 1, dtype=F32, device=dev)
        self.gates = torch.empty(rows, N_HEAD, dtype=F32, device=dev)
        self.loss_tok = torch.empty(rows, dtype=F32, device=dev)


_ZERO_ROWS = {}


def _zero_b(dev, width):
    """A single zero row with stride 0: the b of an unperturbed matrix whose dot slot must still exist."""
    key = (dev, width)
    if key not in _ZERO_ROWS:
        _ZERO_ROWS[key] = torch.zeros(width, dtype=F32, device=dev)
    z = _ZERO_ROWS[key]
    return _lib.Rank1(None, z.data_ptr(), 0, 0)


def population_forward(W, noise, sign, idx, targets, dir_div=1, rope=None, buffers=None, per_token=False,
                       rounding=_lib.ROUNDING_FUSED, fuse_qkv=True):
    """Per-member mean cross-entropy [m] of the perturbed models (eggroll.py:66-103 semantics).

    W: Weights. noise: name -> (a [dirs, out], b [dirs, in]) fp32 row views for matrices and embeddings,
    or eps [dirs, L] for 'resid_lambdas' / 'x0_lambdas'; absent names are unperturbed. sign: [m] fp32
    (+-sigma). Member m uses noise row m // dir_div. idx, targets: [T] int64 token ids shared by all
    members, or [m, T] with one sequence per member (scoring distinct sequences, utils/eval.py:43-46; the
    embedding and mixing scalars unperturbed). rope: (cos, sin) bf16 [T][32] rotary tables on the device
    (default: rotary_tables(T)). per_token: return the [m, T] per-token losses (0 at targets < 0) instead
    of the member means (a view of the buffers' storage). rounding: ROUNDING_FUSED (the compiled training
    forward) or ROUNDING_EAGER (the scorer's eager autocast forward, bf16 residual stream; noise must be
    empty). fuse_qkv: with fused rounding, each block's kernel also forms the next block's gates and q/k/v
    (noise_pop_block_qkv); False launches them on their own (same results up to the products' summation
    order)."""
    dev = W.device
    m, T = sign.shape[0], idx.shape[-1]
    if T % 256:
        raise ValueError(f'sequence length must be a multiple of 256, got {T}')
    rows_in = idx.dim() == 2
    if idx.dim() not in (1, 2) or (rows_in and idx.shape[0] != m) or targets.shape != idx.shape:
        raise ValueError(f'idx and targets must both be [T] or [members, T]; got {tuple(idx.shape)}, '
                         f'{tuple(targets.shape)} for {m} members')
    sign = sign.to(device=dev, dtype=F32).contiguous()
    idx = idx.to(device=dev, dtype=torch.int64).contiguous()
    targets = targets.to(device=dev, dtype=torch.int64).contiguous()
    stream = _lib.stream_ptr(dev)
    if rounding not in (_lib.ROUNDING_FUSED, _lib.ROUNDING_EAGER):
        raise ValueError(f'unknown rounding mode {rounding}')
    if rounding == _lib.ROUNDING_EAGER and (noise or W.fp32_head):
        raise ValueError('eager rounding is the unperturbed bf16 forward: no noise, no fp32 head')
    pop = _lib.Population(m, T, sign.data_ptr(), dir_div, rounding)
    popp = ctypes.byref(pop)
    if rope is None:
        rope = _rope_tables(T, dev)
    cos_t, sin_t = rope
    L = W.n_layer
    E = N_EMBD

    def nz(name):
        v = noise.get(name)
        return v

    eps_r, eps_x = nz('resid_lambdas'), nz('x0_lambdas')
    emb = nz('transformer.wte.weight')
    noisy_entry = emb is not None or eps_r is not None or eps_x is not None
    if rows_in and noisy_entry:
        raise ValueError('per-member token rows need the embedding and mixing scalars unperturbed')
    per_member = noisy_entry or rows_in
    B = buffers if buffers is not None else _Buffers(m, T, dev, W.fp32_head, per_member,
                                                     eager=rounding == _lib.ROUNDING_EAGER)
    # block 0 entry: embedding, norm, mix, norm (shared by every member when nothing there is perturbed;
    # per-member token rows go through as one sequence of m * T tokens: the entry is token-local)
    emb_r1 = _rank1(emb)
    embed_pop = _lib.Population(1, m * T, None, 1, rounding) if rows_in else pop
    _call('noise_pop_embed', ctypes.byref(embed_pop), 1 if noisy_entry else 0, W.wte.data_ptr(), W.wte.shape[0],
              idx.data_ptr(), ctypes.byref(emb_r1), W.lam_r(0), W.lam_x(0),
              None if eps_r is None else eps_r.data_ptr(), None if eps_x is None else eps_x.data_ptr(),
              0 if eps_r is None and eps_x is None else (eps_r if eps_r is not None else eps_x).stride(0),
              B.x0.data_ptr(), B.xin0.data_ptr(), B.h0.data_ptr(), stream)
    sm_e = T * E if per_member else 0
    idx_sm = T if rows_in else 0
    eps_ptr = lambda e, i: None if e is None else e[:, i].data_ptr()
    eps_stride = (eps_r if eps_r is not None else eps_x).stride(0) if (eps_r is not None or eps_x is not None) else 0

    def qkv_noise(i):
        pre = f'transformer.h.{i}.'
        return [nz(pre + 'attn.c_q.weight'), nz(pre + 'attn.c_k.weight'), nz(pre + 'attn.c_v.weight')]

    def dot_vecs(pairs, width):
        arr = (_lib.Rank1 * len(pairs))()
        for k, pr in enumerate(pairs):
            arr[k] = _rank1(pr) if pr is not None else _zero_b(dev, width)
        return arr

    # q/k/v dots of block 0
    n0 = qkv_noise(0)
    if any(v is not None for v in n0):
        _call('noise_member_dots', popp, _view(B.h0, sm_e, E), E, dot_vecs(n0, E), 3, B.d_qkv.data_ptr(), stream)

    qkv_out = (ctypes.c_void_p * 3)(*(B.qkv[i].data_ptr() for i in range(3)))
    qkv_ready = False
    for i in range(L):
        pre = f'transformer.h.{i}.'
        blk = W.blocks[i]
        nq = qkv_noise(i)
        x_in = _view(B.h0, sm_e, E) if i == 0 else _view(B.h, T * E, E)
        ws = (ctypes.c_void_p * 3)(blk['q'].data_ptr(), blk['k'].data_ptr(), blk['v'].data_ptr())
        ve_r1 = _rank1(nz(f'value_embeds.{i}.weight'))
        if qkv_ready:
            qkv_ready = False  # the previous block's kernel formed this block's gates and q/k/v
        else:
            if 've' in blk:
                gate_r1 = _rank1(nz(pre + 'attn.ve_gate.weight'))
                _call('noise_pop_gate', popp, x_in, blk['gate'].data_ptr(), ctypes.byref(gate_r1), B.gates.data_ptr(),
                      stream)
            if i == 0 and B.qkv_base is not None and 've' not in blk and rounding == _lib.ROUNDING_FUSED:
                # every member reads the same block input: its product with c_q, c_k, c_v is computed once and
                # each member adds its rank-1 terms before rotary and norm
                one = _lib.Population(1, T, None, 1, _lib.ROUNDING_FUSED)
                for j in range(3):
                    _call('noise_pop_linear', ctypes.byref(one), x_in, ws[j], E, E, None, None,
                          B.qkv_base.data_ptr() + 4 * E * j, 1, T * 3 * E, 3 * E, stream)
                _call('noise_pop_qkv_shared', popp, B.qkv_base.data_ptr(), _rank1_array(nq), B.d_qkv.data_ptr(),
                      cos_t.data_ptr(), sin_t.data_ptr(), qkv_out, stream)
            else:
                _call('noise_pop_qkv', popp, x_in, ws, _rank1_array(nq), B.d_qkv.data_ptr(), cos_t.data_ptr(),
                      sin_t.data_ptr(), blk['ve'].data_ptr() if 've' in blk else None,
                      blk['ve'].shape[0] if 've' in blk else 0, idx.data_ptr(), idx_sm,
                      B.gates.data_ptr() if 've' in blk else None, ctypes.byref(ve_r1), qkv_out, stream)
        # attention; its epilogue also forms y . b_o per head for c_proj's rank-1 term
        no = nz(pre + 'attn.c_proj.weight')
        q4, k4 = (B.qkv[j].transpose(1, 2) for j in range(2))  # [m, T, H, D] views of [m, H, T, D]
        vt = B.qkv[2].view(m, N_HEAD, HEAD_DIM, T)               # V^T as the qkv kernel writes it
        yv = B.y.view(m, T, N_HEAD, HEAD_DIM)
        _call('noise_attention_fwd', q4.data_ptr(), k4.data_ptr(), vt.data_ptr(), yv.data_ptr(), m, N_HEAD, T,
                  HEAD_DIM, q4.stride(0), q4.stride(2), q4.stride(1), k4.stride(0), k4.stride(2), k4.stride(1),
                  vt.stride(0), vt.stride(1), vt.stride(2), ATTN_V_TRANSPOSED | ATTN_QK_NORMED,
                  yv.stride(0), yv.stride(2), yv.stride(1),
                  W.windows[i], 1.0 / math.sqrt(HEAD_DIM), None if no is None else no[1].data_ptr(),
                  0 if no is None else no[1].stride(0), dir_div, None if no is None else B.d_attn.data_ptr(),
                  stream, label=f'window {W.windows[i]}')
        nfc, nmp = nz(pre + 'mlp.c_fc.weight'), nz(pre + 'mlp.c_proj.weight')
        o_r1 = _rank1(no)
        xres = _view(B.xin0, sm_e, E) if i == 0 else _view(B.resid, T * E, E)
        fc_r1 = _rank1(nfc)
        mp_r1 = _rank1(nmp)
        last = i == L - 1
        if rounding == _lib.ROUNDING_FUSED:
            # attn.c_proj, residual, norm and the whole MLP with its residual writer in one kernel: neither the
            # mid-block residual, its norm nor the [m, T, 2048] hidden layer reaches HBM; then the next block's
            # mix, norm and q/k/v dots (or the head input)
            if not last:
                nn = qkv_noise(i + 1)
                want = any(v is not None for v in nn)
                nxt, nnext, ndots = (dot_vecs(nn, E), 3, B.d_qkv.data_ptr()) if want else (None, 0, None)
                hout, split3 = B.h, 0
                mixargs = (1, W.lam_r(i + 1), W.lam_x(i + 1), eps_ptr(eps_r, i + 1), eps_ptr(eps_x, i + 1), eps_stride)
            else:
                nh = nz('lm_head.weight')
                nxt, nnext, ndots = (dot_vecs([nh], E), 1, B.d_head.data_ptr()) if nh is not None else (None, 0, None)
                hout, split3 = (B.h3, 1) if W.fp32_head else (B.h, 0)
                mixargs = (0, None, None, None, None, 0)
            if not last and fuse_qkv:
                # ... and the next block's gates and q/k/v from its normalised input, which stays in registers
                nblk, npre = W.blocks[i + 1], f'transformer.h.{i + 1}.'
                nws = (ctypes.c_void_p * 3)(nblk['q_blk'].data_ptr(), nblk['k_blk'].data_ptr(),
                                            nblk['v_blk'].data_ptr())
                n_ve, n_gate = _rank1(nz(f'value_embeds.{i + 1}.weight')), _rank1(nz(npre + 'attn.ve_gate.weight'))
                _call('noise_pop_block_qkv', popp, _view(B.y, T * E, E), blk['o'].data_ptr(), ctypes.byref(o_r1),
                      B.d_attn.data_ptr(), N_HEAD, xres, blk['fc_blk'].data_ptr(), ctypes.byref(fc_r1),
                      blk['mp_blk'].data_ptr(), ctypes.byref(mp_r1), B.resid.data_ptr(), *mixargs,
                      _view(B.x0, sm_e, E), nws, _rank1_array(nn), cos_t.data_ptr(), sin_t.data_ptr(),
                      nblk['ve'].data_ptr() if 've' in nblk else None, nblk['ve'].shape[0] if 've' in nblk else 0,
                      idx.data_ptr(), idx_sm, nblk['gate'].data_ptr() if 've' in nblk else None,
                      ctypes.byref(n_gate), ctypes.byref(n_ve), qkv_out, stream, label='block')
                qkv_ready = True
                continue
            _call('noise_pop_block', popp, _view(B.y, T * E, E), blk['o'].data_ptr(), ctypes.byref(o_r1),
                  B.d_attn.data_ptr(), N_HEAD, xres, blk['fc_blk'].data_ptr(), ctypes.byref(fc_r1),
                  blk['mp_blk'].data_ptr(), ctypes.byref(mp_r1), None if last else B.resid.data_ptr(), *mixargs,
                  _view(B.x0, sm_e, E), hout.data_ptr(), split3, nxt, nnext, ndots, stream, label='block')
            continue
        # eager rounding: attn.c_proj + residual; h = norm(x_mid) (no rank-1 terms in this mode)
        _call('noise_pop_residual', popp, _view(B.y, T * E, E), blk['o'].data_ptr(), E, ctypes.byref(o_r1),
                  B.d_attn.data_ptr(), N_HEAD, N_HEAD, xres, B.resid.data_ptr(), 0, None, None, None, None, 0,
                  _view(B.x0, sm_e, E), B.h.data_ptr(), 0, None, 0, None, stream, label='attn.c_proj')
        # mlp.c_fc, ReLU^2 and partial dots for mlp.c_proj, then mlp.c_proj + residual
        mp_next = _rank1(nmp)
        _call('noise_pop_fc', popp, _view(B.h, T * E, E), blk['fc'].data_ptr(), ctypes.byref(fc_r1),
                  B.d_fc.data_ptr(), B.act.data_ptr(), ctypes.byref(mp_next) if nmp is not None else None,
                  B.d_mp.data_ptr(), stream)
        if not last:
            nn = qkv_noise(i + 1)
            want = any(v is not None for v in nn)
            nxt, nnext, ndots = (dot_vecs(nn, E), 3, B.d_qkv.data_ptr()) if want else (None, 0, None)
            _call('noise_pop_residual', popp, _view(B.act, T * 4 * E, 4 * E), blk['mp'].data_ptr(), 4 * E,
                  ctypes.byref(mp_r1), B.d_mp.data_ptr(), 16, 16, _view(B.resid, T * E, E), B.resid.data_ptr(),
                  1, W.lam_r(i + 1), W.lam_x(i + 1), eps_ptr(eps_r, i + 1), eps_ptr(eps_x, i + 1),
                  eps_stride, _view(B.x0, sm_e, E), B.h.data_ptr(), 0, nxt, nnext, ndots, stream, label='mlp.c_proj')
        else:
            nh = nz('lm_head.weight')
            nxt, nnext, ndots = (dot_vecs([nh], E), 1, B.d_head.data_ptr()) if nh is not None else (None, 0, None)
            hout = B.h3 if W.fp32_head else B.h
            _call('noise_pop_residual', popp, _view(B.act, T * 4 * E, 4 * E), blk['mp'].data_ptr(), 4 * E,
                  ctypes.byref(mp_r1), B.d_mp.data_ptr(), 16, 16, _view(B.resid, T * E, E), None, 0, None, None,
                  None, None, 0, _view(B.x0, sm_e, E), hout.data_ptr(), 1 if W.fp32_head else 0, nxt, nnext,
                  ndots, stream, label='mlp.c_proj')
    nh = nz('lm_head.weight')
    head_r1 = _rank1(nh)
    if W.fp32_head:
        hx, hw, K = _view(B.h3, T * 3 * E, 3 * E), W.lm_head3, 3 * E
    else:
        hx, hw, K = _view(B.h, T * E, E), W.lm_head, E
    _call('noise_pop_head_ce', popp, hx, hw.data_ptr(), K, VOCAB, ctypes.byref(head_r1), B.d_head.data_ptr(),
              targets.data_ptr(), idx_sm, B.loss_tok.data_ptr(), stream)
    if per_token:
        return B.loss_tok.view(m, T)
    out = torch.empty(m, dtype=F32, device=dev)
    _call('noise_member_mean', B.loss_tok.data_ptr(), m, T, out.data_ptr(), stream)
    return out


_ZERO_BF16 = {}


def _zero_row_bf16(dev):
    """512 zero bf16 values on dev (the mlp.c_proj jitter row a jittered block reads when it has none)."""
    if dev not in _ZERO_BF16:
        _ZERO_BF16[dev] = torch.zeros(N_EMBD, dtype=BF16, device=dev)
    return _ZERO_BF16[dev]


def blocks_forward(W, first, x_in, h_in, x0, idx, targets, rope=None, buffers=None, jitter=None):
    """Per-token losses [m, T] of the fixed (unperturbed) model run from block `first` on m token rows: the
    blocks first .. L-1 on the population kernels (the same launches as population_forward's fused path), the
    final norm and the head (fp32 as split-bf16x3 when W.fp32_head), the soft cap and CE (ignore_index -1).

    x_in: fp32 [m, T, 512], block `first`'s input after its mixing; h_in: bf16 [m, T, 512] = norm(x_in); x0:
    fp32 [m, T, 512], the normed embedding every block mixes in; idx, targets: [m, T] int64 (one token row per
    member: the value embeddings of blocks with them, and the head's targets). jitter: block `first`'s
    block_forward jitter (run.py:102-117) by keyword, bf16 [m, T, width] each: 'o' (the attention output),
    'fc' (mlp.c_fc's product, before ReLU^2), 'mlp' (mlp.c_proj's product); its attn.c_proj jitter is the
    caller's to fold into x_in (noise_block_entry). DUST's rerun runs its blocks this way (run.py:256-279)."""
    dev = W.device
    m, T = idx.shape
    E = N_EMBD
    L = W.n_layer
    if T % 256 or targets.shape != idx.shape:
        raise ValueError(f'blocks_forward: [members, T] rows with T a multiple of 256; got {tuple(idx.shape)}, '
                         f'{tuple(targets.shape)}')
    if not 0 <= first < L:
        raise ValueError(f'blocks_forward: first block {first} outside 0 .. {L - 1}')
    jitter = {k: v for k, v in (jitter or {}).items() if v is not None}
    if set(jitter) - {'o', 'fc', 'mlp'}:
        raise ValueError(f'blocks_forward: jitter at o, fc or mlp only, got {sorted(jitter)}')
    if jitter and not W.fp32_head and first == L - 1:
        raise ValueError('blocks_forward: a jittered last block feeds the fp32 head (Weights(fp32_head=True))')
    jit = {}
    for k, width in (('o', E), ('fc', 4 * E), ('mlp', E)):
        if k in jitter:
            t = jitter[k]
            if t.shape != (m, T, width) or t.dtype != BF16 or not t.is_contiguous():
                raise ValueError(f'blocks_forward: jitter {k!r} must be contiguous bf16 [{m}, {T}, {width}]')
            jit[k] = t
    for t, dt in ((x_in, F32), (h_in, BF16), (x0, F32)):
        if t.shape != (m, T, E) or t.dtype != dt or not t.is_contiguous():
            raise ValueError(f'blocks_forward: x_in, x0 fp32 and h_in bf16, contiguous [{m}, {T}, {E}]')
    idx = idx.to(device=dev, dtype=torch.int64).contiguous()
    targets = targets.to(device=dev, dtype=torch.int64).contiguous()
    stream = _lib.stream_ptr(dev)
    sign = torch.zeros(m, dtype=F32, device=dev)
    pop = _lib.Population(m, T, sign.data_ptr(), 1, _lib.ROUNDING_FUSED)
    popp = ctypes.byref(pop)
    cos_t, sin_t = rope if rope is not None else _rope_tables(T, dev)
    B = buffers if buffers is not None else _Buffers(m, T, dev, W.fp32_head, True)
    none = _lib.Rank1(None, None, 0, 0)
    none3 = _rank1_array([None, None, None])
    qkv_out = (ctypes.c_void_p * 3)(*(B.qkv[i].data_ptr() for i in range(3)))
    x0v = _view(x0, T * E, E)
    # block `first`: its value-embedding gates and q/k/v from h_in
    blk = W.blocks[first]
    ws = (ctypes.c_void_p * 3)(blk['q'].data_ptr(), blk['k'].data_ptr(), blk['v'].data_ptr())
    if 've' in blk:
        _call('noise_pop_gate', popp, _view(h_in, T * E, E), blk['gate'].data_ptr(), ctypes.byref(none),
              B.gates.data_ptr(), stream)
    _call('noise_pop_qkv', popp, _view(h_in, T * E, E), ws, none3, B.d_qkv.data_ptr(), cos_t.data_ptr(),
          sin_t.data_ptr(), blk['ve'].data_ptr() if 've' in blk else None, blk['ve'].shape[0] if 've' in blk else 0,
          idx.data_ptr(), T, B.gates.data_ptr() if 've' in blk else None, ctypes.byref(none), qkv_out, stream)
    for i in range(first, L):
        blk = W.blocks[i]
        q4, k4 = (B.qkv[j].transpose(1, 2) for j in range(2))
        vt = B.qkv[2].view(m, N_HEAD, HEAD_DIM, T)
        yv = B.y.view(m, T, N_HEAD, HEAD_DIM)
        _call('noise_attention_fwd', q4.data_ptr(), k4.data_ptr(), vt.data_ptr(), yv.data_ptr(), m, N_HEAD, T,
              HEAD_DIM, q4.stride(0), q4.stride(2), q4.stride(1), k4.stride(0), k4.stride(2), k4.stride(1),
              vt.stride(0), vt.stride(1), vt.stride(2), ATTN_V_TRANSPOSED | ATTN_QK_NORMED,
              yv.stride(0), yv.stride(2), yv.stride(1), W.windows[i], 1.0 / math.sqrt(HEAD_DIM), None, 0, 1, None,
              stream, label=f'window {W.windows[i]}')
        xres = _view(x_in, T * E, E) if i == first else _view(B.resid, T * E, E)
        if i == first and jit:
            if 'o' in jit:
                _call('noise_add_bf16', B.y.data_ptr(), jit['o'].data_ptr(), B.y.numel(), stream)
            if 'fc' in jit or 'mlp' in jit:
                js = _lib.BlockJitter(_lib.ptr(jit.get('fc')), _lib.ptr(jit.get('mlp')),
                                      _zero_row_bf16(dev).data_ptr())
                if i < L - 1:
                    nblk = W.blocks[i + 1]
                    nws = (ctypes.c_void_p * 3)(nblk['q_blk'].data_ptr(), nblk['k_blk'].data_ptr(),
                                                nblk['v_blk'].data_ptr())
                    _call('noise_pop_block_qkv_jit', popp, _view(B.y, T * E, E), blk['o'].data_ptr(), xres,
                          blk['fc_blk'].data_ptr(), blk['mp_blk'].data_ptr(), B.resid.data_ptr(), W.lam_r(i + 1),
                          W.lam_x(i + 1), x0v, nws, cos_t.data_ptr(), sin_t.data_ptr(),
                          nblk['ve'].data_ptr() if 've' in nblk else None, nblk['ve'].shape[0] if 've' in nblk else 0,
                          idx.data_ptr(), T, nblk['gate'].data_ptr() if 've' in nblk else None, qkv_out,
                          ctypes.byref(js), stream, label='block (jitter)')
                else:
                    _call('noise_pop_block_jit', popp, _view(B.y, T * E, E), blk['o'].data_ptr(), xres,
                          blk['fc_blk'].data_ptr(), blk['mp_blk'].data_ptr(), 0, None, None, x0v, B.h3.data_ptr(), 1,
                          ctypes.byref(js), stream, label='block (jitter)')
                continue
        if i < L - 1:
            # the block, then the next block's mixing, norm, gates and q/k/v (norm and dots stay in registers)
            nblk = W.blocks[i + 1]
            nws = (ctypes.c_void_p * 3)(nblk['q_blk'].data_ptr(), nblk['k_blk'].data_ptr(), nblk['v_blk'].data_ptr())
            _call('noise_pop_block_qkv', popp, _view(B.y, T * E, E), blk['o'].data_ptr(), ctypes.byref(none),
                  B.d_attn.data_ptr(), N_HEAD, xres, blk['fc_blk'].data_ptr(), ctypes.byref(none),
                  blk['mp_blk'].data_ptr(), ctypes.byref(none), B.resid.data_ptr(), 1, W.lam_r(i + 1),
                  W.lam_x(i + 1), None, None, 0, x0v, nws, none3, cos_t.data_ptr(), sin_t.data_ptr(),
                  nblk['ve'].data_ptr() if 've' in nblk else None, nblk['ve'].shape[0] if 've' in nblk else 0,
                  idx.data_ptr(), T, nblk['gate'].data_ptr() if 've' in nblk else None, ctypes.byref(none),
                  ctypes.byref(none), qkv_out, stream, label='block')
        else:
            hout, split3 = (B.h3, 1) if W.fp32_head else (B.h, 0)
            _call('noise_pop_block', popp, _view(B.y, T * E, E), blk['o'].data_ptr(), ctypes.byref(none),
                  B.d_attn.data_ptr(), N_HEAD, xres, blk['fc_blk'].data_ptr(), ctypes.byref(none),
                  blk['mp_blk'].data_ptr(), ctypes.byref(none), None, 0, None, None, None, None, 0, x0v,
                  hout.data_ptr(), split3, None, 0, None, stream, label='block')
    if W.fp32_head:
        hx, hw, K = _view(B.h3, T * 3 * E, 3 * E), W.lm_head3, 3 * E
    else:
        hx, hw, K = _view(B.h, T * E, E), W.lm_head, E
    _call('noise_pop_head_ce', popp, hx, hw.data_ptr(), K, VOCAB, ctypes.byref(none), B.d_head.data_ptr(),
          targets.data_ptr(), T, B.loss_tok.data_ptr(), stream)
    return B.loss_tok.view(m, T)


def population_loss(model, p, noise, sign, idx, targets, dir_div=1, fp32_head=False):
    """eggroll.py:66-103 `population_loss(model, p, noise, sign, idx, targets)` on the GPU: the mean
    cross-entropy [m] of m perturbed models on one sequence.

    p: parameters by name; noise: name -> (a, b) for matrices and embeddings, or eps [m, L] for the mixing
    scalars (names absent from noise are unperturbed). noise values may be per member (dir_div = 1, as the
    reference passes them after repeat_interleave(2), eggroll.py:141) or per direction with dir_div = 2
    (member m uses row m // 2). The call goes through the registered op torch.ops.noise_amd.population_loss,
    so it also runs behind the reference's `torch.compile(population_loss)` (eggroll.py:115) and under its
    autocast (eggroll.py:144)."""
    names = list(p.keys())
    noise_a, noise_b = [], []
    for n in names:
        v = noise.get(n)
        if isinstance(v, (tuple, list)):
            noise_a.append(v[0])
            noise_b.append(v[1])
        else:
            noise_a.append(v)
            noise_b.append(None)
    n_layer = model.config.n_layer if model is not None else 8
    return torch.ops.noise_amd.population_loss('\n'.join(names), [p[n] for n in names], noise_a, noise_b, sign,
                                               idx, targets, n_layer, dir_div, fp32_head)


def population_loss_eager(p, noise, sign, idx, targets, n_layer=8, dir_div=1, fp32_head=False):
    """The op behind population_loss: device weights from p, then the fused forward."""
    W = Weights(p, fp32_head=fp32_head, n_layer=n_layer)
    return population_forward(W, noise, sign, idx, targets, dir_div=dir_div)


def _pop(m, T, sign, dir_div):
    return _lib.Population(m, T, None if sign is None else sign.data_ptr(), dir_div)


def lowrank(x, weight, a, b, sign, dir_div=1):
    """eggroll.py:56-58 `lowrank(x, weight, a, b, sign)`: lowrank_eager through the registered op
    torch.ops.noise_amd.lowrank, so compiled callers trace it."""
    return torch.ops.noise_amd.lowrank(x, weight, a, b, sign, dir_div)


def lowrank_eager(x, weight, a, b, sign, dir_div=1):
    """eggroll.py:56-58: x [m, T, in] through W [out, in] + sign * a b^T per member, never materialised.

    a [dirs, out], b [dirs, in] fp32 rows, member m uses row m // dir_div; sign [m]. Returns fp32
    [m, T, out] in autocast's form (the reference calls it under torch.autocast, eggroll.py:144): the
    product x W^T and the dot x . b are bf16, the rank-1 term is added in fp32. Any shape is served: in a
    multiple of 512 with out and T multiples of 256 run on the MFMA tiles (x broadcast over members, stride 0
    in dim 0, is multiplied once and the rank-1 terms streamed out); other shapes, such as the value-embedding
    gate's [8, 32] weight on h[..., :32] (eggroll.py:88), on noise_lowrank_rows. x may be a strided view."""
    m, T, n_in = x.shape
    n_out = weight.shape[0]
    dev = x.device
    if weight.shape[1] != n_in or a.shape[-1] != n_out or b.shape[-1] != n_in or sign.shape[0] != m:
        raise ValueError(f'lowrank: x {tuple(x.shape)}, weight {tuple(weight.shape)}, a {tuple(a.shape)}, '
                         f'b {tuple(b.shape)} and sign {tuple(sign.shape)} do not agree')
    if a.shape[0] * dir_div < m or b.shape[0] * dir_div < m:
        raise ValueError(f'lowrank: {a.shape[0]} noise rows cannot serve {m} members at dir_div {dir_div}')
    sign = sign.to(device=dev, dtype=F32).contiguous()
    ok = lambda t: t.dtype == F32 and t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and t.stride(0) % 4 == 0
    a = a if ok(a) else a.float().contiguous()
    b = b.to(BF16).to(F32).contiguous()   # autocast rounds b to bf16 for the x . b matmul
    r1 = _rank1((a, b))
    stream = _lib.stream_ptr(dev)
    w = weight.to(device=dev, dtype=BF16).contiguous()
    shared = x.stride(0) == 0
    xb = (x[:1] if shared else x).to(BF16)
    pop = _pop(m, T, sign, dir_div)
    y = torch.empty(m, T, n_out, dtype=F32, device=dev)
    if n_in % 512 or n_out % 256 or T % 256:
        # shapes outside the MFMA tiles: one thread per output element
        if xb.stride(-1) != 1:
            xb = xb.contiguous()
        _lib.call('noise_lowrank_rows', ctypes.byref(pop), _lib.View(xb.data_ptr(), 0 if shared else xb.stride(0),
                                                                      xb.stride(1)),
                  n_in, w.data_ptr(), n_out, ctypes.byref(r1), y.data_ptr(), stream)
        return y
    if xb.stride(-1) != 1 or xb.stride(1) % 8 or xb.data_ptr() % 16 or (not shared and xb.stride(0) % 8):
        xb = xb.contiguous()
    if shared:
        # x is the same for every member, so x W^T and the dots x . b (one per direction) are computed once,
        # as two products over the shared rows (the b rows as a bf16 weight, padded to the 256-row tile); the
        # members' outputs are then a rank-1 expansion
        xv = _lib.View(xb.data_ptr(), 0, xb.stride(1))
        one = _pop(1, T, None, 1)
        base = torch.empty(1, T, n_out, dtype=F32, device=dev)
        _lib.call('noise_pop_linear', ctypes.byref(one), xv, w.data_ptr(), n_in, n_out, None, None, base.data_ptr(),
                  _lib.LINEAR_AUTOCAST, T * n_out, n_out, stream)
        dirs = -(-m // dir_div)
        dpad = -(-dirs // 256) * 256
        bw = torch.zeros(dpad, n_in, dtype=BF16, device=dev)
        bw[:dirs] = b[:dirs]  # b holds bf16 values already: exact
        dots = torch.empty(T, dpad, dtype=F32, device=dev)
        _lib.call('noise_pop_linear', ctypes.byref(one), xv, bw.data_ptr(), n_in, dpad, None, None, dots.data_ptr(),
                  _lib.LINEAR_AUTOCAST, T * dpad, dpad, stream)
        _lib.call('noise_rank1_expand', ctypes.byref(pop), base.data_ptr(), n_out, dots.data_ptr(), dpad,
                  ctypes.byref(r1), y.data_ptr(), _lib.LINEAR_AUTOCAST, stream)
        return y
    dots = torch.empty(m * T, dtype=F32, device=dev)
    _lib.call('noise_member_dots', ctypes.byref(pop), _lib.View(xb.data_ptr(), xb.stride(0), xb.stride(1)), n_in,
              ctypes.byref(r1), 1, dots.data_ptr(), stream)
    _lib.call('noise_pop_linear', ctypes.byref(pop), _lib.View(xb.data_ptr(), xb.stride(0), xb.stride(1)), w.data_ptr(),
              n_in, n_out, ctypes.byref(r1), dots.data_ptr(), y.data_ptr(), _lib.LINEAR_AUTOCAST, T * n_out,
              n_out, stream)
    return y


def lowrank_embed(weight, a, b, idx, sign, dir_div=1):
    """eggroll.py:61-63 `lowrank_embed(weight, a, b, idx, sign)` through the registered op."""
    return torch.ops.noise_amd.lowrank_embed(weight, a, b, idx, sign, dir_div)


def lowrank_embed_eager(weight, a, b, idx, sign, dir_div=1):
    """eggroll.py:61-63: embedding rows of W [V, d] + sign * a b^T for token ids idx [T] -> fp32 [m, T, d]
    (an id outside [0, V) gives a NaN row)."""
    dev = weight.device
    V, d = weight.shape
    m, T = sign.shape[0], idx.shape[0]
    w = weight.to(F32).contiguous()
    sign = sign.to(device=dev, dtype=F32).contiguous()
    idx = idx.to(device=dev, dtype=torch.int64).contiguous()
    a = a.float().contiguous()
    b = b.float().contiguous()
    out = torch.empty(m, T, d, dtype=F32, device=dev)
    r1 = _rank1((a, b))
    _lib.call('noise_lowrank_embed', out.data_ptr(), w.data_ptr(), V, d, idx.data_ptr(),
              ctypes.byref(_pop(m, T, sign, dir_div)), ctypes.byref(r1), _lib.stream_ptr(dev))
    return out


def member_plan(pairs, sequences, rank=0, world=1, chunk=512):
    """The member bookkeeping of eggroll.py:133-146 for one rank: the population has max(2 pairs, 2 sequences)
    members, every sequence hosting the same number (per_seq); rank r evaluates members [r per_rank,
    (r + 1) per_rank) in chunks of `chunk` (an even count; a chunk takes the sequence of its first member,
    as the reference's chunk loop does), member g on direction (g mod 2 pairs) // 2 with sign +sigma for even
    g. Returns [(start, n, first direction, sequence)] per chunk, on the host (no device work)."""
    members = max(2 * pairs, 2 * sequences)
    per_seq, per_rank = members // sequences, members // world
    if chunk % 2 or per_rank % 2:
        raise ValueError(f'member_plan: chunk ({chunk}) and members per rank ({per_rank}) must be even')
    plan = []
    for start in range(rank * per_rank, (rank + 1) * per_rank, chunk):
        n = min(chunk, (rank + 1) * per_rank - start)
        plan.append((start, n, (start % (2 * pairs)) // 2, start // per_seq))
    return plan


class Eggroll:
    """EGGROLL's perturbation bookkeeping (eggroll.py:106-128) over the virtual noise buffer.

    The reference draws buffer = torch.randn(2**28) once (1 GiB of HBM) and slices each direction's a, b
    at per-step offsets. Here the buffer is a Draw: every slice is regenerated from the Philox counter,
    bit-identical to the reference's buffer on the same GPU, and nothing is materialised beyond the
    requested rows."""

    def __init__(self, model, pairs, rank=0, world=1, seed=SEED, noise_numel=BUFFER_NUMEL):
        self.model, self.pairs, self.rank, self.world = model, pairs, rank, world
        self.params = dict(model.named_parameters())
        self.device = next(iter(self.params.values())).device
        self.seed, self.noise_numel = seed, noise_numel
        self.buffer = DeviceGenerator(seed, self.device).take(noise_numel)

    def offsets(self, step):
        """eggroll.py:117-120: one randint draw of [pairs] per parameter, in named_parameters order."""
        g = DeviceGenerator(1_000_003 * self.seed + step, self.device)
        return {name: g.randint(0, self.noise_numel - sum(p.shape), (self.pairs,)) for name, p in self.params.items()}

    def noise(self, offsets, directions):
        """eggroll.py:122-128: name -> (a [n, out], b [n, in]) for matrices and embeddings, eps [n, L]."""
        out = {}
        for name, p in self.params.items():
            rows = self.buffer.gather(offsets[name], sum(p.shape), rows=directions)
            out[name] = tuple(rows.split(list(p.shape), dim=1)) if p.dim() == 2 else rows
        return out

    def noise_tables(self, offsets, directions):
        """Eggroll.noise's values for the parameters in `offsets` at `directions`, regenerated in one launch for
        the matrices whose rows are whole multiples of 256 (every block matrix and the head: a [dirs, sum of
        out + in] table, each parameter's a and b column views of it) and per parameter for the rest."""
        out = {}
        grouped = [n for n in offsets if self.params[n].dim() == 2 and sum(self.params[n].shape) % 256 == 0]
        if grouped:
            widths = [sum(self.params[n].shape) for n in grouped]
            table = self.buffer.gather_many([offsets[n] for n in grouped], widths, directions)
            col = 0
            for n, w in zip(grouped, widths):
                o, i = self.params[n].shape
                out[n] = (table[:, col:col + o], table[:, col + o:col + w])
                col += w
        for name, o in offsets.items():
            if name in out:
                continue
            p = self.params[name]
            rows = self.buffer.gather(o, sum(p.shape), rows=directions)
            out[name] = tuple(rows.split(list(p.shape), dim=1)) if p.dim() == 2 else rows
        return out

    def population(self, step, x, y, weights=None, chunk=512, names=None, fp32_head=False):
        """This rank's population losses for one update (the hot loop of eggroll.py:133-146): members
        [rank * per_rank, (rank + 1) * per_rank), member g on direction (g mod 2P) // 2 with sign
        +sigma for even g and -sigma for odd g, sequence g // per_seq. names restricts which parameters
        are perturbed (None: all, as the reference)."""
        pairs = self.pairs
        offsets = self.offsets(step)
        if names is not None:
            offsets = {n: o for n, o in offsets.items() if n in names}
        W = weights if weights is not None else Weights(self.params, fp32_head=fp32_head)
        plan = member_plan(pairs, len(x), self.rank, self.world, chunk)
        per_rank = sum(c[1] for c in plan)
        losses = torch.empty(per_rank, device=self.device)
        for start, n, _, seq in plan:
            directions = (torch.arange(start, start + n, 2, device=self.device) % (2 * pairs)) // 2
            noise = self.noise_tables(offsets, directions)
            sign = _pair_signs(n // 2, SIGMA, self.device)
            losses[start - self.rank * per_rank:start - self.rank * per_rank + n] = population_forward(
                W, noise, sign, x[seq], y[seq], dir_div=2)
        return losses

    def update(self, losses, offsets, chunk=8192, materialise=None):
        """The gradients of eggroll.py:151-165 (name -> p.grad, fp32 in the parameter's shape) from one
        update's gathered losses [members] and its offsets (self.offsets(step)).

        noise_update_weights turns the antithetic losses into per-direction weights (z-scored fitness summed
        per direction); noise_update_gradients forms -(1/F) sum_d w_d a_d b_d^T for every matrix and
        -(1/F) sum_d w_d eps_d for the 1-D scalars, matrices as split-bf16x3 MFMA GEMMs over chunks of
        `chunk` directions. The matrices' slices are regenerated from the Philox counter when the update
        draws fewer elements than the buffer holds; past that (materialise None) the draw is materialised
        once (1 GiB, kept for later updates, as the reference keeps its buffer) and read instead."""
        losses = losses.to(device=self.device, dtype=torch.float32).contiguous()
        members = losses.numel()
        fitness_count = members // 2
        stream = _lib.stream_ptr(self.device)
        weight = torch.empty(self.pairs, device=self.device, dtype=torch.float32)
        _lib.call('noise_update_weights', _lib.ptr(losses), members, self.pairs, _lib.ptr(weight), stream)
        grads = {n: torch.empty(p.shape, device=self.device, dtype=torch.float32) for n, p in self.params.items()}
        names = list(self.params)
        d = self.buffer
        if materialise is None:
            materialise = self.pairs * sum(sum(p.shape) for p in self.params.values()) > d.numel
        if materialise and getattr(self, '_materialised', None) is None:
            self._materialised = d.normal()
        buf = self._materialised if materialise else None
        keep = []
        for start in range(0, len(names), 64):
            group = names[start:start + 64]
            table = (_lib.UpdateParam * len(group))()
            for i, n in enumerate(group):
                p = self.params[n]
                off = offsets[n].to(device=self.device, dtype=torch.int64).contiguous()
                if off.numel() != self.pairs:
                    raise ValueError(f'{n}: {off.numel()} offsets for {self.pairs} pairs')
                keep.append(off)
                table[i] = _lib.UpdateParam(off.data_ptr(), grads[n].data_ptr(), p.shape[0],
                                            p.shape[1] if p.dim() == 2 else 0)
            need = _lib.lib().noise_update_workspace_bytes(table, len(group), self.pairs, chunk)
            if need < 0:
                raise ValueError('noise_update_workspace_bytes: invalid arguments')
            ws = torch.empty(max(need, 1), device=self.device, dtype=torch.uint8)
            _lib.call('noise_update_gradients', table, len(group), self.pairs, _lib.ptr(weight),
                      -1.0 / fitness_count, chunk, d.numel, d.seed, d.offset, d.threads, _lib.ptr(buf), _lib.ptr(ws),
                      need, stream)
        return grads

    def step(self, x, y, optimizer, step, chunk=512, update_chunk=4096):
        """eggroll.py:131-168 on one GPU: evaluate the population, rebuild the update, step the optimizer;
        returns the mean loss."""
        if self.world != 1:
            raise NotImplementedError('Eggroll.step gathers losses across ranks in the reference; this library '
                                      'runs one GPU (call population() per rank and gather the losses first)')
        losses = self.population(step, x, y, chunk=chunk)
        grads = self.update(losses, self.offsets(step), chunk=update_chunk)
        optimizer.zero_grad(set_to_none=True)
        for name, p in self.params.items():
            p.grad = grads[name]
        optimizer.step()
        return losses.mean().item()


SIGMA = 0.002   # eggroll.py:31


BLOCK_MATRIX_SUFFIXES = ('attn.c_q.weight', 'attn.c_k.weight', 'attn.c_v.weight', 'attn.c_proj.weight',
                         'mlp.c_fc.weight', 'mlp.c_proj.weight')


def block_matrix_shapes(params):
    """name -> (out, in) of the 48 block matrices (run.py:647's perturbed set), in named_parameters order."""
    return {n: tuple(p.shape) for n, p in params.items()
            if n.startswith('transformer.h.') and n.endswith(BLOCK_MATRIX_SUFFIXES)}


def orthogonal_directions(shapes, pairs, seed=SEED, rank=0, world=1, device=None, dtype=torch.float32):
    """Weight-space orthogonal perturbation directions: name -> (a [pairs, out], b [pairs, in]) of +-1.

    Each matrix's rank-1 factors are two sites of DUST.orthogonal_noise (run.py:223-238) with a one-token
    frame (b = t = 1): a at site (name, 'a') of width out, then b at site (name, 'b') of width in, matrices
    visited in `shapes` order, all of this rank's `pairs` draws in one call per site (chunk 0), so
    direction i is draw rank * pairs + i. Within a cycle of d draws the directions are exactly orthogonal
    (distinct Hadamard rows); E[a a^T] = I as for Gaussian draws, so sigma keeps its meaning."""
    od = OrthogonalDraws(seed, rank, world, device)
    out = {}
    for name, (o, i) in shapes.items():
        a = od((name, 'a'), pairs, 0, pairs, 1, 1, o, dtype=dtype).view(pairs, o)
        b = od((name, 'b'), pairs, 0, pairs, 1, 1, i, dtype=dtype).view(pairs, i)
        out[name] = (a, b)
    return out


def orthogonal_population(W, noise, x, y, sigma=SIGMA, chunk=1024, directions=None):
    """Losses of the antithetic members of orthogonal directions `noise` (orthogonal_directions): member
    2i is +sigma and 2i+1 is -sigma along direction i (eggroll.py:138-142's pairing), all scored on one
    sequence x -> y, evaluated `chunk` members at a time. directions: optional subset (int tensor) of the
    directions to evaluate; the result then holds their 2 * len(directions) members in that order."""
    dev = x.device
    dirs = torch.arange(next(iter(noise.values()))[0].shape[0], device=dev) if directions is None else \
        directions.to(dev)
    losses = []
    for start in range(0, len(dirs), chunk // 2):
        d = dirs[start:start + chunk // 2]
        sub = {k: (a[d], b[d]) for k, (a, b) in noise.items()}
        sign = _pair_signs(len(d), sigma, dev)
        losses.append(population_forward(W, sub, sign, x, y, dir_div=2))
    return torch.cat(losses)
