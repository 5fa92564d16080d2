"""DUST pieces on the population-forward path (train/val/run.py):

  head_loss(x, weight, targets, vocab)      run.py:89-94, the fp32 head of rerun (run.py:273-278)
  coordinate_differences(raw, y, sigma)     run.py:121-137
  head_error(logits, y, vocab, sigma)       run.py:380-389
  hadamard(d, device, dtype)                run.py:143-152
  OrthogonalDraws                           run.py:218-238 (signs, orthogonal_noise)
"""
import ctypes

import torch

from . import _lib
from .noise import DeviceGenerator

F32, BF16 = torch.float32, torch.bfloat16


def head_loss(x, weight, targets, vocab):
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
    (unit inner stride), y [...] int64 -> fp32 [..., V]."""
    return head_error(raw, y, raw.shape[-1], sigma)


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
