"""The fixed model's ops on libnoise_amd, with utils/model.py's call signatures.

attention(q, k, v, window)  replaces utils/model.py:24-31 (flex_attention over the window block mask).
"""
import math

import torch

from . import _lib

BF16 = torch.bfloat16


def _operand(t):
    """bf16 view usable by the kernels: contiguous head dim, 8-element-aligned strides, 16 B base."""
    if t.dtype != BF16:
        t = t.to(BF16)
    if (t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16):
        t = t.contiguous()
    return t


def attention(q, k, v, window):
    """Causal attention with a left window; tensors [batch, token, head, dim] (model.py:24-31).

    A query at position s sees keys s - window .. s. Computed in bf16 with fp32 accumulation; the output
    has q's dtype, shape [B, T, H, D] (contiguous)."""
    if q.dim() != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f'attention: q, k, v must be [B, T, H, D] of one shape, got {q.shape}, {k.shape}, {v.shape}')
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError('attention: tensors must be on a GPU')
    B, T, H, D = q.shape
    qb, kb, vb = _operand(q), _operand(k), _operand(v)
    out = torch.empty(B, T, H, D, dtype=BF16, device=q.device)
    _lib.call('noise_attention_fwd', qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), out.data_ptr(), B, H, T, D,
              qb.stride(0), qb.stride(2), qb.stride(1), kb.stride(0), kb.stride(2), kb.stride(1),
              vb.stride(0), vb.stride(2), vb.stride(1), 0, out.stride(0), out.stride(2), out.stride(1),
              int(window), 1.0 / math.sqrt(D), None, 0, 1, None, _lib.stream_ptr(q.device))
    return out if q.dtype == BF16 else out.to(q.dtype)


def attention_raw(q, k, v, out, window, v_transposed=False, dot_vec=None, dot_div=1, dot_out=None):
    """Kernel-level entry used by the population path: q, k, out [B, H, T, D] or [B, T, H, D] views,
    v [B, H, D, T] when v_transposed; optional fused per-head dot with dot_vec [B / dot_div, H*D]."""
    B, T, H, D = out.shape
    if v_transposed:
        vs = (v.stride(0), v.stride(1), v.stride(2))  # v viewed as [B, H, D, T]
    else:
        vs = (v.stride(0), v.stride(2), v.stride(1))
    _lib.call('noise_attention_fwd', q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, T, D,
              q.stride(0), q.stride(2), q.stride(1), k.stride(0), k.stride(2), k.stride(1), *vs,
              1 if v_transposed else 0, out.stride(0), out.stride(2), out.stride(1), int(window),
              1.0 / math.sqrt(D), _lib.ptr(dot_vec), 0 if dot_vec is None else dot_vec.stride(0), dot_div,
              _lib.ptr(dot_out), _lib.stream_ptr(out.device))
    return out
