"""The fixed model on libnoise_amd, with utils/model.py's names and call signatures.

attention(q, k, v, window)  replaces utils/model.py:24-31 (flex_attention over the window block mask).
GPTConfig / GPT / make_model hold the same parameters under the same state-dict names as
utils/model.py:34-175 and train/val/eggroll.py:38-53, so weights load strictly either way.
"""
import math
from dataclasses import dataclass

import torch
from torch import nn

from . import _lib
from ._lib import ATTN_QK_NORMED, ATTN_V_TRANSPOSED

BF16 = torch.bfloat16
N_LAYER, N_HEAD, HEAD_DIM, N_EMBD, VOCAB, SEQ = 8, 8, 64, 512, 4096, 2048


@dataclass
class GPTConfig:
    """utils/model.py:34-43."""
    sequence_len: int = 2048
    vocab_size: int = 4096
    n_layer: int = 8
    n_head: int = 8
    n_kv_head: int = 8
    n_embd: int = 512
    window_pattern: str = 'SSSL'


def has_ve(layer_idx, n_layer=N_LAYER):
    """Value embeddings on every other block, counting back from the last (model.py:50-52)."""
    return layer_idx % 2 == (n_layer - 1) % 2


def window_sizes(n_layer=N_LAYER, sequence_len=SEQ, pattern='SSSL'):
    """Left window per block (model.py:185-191): 'S' = half the sequence, 'L' = all of it; last is L."""
    pattern = pattern.upper()
    sizes = [sequence_len if pattern[i % len(pattern)] == 'L' else sequence_len // 2 for i in range(n_layer)]
    sizes[-1] = sequence_len
    return sizes


def rotary_tables(length, head_dim=HEAD_DIM, base=10000):
    """cos, sin [length, head_dim/2] fp32 holding the bf16 tables of model.py:177-183 (fp32 angles
    t * base^(-2i/d), cos/sin rounded to bf16)."""
    inv_freq = 1.0 / base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)
    angles = torch.outer(torch.arange(length, dtype=torch.float32), inv_freq)
    return angles.cos().bfloat16().float(), angles.sin().bfloat16().float()


class _Attn(nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        d, kv = cfg.n_embd, cfg.n_kv_head * (cfg.n_embd // cfg.n_head)
        self.c_q = nn.Linear(d, d, bias=False)
        self.c_k = nn.Linear(d, kv, bias=False)
        self.c_v = nn.Linear(d, kv, bias=False)
        self.c_proj = nn.Linear(d, d, bias=False)
        self.ve_gate = nn.Linear(32, cfg.n_kv_head, bias=False) if has_ve(layer_idx, cfg.n_layer) else None


class _MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.c_fc = nn.Linear(cfg.n_embd, 4 * cfg.n_embd, bias=False)
        self.c_proj = nn.Linear(4 * cfg.n_embd, cfg.n_embd, bias=False)


class _Block(nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        self.attn = _Attn(cfg, layer_idx)
        self.mlp = _MLP(cfg)


class GPT(nn.Module):
    """Parameter container of the fixed model (model.py:122-147), same names and shapes. The forward
    lives in population_loss / gpt_loss (noise_amd.eggroll)."""

    def __init__(self, config, pad_vocab_size_to=64):
        super().__init__()
        self.config = config
        self.window_sizes = [(w, 0) for w in window_sizes(config.n_layer, config.sequence_len, config.window_pattern)]
        vocab = -(-config.vocab_size // pad_vocab_size_to) * pad_vocab_size_to
        self.transformer = nn.ModuleDict({
            'wte': nn.Embedding(vocab, config.n_embd),
            'h': nn.ModuleList([_Block(config, i) for i in range(config.n_layer)]),
        })
        self.lm_head = nn.Linear(config.n_embd, vocab, bias=False)
        self.resid_lambdas = nn.Parameter(torch.ones(config.n_layer))
        self.x0_lambdas = nn.Parameter(torch.zeros(config.n_layer))
        kv = config.n_kv_head * (config.n_embd // config.n_head)
        self.value_embeds = nn.ModuleDict({str(i): nn.Embedding(vocab, kv)
                                           for i in range(config.n_layer) if has_ve(i, config.n_layer)})

    @torch.no_grad()
    def init_weights(self):
        """model.py:149-175's draws, in its order, on this module's device generator."""
        s = 3 ** 0.5 * self.config.n_embd ** -0.5
        nn.init.normal_(self.transformer.wte.weight, mean=0.0, std=1.0)
        nn.init.normal_(self.lm_head.weight, mean=0.0, std=0.001)
        for blk in self.transformer.h:
            for lin in (blk.attn.c_q, blk.attn.c_k, blk.attn.c_v):
                nn.init.uniform_(lin.weight, -s, s)
            nn.init.zeros_(blk.attn.c_proj.weight)
            nn.init.uniform_(blk.mlp.c_fc.weight, -s, s)
            nn.init.zeros_(blk.mlp.c_proj.weight)
        self.resid_lambdas.fill_(1.0)
        self.x0_lambdas.fill_(0.1)
        for emb in self.value_embeds.values():
            nn.init.uniform_(emb.weight, -s, s)
        for blk in self.transformer.h:
            if blk.attn.ve_gate is not None:
                nn.init.zeros_(blk.attn.ve_gate.weight)
        if self.transformer.wte.weight.device.type == 'cuda':
            # on a GPU the token and value embeddings are stored in bf16 (model.py:171-175)
            for emb in self._embeddings():
                emb.to(dtype=BF16)

    def _embeddings(self):
        return [self.transformer.wte, *self.value_embeds.values()]


def make_model(device='cpu', seed=0, fp32_embeddings=True):
    """The training scripts' model: seeded init_weights, then the output projections (every '*c_proj'
    Linear, in module order) re-drawn U(+-1.5 sqrt(3 / fan_in)). Built on `device` with that device's
    generator. fp32_embeddings=True is EGGROLL's make_model (eggroll.py:38-53): the embeddings are cast to
    fp32 for the ES updates, so on a GPU they hold init_weights' bf16-rounded values; False is DUST's
    (run.py:545-557), which keeps the GPU's bf16 storage. On the CPU the embeddings are fp32 either way."""
    torch.manual_seed(seed)
    with torch.device('meta'):
        model = GPT(GPTConfig())
    model.to_empty(device=device)
    model.init_weights()
    with torch.no_grad():
        for name, module in model.named_modules():
            if 'c_proj' in name and isinstance(module, nn.Linear):
                bound = 1.5 * (3 / module.weight.shape[1]) ** 0.5
                nn.init.uniform_(module.weight, -bound, bound)
    if fp32_embeddings:
        for emb in model._embeddings():
            emb.float()
    return model.requires_grad_(False)


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
    # V in its own layout: lengths in whole 256-query tiles run the ring kernel, which reads V^T fragments
    # from natural V tiles with transposing LDS reads; other lengths run the general kernel
    _lib.call('noise_attention_fwd', qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), out.data_ptr(), B, H, T, D,
              qb.stride(0), qb.stride(2), qb.stride(1), kb.stride(0), kb.stride(2), kb.stride(1),
              vb.stride(0), vb.stride(2), vb.stride(1), 0, out.stride(0), out.stride(2), out.stride(1),
              int(window), 1.0 / math.sqrt(D), None, 0, 1, None, _lib.stream_ptr(q.device))
    return out if q.dtype == BF16 else out.to(q.dtype)


def attention_raw(q, k, v, out, window, v_transposed=False, dot_vec=None, dot_div=1, dot_out=None,
                  qk_normed=False):
    """Kernel-level entry used by the population path: q, k, out [B, H, T, D] or [B, T, H, D] views,
    v [B, H, D, T] when v_transposed; optional fused per-head dot with dot_vec [B / dot_div, H*D].
    qk_normed promises q and k rows of RMS <= 1 (RMSNorm outputs): the softmax then needs no running max."""
    B, T, H, D = out.shape
    if v_transposed:
        vs = (v.stride(0), v.stride(1), v.stride(2))  # v viewed as [B, H, D, T]
    else:
        vs = (v.stride(0), v.stride(2), v.stride(1))
    _lib.call('noise_attention_fwd', q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, T, D,
              q.stride(0), q.stride(2), q.stride(1), k.stride(0), k.stride(2), k.stride(1), *vs,
              (ATTN_V_TRANSPOSED if v_transposed else 0) | (ATTN_QK_NORMED if qk_normed else 0),
              out.stride(0), out.stride(2), out.stride(1), int(window),
              1.0 / math.sqrt(D), _lib.ptr(dot_vec), 0 if dot_vec is None else dot_vec.stride(0), dot_div,
              _lib.ptr(dot_out), _lib.stream_ptr(out.device))
    return out
