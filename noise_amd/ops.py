"""torch.library registrations of the tensor-only ops, so torch.compile'd callers (the reference compiles
population_loss, eggroll.py:115, and head_loss / block_forward, run.py:89-120) trace through them without
graph breaks. Fake implementations give output shapes and dtypes; the real ones call libnoise_amd.

  torch.ops.noise_amd.attention(q, k, v, window)            utils/model.py:24
  torch.ops.noise_amd.lowrank(x, weight, a, b, sign, dir_div) eggroll.py:56
  torch.ops.noise_amd.head_loss(x, weight, targets, vocab)    run.py:90
"""
import torch
from torch.library import custom_op

from . import dust, eggroll, model


@custom_op('noise_amd::attention', mutates_args=())
def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int) -> torch.Tensor:
    return model.attention(q, k, v, window)


@attention.register_fake
def _attention_fake(q, k, v, window):
    return q.new_empty(q.shape)


@custom_op('noise_amd::lowrank', mutates_args=())
def lowrank(x: torch.Tensor, weight: torch.Tensor, a: torch.Tensor, b: torch.Tensor, sign: torch.Tensor,
            dir_div: int) -> torch.Tensor:
    return eggroll.lowrank(x, weight, a, b, sign, dir_div=dir_div)


@lowrank.register_fake
def _lowrank_fake(x, weight, a, b, sign, dir_div):
    return x.new_empty((x.shape[0], x.shape[1], weight.shape[0]), dtype=torch.float32)


@custom_op('noise_amd::head_loss', mutates_args=())
def head_loss(x: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor, vocab: int) -> torch.Tensor:
    return dust.head_loss(x, weight, targets, vocab)


@head_loss.register_fake
def _head_loss_fake(x, weight, targets, vocab):
    return x.new_empty((targets.numel(),), dtype=torch.float32)
