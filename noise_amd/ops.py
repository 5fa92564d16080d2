"""torch.library registrations of the drop-ins, so the reference's torch.compile'd callers trace through them
without graph breaks: population_loss is compiled at eggroll.py:115, head_loss, block_forward and
coordinate_differences at run.py:89, 102, 120, and attention sits inside the compiled forwards
(utils/model.py:14, 95). Fake implementations give output shapes and dtypes; the real ones call libnoise_amd.

  torch.ops.noise_amd.attention(q, k, v, window)                      utils/model.py:24
  torch.ops.noise_amd.lowrank(x, weight, a, b, sign, dir_div)         eggroll.py:56
  torch.ops.noise_amd.lowrank_embed(weight, a, b, idx, sign, dir_div) eggroll.py:61
  torch.ops.noise_amd.population_loss(names, params, noise_a, noise_b, sign, idx, targets, n_layer,
                                      dir_div, fp32_head)             eggroll.py:66
  torch.ops.noise_amd.head_loss(x, weight, targets, vocab)            run.py:90
  torch.ops.noise_amd.block_forward(x, w, ve, cos, sin, window, o, attn, fc, mlp)   run.py:103
  torch.ops.noise_amd.coordinate_differences(raw, y, sigma)           run.py:121

Ops take flat tensor lists where the reference passes dicts: population_loss's parameter and noise dicts
become one list per field in the order of `names` (newline-separated parameter names), with the noise of
a 1-D parameter (the mixing scalars' eps) in noise_a and None in noise_b; block_forward's weight dict is
the list (q, k, v, gate or None, proj, fc, out). The reference-signature wrappers that pack them are
noise_amd.eggroll.population_loss and noise_amd.dust.head_loss / block_forward / coordinate_differences.
"""
from typing import List, Optional

import torch
from torch import Tensor
from torch.library import custom_op

from . import dust, eggroll, model

BLOCK_WEIGHTS = ('q', 'k', 'v', 'gate', 'proj', 'fc', 'out')


@custom_op('noise_amd::attention', mutates_args=())
def attention(q: Tensor, k: Tensor, v: Tensor, window: int) -> Tensor:
    return model.attention(q, k, v, window)


@attention.register_fake
def _attention_fake(q, k, v, window):
    return q.new_empty(q.shape)


@custom_op('noise_amd::lowrank', mutates_args=())
def lowrank(x: Tensor, weight: Tensor, a: Tensor, b: Tensor, sign: Tensor, dir_div: int) -> Tensor:
    return eggroll.lowrank_eager(x, weight, a, b, sign, dir_div=dir_div)


@lowrank.register_fake
def _lowrank_fake(x, weight, a, b, sign, dir_div):
    return x.new_empty((x.shape[0], x.shape[1], weight.shape[0]), dtype=torch.float32)


@custom_op('noise_amd::lowrank_embed', mutates_args=())
def lowrank_embed(weight: Tensor, a: Tensor, b: Tensor, idx: Tensor, sign: Tensor, dir_div: int) -> Tensor:
    return eggroll.lowrank_embed_eager(weight, a, b, idx, sign, dir_div=dir_div)


@lowrank_embed.register_fake
def _lowrank_embed_fake(weight, a, b, idx, sign, dir_div):
    return weight.new_empty((sign.shape[0], idx.shape[0], weight.shape[1]), dtype=torch.float32)


@custom_op('noise_amd::population_loss', mutates_args=())
def population_loss(names: str, params: List[Tensor], noise_a: List[Optional[Tensor]],
                    noise_b: List[Optional[Tensor]], sign: Tensor, idx: Tensor, targets: Tensor, n_layer: int,
                    dir_div: int, fp32_head: bool) -> Tensor:
    keys = names.split('\n')
    if not (len(keys) == len(params) == len(noise_a) == len(noise_b)):
        raise ValueError(f'population_loss: {len(keys)} names for {len(params)} parameters, '
                         f'{len(noise_a)} / {len(noise_b)} noise entries')
    p = dict(zip(keys, params))
    noise = {}
    for k, a, b in zip(keys, noise_a, noise_b):
        if a is not None:
            noise[k] = a if b is None else (a, b)
    return eggroll.population_loss_eager(p, noise, sign, idx, targets, n_layer=n_layer, dir_div=dir_div,
                                         fp32_head=fp32_head)


@population_loss.register_fake
def _population_loss_fake(names, params, noise_a, noise_b, sign, idx, targets, n_layer, dir_div, fp32_head):
    return sign.new_empty((sign.shape[0],), dtype=torch.float32)


@custom_op('noise_amd::head_loss', mutates_args=())
def head_loss(x: Tensor, weight: Tensor, targets: Tensor, vocab: int) -> Tensor:
    return dust.head_loss_eager(x, weight, targets, vocab)


@head_loss.register_fake
def _head_loss_fake(x, weight, targets, vocab):
    return x.new_empty((targets.numel(),), dtype=torch.float32)


@custom_op('noise_amd::block_forward', mutates_args=())
def block_forward(x: Tensor, w: List[Optional[Tensor]], ve: Optional[Tensor], cos: Tensor, sin: Tensor, window: int,
                  o: Optional[Tensor], attn: Optional[Tensor], fc: Optional[Tensor],
                  mlp: Optional[Tensor]) -> Tensor:
    if len(w) != len(BLOCK_WEIGHTS):
        raise ValueError(f'block_forward: expected the weights {BLOCK_WEIGHTS}, got {len(w)} tensors')
    return dust.block_forward_eager(x, dict(zip(BLOCK_WEIGHTS, w)), ve, cos, sin, window, o, attn, fc, mlp)


@block_forward.register_fake
def _block_forward_fake(x, w, ve, cos, sin, window, o, attn, fc, mlp):
    return x.new_empty(x.shape, dtype=torch.float32)


@custom_op('noise_amd::coordinate_differences', mutates_args=())
def coordinate_differences(raw: Tensor, y: Tensor, sigma: float) -> Tensor:
    return dust.head_error(raw, y, raw.shape[-1], sigma)


@coordinate_differences.register_fake
def _coordinate_differences_fake(raw, y, sigma):
    return raw.new_empty(raw.shape, dtype=torch.float32)
