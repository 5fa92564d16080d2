"""The speedrun's score on libnoise_amd: mean next-token cross-entropy of a state dict on the fixed
validation split (utils/eval.py).

  load_model(state_dict, device)                 eval.py:24-31
  evaluate(state_dict, data_dir, batch_size)     eval.py:34-53
  score_rows(weights, rows, batch_size)          the loop of eval.py:43-48 over given rows

The scorer's forward is the population forward with one validation row per member and no noise: every
row is a member with its own tokens (population_forward with [members, T] token ids). It follows the
reference scorer's dtypes: the token and value embeddings are held in bfloat16 (model.py:170-174 casts
their storage when the model lives on the GPU, so load_state_dict rounds them), and the forward runs
eagerly under autocast, so every elementwise op rounds its result to bfloat16 and the residual stream is
bfloat16 (the kernels' ROUNDING_EAGER mode), where the compiled training forward keeps it in fp32.
"""
from pathlib import Path

import torch
from torch import distributed as dist

from . import _lib
from .eggroll import F32, Weights, _Buffers, population_forward
from .model import GPT, GPTConfig
from .prepare_data import VAL_ROWS, load_rows

BF16_STORAGE = ('transformer.wte.weight', 'value_embeds.')


def _expected_shapes():
    with torch.device('meta'):
        model = GPT(GPTConfig())
    return {k: tuple(v.shape) for k, v in model.state_dict().items()}


def check_state_dict(state_dict):
    """load_state_dict(strict=True)'s checks (eval.py:31): the fixed architecture's tensors, no more, no
    fewer, same shapes. Raises RuntimeError naming what differs."""
    expected = _expected_shapes()
    missing = sorted(set(expected) - set(state_dict))
    unexpected = sorted(set(state_dict) - set(expected))
    reshaped = sorted(k for k in set(expected) & set(state_dict) if tuple(state_dict[k].shape) != expected[k])
    if missing or unexpected or reshaped:
        parts = []
        if missing:
            parts.append(f'missing keys {missing}')
        if unexpected:
            parts.append(f'unexpected keys {unexpected}')
        if reshaped:
            parts.append('size mismatch for ' + ', '.join(
                f'{k}: {tuple(state_dict[k].shape)} vs {expected[k]}' for k in reshaped))
        raise RuntimeError('Error(s) in loading state_dict for GPT: ' + '; '.join(parts))


def load_model(state_dict, device):
    """The fixed architecture with these weights, in the layouts the kernels read (Weights). A missing,
    extra or reshaped tensor is an error. Token and value embeddings are rounded to bfloat16, as the
    reference's GPU model stores them."""
    check_state_dict(state_dict)
    dev = torch.device(device)
    p = {}
    for k, v in state_dict.items():
        v = v.detach().to(dev)
        if k.startswith(BF16_STORAGE):
            v = v.to(torch.bfloat16)
        p[k] = v
    return Weights(p, device=dev)


@torch.no_grad()
def score_rows(weights, rows, batch_size=16):
    """(summed loss, predictions) over token rows [n, T + 1]: row r predicts rows[r, 1:] from
    rows[r, :-1], ignore index -1 contributing 0 but counted, as cross_entropy(reduction='sum') and
    eval.py:47-48 do. The sum is accumulated in float64 on the device, batch by batch."""
    if rows.dim() != 2 or rows.shape[1] < 2:
        raise ValueError('rows must be [n, T + 1]')
    dev = weights.device
    T = rows.shape[1] - 1
    total = torch.zeros((), dtype=torch.float64, device=dev)
    buffers = {}
    for batch in rows.split(batch_size):
        batch = batch.to(dev)
        m = batch.shape[0]
        if m not in buffers:
            buffers[m] = _Buffers(m, T, dev, weights.fp32_head, True, eager=True)
        sign = torch.zeros(m, dtype=F32, device=dev)
        loss = population_forward(weights, {}, sign, batch[:, :-1].contiguous(), batch[:, 1:].contiguous(),
                                  buffers=buffers[m], per_token=True, rounding=_lib.ROUNDING_EAGER)
        total += loss.sum(dtype=torch.float64)
    return total, rows.shape[0] * T


@torch.no_grad()
def evaluate(state_dict, data_dir='data', batch_size=16):
    """Mean loss over all 1,114,112 validation predictions of data_dir/val.pt. Under torch.distributed
    the rows are split rank::world and the sums all-reduced (float64), as eval.py:41-50 does."""
    rank, world = (dist.get_rank(), dist.get_world_size()) if dist.is_initialized() else (0, 1)
    device = torch.device('cuda', torch.cuda.current_device())
    weights = load_model(state_dict, device)
    rows = load_rows(Path(data_dir) / 'val.pt', VAL_ROWS)[rank::world]
    loss, count = score_rows(weights, rows, batch_size)
    total = torch.stack([loss, torch.tensor(float(count), dtype=torch.float64, device=device)])
    if world > 1:
        if dist.get_backend() == 'gloo':
            total = total.cpu()
        dist.all_reduce(total)
    value = (total[0] / total[1]).item()
    if value != value:
        raise FloatingPointError('Non-finite validation loss')
    return value
