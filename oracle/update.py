"""ORACLE (test infrastructure only): EGGROLL's update reassembly on the CPU.

Restates train/val/eggroll.py:151-163 (Eggroll.step after the losses are gathered):

    fitness = losses[1::2] - losses[0::2]                        # fp32, as the reference
    fitness = fitness / (fitness.std() + 1e-8)                   # unbiased std (torch's default)
    weight = zeros(pairs).index_add_(0, arange(len(fitness)) % pairs, fitness)
    gradients[name] -= (w[:, None] * a).t() @ b                  # 2-D parameters, eggroll.py:159-160
    gradients[name] -= w @ eps                                   # 1-D parameters, eggroll.py:161-162
    p.grad = gradients[name] / len(fitness)                      # eggroll.py:165

with a = buffer[off_d : off_d + rows], b = buffer[off_d + rows : off_d + rows + cols] the direction's slices
of the noise buffer (eggroll.py:122-128), here drawn from oracle.noise.randn at those indices. Sums run in
float64 (the reference's TF32/fp32 products are within tolerance of it).
"""
import numpy as np

from . import noise as onoise


def fitness_weights(losses, pairs):
    """eggroll.py:151-154: the per-direction weight [pairs] (float64) of one update's losses [members]."""
    losses = np.asarray(losses, dtype=np.float32)
    fitness = losses[1::2] - losses[0::2]
    std = np.float32(fitness.astype(np.float64).std(ddof=1))
    z = (fitness / (std + np.float32(1e-8))).astype(np.float64)
    weight = np.zeros(pairs, dtype=np.float64)
    np.add.at(weight, np.arange(len(fitness)) % pairs, z)
    return weight


def direction_slices(offsets, width, draw):
    """[pairs, width] float64: row d = elements offsets[d] .. offsets[d] + width of the normal draw
    (seed, offset, threads) (eggroll.py:126)."""
    seed, offset, threads = draw
    off = np.asarray(offsets, dtype=np.int64)
    idx = off[:, None] + np.arange(width, dtype=np.int64)[None, :]
    return onoise.randn(seed, offset, threads, idx.ravel()).reshape(len(off), width).astype(np.float64)


def gradients_from_weights(weight, offsets, shapes, draw, scale):
    """name -> scale * sum_d weight[d] a_d b_d^T (2-D) or scale * sum_d weight[d] a_d (1-D), float64."""
    weight = np.asarray(weight, dtype=np.float64)
    out = {}
    for name, shape in shapes.items():
        rows = direction_slices(offsets[name], int(sum(shape)), draw)
        if len(shape) == 2:
            a, b = rows[:, :shape[0]], rows[:, shape[0]:]
            out[name] = scale * ((weight[:, None] * a).T @ b)
        else:
            out[name] = scale * (weight @ rows)
    return out


def update_gradients(losses, pairs, offsets, shapes, draw):
    """The reference's p.grad for every parameter of `shapes` (eggroll.py:151-165)."""
    weight = fitness_weights(losses, pairs)
    fitness_count = len(np.asarray(losses)) // 2
    return gradients_from_weights(weight, offsets, shapes, draw, -1.0 / fitness_count)
