"""ORACLE (test infrastructure only): DUST.orthogonal_noise (train/val/run.py:223-238) on the CPU.

Restates the reference's frames and draws with OracleGenerator (torch-ROCm's device randint in closed form,
oracle/noise.py) standing in for its two cuda generators (run.py:169-170: seed + 3 + 7777 * rank for the
per-draw signs, seed + 5 shared by all GPUs for the frames) and oracle.model.hadamard for run.py:143-152.
A site's frame is drawn on first use: the cycle patterns randint(0, 2, (cycles, d)) (run.py:218-221 signs,
shared) then the row offsets randint(0, d, (b, t)) (run.py:232). Draw i is row (offset + index) mod d of H
times pattern[index // d] times its own sign, index = rank * draws + chunk * n + i (run.py:235-237).
"""
import numpy as np

from .model import hadamard
from .noise import OracleGenerator


class OrthogonalDrawsOracle:
    def __init__(self, seed=0, rank=0, world=1, cus=256, max_threads_per_cu=2048):
        self.rank, self.world = rank, world
        self.generator = OracleGenerator(seed + 3 + 7777 * rank, cus, max_threads_per_cu)
        self.shared = OracleGenerator(seed + 5, cus, max_threads_per_cu)
        self.frames = {}

    def __call__(self, site, draws, chunk, n, b, t, d):
        """[n, b, t, d] float32 of +-1."""
        if site not in self.frames:
            cycles = -(-self.world * draws // d)
            patterns = self.shared.randint(0, 2, cycles * d).reshape(cycles, d) * 2 - 1
            offset = self.shared.randint(0, d, b * t).reshape(b, t)
            self.frames[site] = (patterns, offset)
        patterns, offset = self.frames[site]
        index = self.rank * draws + chunk * n + np.arange(n)
        rows = (offset[None, :, :] + index[:, None, None]) % d
        signs = self.generator.randint(0, 2, n * b * t).reshape(n, b, t, 1) * 2 - 1
        H = hadamard(d).numpy()
        return (H[rows] * patterns[index // d][:, None, None, :] * signs).astype(np.float32)


def orthogonal_directions(shapes, pairs, seed=0, rank=0, world=1):
    """oracle twin of noise_amd.eggroll.orthogonal_directions: name -> (a [pairs, out], b [pairs, in])."""
    od = OrthogonalDrawsOracle(seed, rank, world)
    out = {}
    for name, (o, i) in shapes.items():
        a = od((name, 'a'), pairs, 0, pairs, 1, 1, o).reshape(pairs, o)
        b = od((name, 'b'), pairs, 0, pairs, 1, 1, i).reshape(pairs, i)
        out[name] = (a, b)
    return out
