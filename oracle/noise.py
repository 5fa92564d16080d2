"""ORACLE (test infrastructure only): Python face of oracle/philox.c.

Restates torch-ROCm's device draws (torch: ATen/native/hip/DistributionTemplates.h:52-89, 318-348,
446-457) over rocRAND Philox4x32-10 (rocrand_philox4x32_10.h) on the CPU. Integer results are exact;
normals use the host libm (rocrand_normal.h:62-64 host branch) and match the device to a few ulp.
"""
import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / '_build' / 'liboracle_philox.so'
_lib = None


def build():
    """Compile the oracle (gcc) and its cross-check drivers into oracle/_build."""
    subprocess.run(['make', '-s', '-C', str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        u64, i64, p = ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p
        L.oracle_philox4x32.argtypes = [p, p, ctypes.c_int, p]
        L.oracle_grid_threads.argtypes = [u64, ctypes.c_uint32, ctypes.c_uint32]
        L.oracle_grid_threads.restype = u64
        L.oracle_offset_increment.argtypes = [u64, u64]
        L.oracle_offset_increment.restype = u64
        L.oracle_draw_u32.argtypes = [u64, u64, u64, p, i64, p]
        L.oracle_randint.argtypes = [u64, u64, u64, u64, i64, p, i64, p]
        L.oracle_randn.argtypes = [u64, u64, u64, p, i64, p]
        L.oracle_randn_uv.argtypes = [u64, u64, u64, p, i64, p, p, p]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def philox4x32(counter, key, rounds=10):
    c = np.ascontiguousarray(counter, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().oracle_philox4x32(_ptr(c), _ptr(k), rounds, _ptr(out))
    return out


def grid_threads(numel, cus, max_threads_per_cu):
    return int(lib().oracle_grid_threads(numel, cus, max_threads_per_cu))


def offset_increment(numel, threads):
    return int(lib().oracle_offset_increment(numel, threads))


def _idx(idx):
    return np.ascontiguousarray(idx, dtype=np.int64)


def draw_u32(seed, offset, threads, idx):
    i = _idx(idx)
    out = np.zeros(i.size, dtype=np.uint32)
    lib().oracle_draw_u32(seed, offset, threads, _ptr(i), i.size, _ptr(out))
    return out


def randint(seed, offset, threads, rng, idx, base=0):
    i = _idx(idx)
    out = np.zeros(i.size, dtype=np.int64)
    lib().oracle_randint(seed, offset, threads, rng, base, _ptr(i), i.size, _ptr(out))
    return out


def randn(seed, offset, threads, idx):
    i = _idx(idx)
    out = np.zeros(i.size, dtype=np.float32)
    lib().oracle_randn(seed, offset, threads, _ptr(i), i.size, _ptr(out))
    return out


def randn_uv(seed, offset, threads, idx):
    """Box-Muller inputs (x word, y word, takes cos) of each element."""
    i = _idx(idx)
    ux = np.zeros(i.size, dtype=np.uint32)
    vy = np.zeros(i.size, dtype=np.uint32)
    is_cos = np.zeros(i.size, dtype=np.int32)
    lib().oracle_randn_uv(seed, offset, threads, _ptr(i), i.size, _ptr(ux), _ptr(vy), _ptr(is_cos))
    return ux, vy, is_cos


class OracleGenerator:
    """torch.Generator('cuda').manual_seed(seed) offset bookkeeping on a device with `cus` compute units
    and `max_threads_per_cu` threads per unit (MI355X: 256 and 2048)."""

    def __init__(self, seed, cus=256, max_threads_per_cu=2048):
        self.seed, self.offset = int(seed), 0
        self.cus, self.max_threads = cus, max_threads_per_cu

    def take(self, numel):
        threads = grid_threads(numel, self.cus, self.max_threads)
        draw = (self.seed, self.offset, threads)
        self.offset += offset_increment(numel, threads)
        return draw

    def randint(self, low, high, n):
        seed, offset, threads = self.take(n)
        return randint(seed, offset, threads, high - low, np.arange(n), low)

    def randn(self, n, idx=None):
        seed, offset, threads = self.take(n)
        return randn(seed, offset, threads, np.arange(n) if idx is None else idx)
