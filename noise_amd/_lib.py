"""Loader of libnoise_amd.so, the C ABI declared in include/noise_amd.h.

There is no fallback: if the library is missing or does not load, every op raises.
"""
import ctypes
from pathlib import Path

import torch

from .abi import (SIGNATURES, LINEAR_AUTOCAST, ROUNDING_FUSED, ROUNDING_EAGER, ATTN_V_TRANSPOSED,  # noqa: F401
                  ATTN_QK_NORMED, View, Rank1, Population, UpdateParam, SliceGroups, SLICE_GROUPS_MAX, BlockJitter, bind)

# the in-tree build (noise_amd/build.py); no other library is ever loaded
LIB_PATH = Path(__file__).resolve().with_name('libnoise_amd.so')

_lib = None


def lib():
    """The loaded library (raises RuntimeError when it is not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f'{LIB_PATH} is not built: run noise_amd.build.build() (hipcc, gfx950)')
        _lib = bind(ctypes.CDLL(str(LIB_PATH)))
    return _lib


def call(name, *args):
    """Call entry point `name`; raise RuntimeError with the library's message on a non-zero status."""
    status = getattr(lib(), name)(*args)
    if status != 0:
        msg = lib().noise_last_error().decode(errors='replace')
        kind = 'invalid argument' if status < 0 else f'HIP error {status}'
        raise RuntimeError(f'{name}: {kind}: {msg}')
    return status


def stream_ptr(device=None):
    """hipStream_t of torch's current stream on `device`, as an integer for ctypes."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t):
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()
