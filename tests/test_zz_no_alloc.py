"""noise_dust_block_static: DUST's block_forward (run.py:102-117) over the library's static scratch array, with
no allocation (collected last: it leaves the static array of the GPU in use). Checked bit for bit against noise_dust_block with a caller workspace (the same kernels), on two
calls in a row -- the second smaller, reusing the scratch the first one left -- and its size limit rejected on
the host."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def _fn(lib, name, argtypes, restype=ctypes.c_int):
    f = getattr(lib, name)
    f.argtypes, f.restype = argtypes, restype
    return f


def _inputs(S, T, with_ve, seed):
    from noise_amd.model import make_model, rotary_tables
    P = {k: v.to(DEV) for k, v in make_model('cpu', 0).state_dict().items()}
    pre = 'transformer.h.1.' if with_ve else 'transformer.h.0.'
    g = torch.Generator().manual_seed(seed)
    bf = lambda n: P[pre + n].bfloat16().contiguous()
    gate = (torch.randn(8, 32, generator=g) * 0.3).bfloat16().float().to(DEV) if with_ve else None
    w = [bf('attn.c_q.weight'), bf('attn.c_k.weight'), bf('attn.c_v.weight'), gate, bf('attn.c_proj.weight'),
         bf('mlp.c_fc.weight'), bf('mlp.c_proj.weight')]
    x = torch.randn(S, T, 512, generator=g).to(DEV)
    ve = torch.randn(S, T, 512, generator=g).bfloat16().to(DEV) if with_ve else None
    jit_fc = (torch.randn(S, T, 2048, generator=g) * 0.05).bfloat16().to(DEV)
    jit_o = (torch.randn(S, T, 512, generator=g) * 0.05).bfloat16().to(DEV)
    cos, sin = (t.bfloat16().contiguous().to(DEV) for t in rotary_tables(T))
    return x, w, ve, cos, sin, jit_o, jit_fc


def _run(lib, static, S, T, with_ve, seed, window):
    from noise_amd import _lib
    x, w, ve, cos, sin, jit_o, jit_fc = _inputs(S, T, with_ve, seed)
    out = torch.full((S, T, 512), float('nan'), device=DEV)
    wp = (ctypes.c_void_p * 7)(*[None if t is None else t.data_ptr() for t in w])
    p = ctypes.c_void_p
    stream = _lib.stream_ptr(DEV)
    common = [x.data_ptr(), out.data_ptr(), S, T, wp, _lib.ptr(ve), cos.data_ptr(), sin.data_ptr(), window,
              jit_o.data_ptr(), None, jit_fc.data_ptr(), None]
    types = [p, p, ctypes.c_int64, ctypes.c_int64, p, p, p, p, ctypes.c_int64, p, p, p, p]
    if static:
        f = _fn(lib, 'noise_dust_block_static', types + [p])
        st = f(*common, stream)
    else:
        need = _fn(lib, 'noise_dust_block_workspace_bytes', [ctypes.c_int64, ctypes.c_int64, ctypes.c_int],
                   ctypes.c_int64)(S, T, 1 if with_ve else 0)
        work = torch.empty(need, dtype=torch.uint8, device=DEV)
        f = _fn(lib, 'noise_dust_block', types + [p, ctypes.c_int64, p])
        st = f(*common, work.data_ptr(), need, stream)
    assert st == 0, lib.noise_last_error().decode()
    torch.cuda.synchronize()
    return out


def test_static_matches_workspace_entry_two_calls():
    from noise_amd import _lib
    lib = _lib.lib()
    # first call: 2 sequences x 1024 tokens with value embeddings; second: 1 x 512 without (smaller)
    for S, T, with_ve, seed, window in ((2, 1024, True, 1, 512), (1, 512, False, 2, 512)):
        print(f'noise_dust_block_static: {S} x {T} tokens, value embeddings {with_ve}', flush=True)
        got = _run(lib, True, S, T, with_ve, seed, window)
        ref = _run(lib, False, S, T, with_ve, seed, window)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref)


def test_static_rejects_inputs_beyond_the_scratch():
    """64 sequences x 2048 tokens need more scratch than the static array holds: rejected on the host before any
    launch. Every pointer is a real device buffer of the full shape (inputs, output, value rows, weights, rotary
    tables), so only the scratch size is at stake in this call."""
    from noise_amd import _lib
    lib = _lib.lib()
    S, T = 64, 2048
    cap = _fn(lib, 'noise_dust_block_static_max_bytes', [], ctypes.c_int64)()
    need = _fn(lib, 'noise_dust_block_workspace_bytes', [ctypes.c_int64, ctypes.c_int64, ctypes.c_int],
               ctypes.c_int64)(S, T, 1)
    assert need > cap
    _, w, _, cos, sin, _, _ = _inputs(1, T, True, 3)
    x = torch.zeros(S, T, 512, device=DEV)
    out = torch.full((S, T, 512), float('nan'), device=DEV)
    ve = torch.zeros(S, T, 512, dtype=torch.bfloat16, device=DEV)
    p = ctypes.c_void_p
    f = _fn(lib, 'noise_dust_block_static', [p, p, ctypes.c_int64, ctypes.c_int64, p, p, p, p, ctypes.c_int64, p, p,
                                              p, p, p])
    wp = (ctypes.c_void_p * 7)(*[t.data_ptr() for t in w])
    st = f(x.data_ptr(), out.data_ptr(), S, T, wp, ve.data_ptr(), cos.data_ptr(), sin.data_ptr(), 1024, None, None,
           None, None, _lib.stream_ptr(DEV))
    assert st == -1 and 'static array holds' in lib.noise_last_error().decode()
    torch.cuda.synchronize()
    assert torch.isnan(out).all(), 'a rejected call must not have launched'
