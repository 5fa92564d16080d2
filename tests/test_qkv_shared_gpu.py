"""noise_pop_qkv_shared (block 0 of the population, eggroll.py:81-90 with an input every member shares)
against noise_pop_qkv on the same inputs, through the C ABI.

The shared path computes base = x [c_q; c_k; c_v]^T once (noise_pop_linear, the same K loop and
accumulation order as noise_pop_qkv's) and adds each member's rank-1 term before rotary and norm, so the
two agree to the bf16 rounding of the outputs: every element within one bf16 ulp of its magnitude and
almost all bit-equal. The population tests cover the path end to end against the oracle.
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def _run(m, T, dirs, perturbed, seed):
    from noise_amd import _lib
    from noise_amd.model import rotary_tables
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, 512, generator=g).bfloat16().to(DEV)
    ws = [(torch.randn(512, 512, generator=g) * 0.04).bfloat16().to(DEV) for _ in range(3)]
    a = [torch.randn(dirs, 512, generator=g).to(DEV) for _ in range(3)]
    dots = torch.randn(m * T, 3, generator=g).to(DEV)
    sign = (torch.tensor([0.05, -0.05]).repeat(m // 2)).to(DEV)
    cos, sin = (t.bfloat16().to(DEV).contiguous() for t in rotary_tables(T))
    pop = _lib.Population(m, T, sign.data_ptr(), m // dirs, _lib.ROUNDING_FUSED)
    r1 = (_lib.Rank1 * 3)()
    for i in range(3):
        r1[i] = _lib.Rank1(a[i].data_ptr() if perturbed else None, a[i].data_ptr(), a[i].stride(0), a[i].stride(0))
    wp = (ctypes.c_void_p * 3)(*(w.data_ptr() for w in ws))
    stream = _lib.stream_ptr(DEV)
    outs = []
    for shared in (False, True):
        qkv = torch.full((3, m, 8, T, 64), float('nan'), dtype=torch.bfloat16, device=DEV)
        op = (ctypes.c_void_p * 3)(*(qkv[i].data_ptr() for i in range(3)))
        if shared:
            base = torch.empty(T, 1536, device=DEV)
            one = _lib.Population(1, T, None, 1, _lib.ROUNDING_FUSED)
            for i in range(3):
                _lib.call('noise_pop_linear', ctypes.byref(one), _lib.View(x.data_ptr(), 0, 512), ws[i].data_ptr(),
                          512, 512, None, None, base.data_ptr() + 4 * 512 * i, 1, T * 1536, 1536, stream)
            _lib.call('noise_pop_qkv_shared', ctypes.byref(pop), base.data_ptr(), r1, dots.data_ptr(), cos.data_ptr(),
                      sin.data_ptr(), op, stream)
        else:
            _lib.call('noise_pop_qkv', ctypes.byref(pop), _lib.View(x.data_ptr(), 0, 512), wp, r1, dots.data_ptr(),
                      cos.data_ptr(), sin.data_ptr(), None, 0, None, 0, None, None, op, stream)
        torch.cuda.synchronize()
        outs.append(qkv.float().cpu())
    return outs


@pytest.mark.parametrize('perturbed', [False, True])
def test_shared_matches_per_member(perturbed):
    print(f'qkv_shared: 8 members x 512 tokens, perturbed={perturbed}', flush=True)
    ref, got = _run(8, 512, 4, perturbed, 3)
    assert torch.isfinite(got).all()
    ulp = ref.abs() * 2.0 ** -7 + 1e-6
    assert ((got - ref).abs() <= ulp).all()
    assert (got != ref).float().mean().item() < 0.01
    # members differ when perturbed (the rank-1 terms reach the outputs), not otherwise
    assert torch.equal(got[:, 0], got[:, 1]) != perturbed


def test_shared_rejects_bad_arguments():
    from noise_amd import _lib
    pop = _lib.Population(2, 100, None, 1, _lib.ROUNDING_FUSED)  # tokens not a multiple of 64
    out = (ctypes.c_void_p * 3)(None, None, None)
    with pytest.raises(RuntimeError, match='multiple of 64'):
        _lib.call('noise_pop_qkv_shared', ctypes.byref(pop), None, None, None, None, None, out, _lib.stream_ptr(DEV))
    pop = _lib.Population(2, 128, None, 1, _lib.ROUNDING_EAGER)
    with pytest.raises(RuntimeError, match='eager'):
        _lib.call('noise_pop_qkv_shared', ctypes.byref(pop), None, None, None, None, None, out, _lib.stream_ptr(DEV))
