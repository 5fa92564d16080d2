"""noise_pop_qkv's two kernels against each other through the C ABI: the two-waves-per-SIMD kernel (fused
rounding, 16 B aligned outputs) and the tiled one (taken when an output is only 8 B aligned), on the same
inputs with rank-1 terms, value embeddings with gates, value-table noise and an out-of-range token id.

Both accumulate the products in fp32 in different orders and round Q, K, V to bf16: elements agree within one
bf16 ulp of their magnitude (plus 1e-6), and the NaN rows of the bad token id match."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def _inputs(m, T, dirs, seed, ve):
    from noise_amd.model import rotary_tables
    g = torch.Generator().manual_seed(seed)
    c = dict(x=torch.randn(m, T, 512, generator=g).bfloat16(),
             ws=[(torch.randn(512, 512, generator=g) * 0.04).bfloat16() for _ in range(3)],
             a=[torch.randn(dirs, 512, generator=g) for _ in range(3)],
             dots=torch.randn(m * T, 3, generator=g),
             sign=torch.tensor([0.05, -0.05]).repeat(m // 2))
    c['cos'], c['sin'] = (t.bfloat16().contiguous() for t in rotary_tables(T))
    if ve:
        c['ve'] = torch.randn(100, 512, generator=g)
        c['idx'] = torch.randint(0, 100, (T,), generator=g)
        c['idx'][5] = 100  # outside the table: V rows of this token are NaN
        c['gates'] = torch.rand(m * T, 8, generator=g) * 2
        c['ve_a'] = torch.randn(dirs, 100, generator=g)
        c['ve_b'] = torch.randn(dirs, 512, generator=g)
    return {k: ([t.to(DEV) for t in v] if isinstance(v, list) else v.to(DEV)) for k, v in c.items()}


def _run(c, m, T, dirs, aligned16):
    from noise_amd import _lib
    pop = _lib.Population(m, T, c['sign'].data_ptr(), m // dirs, _lib.ROUNDING_FUSED)
    r1 = (_lib.Rank1 * 3)(*[_lib.Rank1(a.data_ptr(), a.data_ptr(), a.stride(0), a.stride(0)) for a in c['a']])
    wp = (ctypes.c_void_p * 3)(*(w.data_ptr() for w in c['ws']))
    off = 0 if aligned16 else 4  # 4 bf16 = 8 bytes: the tiled kernel
    flat = torch.full((3 * m * 8 * T * 64 + off,), float('nan'), dtype=torch.bfloat16, device=DEV)
    qkv = flat[off:].view(3, m, 8, T, 64)
    op = (ctypes.c_void_p * 3)(*(qkv[i].data_ptr() for i in range(3)))
    ve = 've' in c
    vn = _lib.Rank1(c['ve_a'].data_ptr(), c['ve_b'].data_ptr(), c['ve_a'].stride(0), c['ve_b'].stride(0)) if ve else None
    _lib.call('noise_pop_qkv', ctypes.byref(pop), _lib.View(c['x'].data_ptr(), T * 512, 512), wp, r1,
              c['dots'].data_ptr(), c['cos'].data_ptr(), c['sin'].data_ptr(), c['ve'].data_ptr() if ve else None,
              100 if ve else 0, c['idx'].data_ptr() if ve else None, 0, c['gates'].data_ptr() if ve else None,
              ctypes.byref(vn) if ve else None, op, _lib.stream_ptr(DEV))
    torch.cuda.synchronize()
    return qkv.float().cpu()


@pytest.mark.parametrize('ve', [False, True], ids=['plain', 'value-embeddings'])
def test_two_wave_kernel_matches_tiled(ve):
    m, T, dirs = 4, 256, 2
    print(f'qkv rows: {m} members x {T} tokens, value embeddings {ve}', flush=True)
    c = _inputs(m, T, dirs, 7, ve)
    got = _run(c, m, T, dirs, True)
    ref = _run(c, m, T, dirs, False)
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    if ve:
        vt = got[2].reshape(m, 8, 64, T)  # V is stored transposed, [m][8][64][T]
        assert torch.isnan(vt[..., 5]).all() and not torch.isnan(vt[..., 6]).any()
    ok = ~torch.isnan(ref)
    assert ok[:2].all()
    ulp = ref[ok].abs() * 2.0 ** -7 + 1e-6
    assert ((got[ok] - ref[ok]).abs() <= ulp).all()
