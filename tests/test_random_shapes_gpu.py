"""Randomised shapes through the drop-ins, against the oracle on the CPU (hypothesis, derandomised so every run
draws the same cases): attention (utils/model.py:24-31) over lengths off the 256-query tiles and on them, any
window, batch and heads; lowrank (eggroll.py:56-58) over widths on and off the MFMA tiles, shared and per-member
x; lowrank_embed (eggroll.py:61-63); coordinate_differences (run.py:121-137). Tolerances as the fixed-shape
tests of the same functions: attention 2e-2 of the output scale (bf16 operands), lowrank 1e-2 of the output
scale, lowrank_embed 1e-6, coordinate differences 2e-3 of the scale (fp32 logits)."""
import pytest
import torch
from hypothesis import HealthCheck, given, settings, strategies as st

from oracle import dust as od
from oracle import model as om

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)
CASES = settings(max_examples=10, deadline=None, derandomize=True, suppress_health_check=list(HealthCheck))


@CASES
@given(B=st.integers(1, 3), H=st.integers(1, 4), T=st.sampled_from([1, 7, 63, 64, 65, 200, 256, 300, 512]),
       window=st.sampled_from([0, 1, 17, 64, 255, 1024]), seed=st.integers(0, 2 ** 16))
def test_attention_random_shapes(B, H, T, window, seed):
    from noise_amd.model import attention
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, T, H, 64, generator=g).bfloat16() for _ in range(3))
    print(f'attention B={B} H={H} T={T} window={window} seed={seed}', flush=True)
    got = attention(q.to(DEV), k.to(DEV), v.to(DEV), window).float().cpu()
    ref = om.attention(q.float(), k.float(), v.float(), window)
    assert (got - ref).abs().max().item() <= 2e-2 * max(ref.abs().max().item(), 1.0)


@CASES
@given(m=st.sampled_from([2, 4, 6]), T=st.sampled_from([3, 64, 256, 300]), n_in=st.sampled_from([32, 96, 512]),
       n_out=st.sampled_from([8, 40, 256, 512]), shared=st.booleans(), seed=st.integers(0, 2 ** 16))
def test_lowrank_random_shapes(m, T, n_in, n_out, shared, seed):
    from noise_amd.eggroll import lowrank
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1 if shared else m // 2, T, n_in, generator=g)
    x = x.expand(m, T, n_in) if shared else x.repeat_interleave(2, 0)
    w = torch.randn(n_out, n_in, generator=g) * 0.05
    a, b = torch.randn(m // 2, n_out, generator=g), torch.randn(m // 2, n_in, generator=g)
    sign = torch.tensor([1e-2, -1e-2] * (m // 2))
    xd = x[:1].to(DEV).expand(m, T, n_in) if shared else x.to(DEV)
    print(f'lowrank m={m} T={T} in={n_in} out={n_out} shared={shared} seed={seed}', flush=True)
    y = lowrank(xd, w.to(DEV), a.to(DEV), b.to(DEV), sign.to(DEV), dir_div=2).cpu()
    ref = om.lowrank(x.bfloat16().float(), w.bfloat16().float(), a.repeat_interleave(2, 0), b.repeat_interleave(2, 0),
                     sign)
    assert y.shape == ref.shape
    assert (y - ref).abs().max().item() <= 1e-2 * ref.abs().max().item()


@CASES
@given(V=st.sampled_from([16, 100, 4096]), d=st.sampled_from([4, 64, 512]), T=st.integers(1, 300),
       m=st.integers(1, 5), seed=st.integers(0, 2 ** 16))
def test_lowrank_embed_random_shapes(V, d, T, m, seed):
    from noise_amd.eggroll import lowrank_embed
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(V, d, generator=g)
    a, b = torch.randn(m, V, generator=g), torch.randn(m, d, generator=g)
    idx = torch.randint(0, V, (T,), generator=g)
    sign = torch.randn(m, generator=g)
    print(f'lowrank_embed V={V} d={d} T={T} m={m} seed={seed}', flush=True)
    got = lowrank_embed(W.to(DEV), a.to(DEV), b.to(DEV), idx.to(DEV), sign.to(DEV)).cpu()
    assert torch.allclose(got, om.lowrank_embed(W, a, b, idx, sign), rtol=1e-6, atol=1e-6)


@CASES
@given(rows=st.integers(1, 40), V=st.sampled_from([64, 256, 1000, 4096]), sigma=st.sampled_from([0.01, 0.1, 1.0]),
       seed=st.integers(0, 2 ** 16))
def test_coordinate_differences_random_shapes(rows, V, sigma, seed):
    from noise_amd.dust import coordinate_differences
    g = torch.Generator().manual_seed(seed)
    raw = torch.randn(rows, V, generator=g) * 20
    y = torch.randint(-1, V, (rows,), generator=g)
    print(f'coordinate_differences rows={rows} V={V} sigma={sigma} seed={seed}', flush=True)
    got = coordinate_differences(raw.to(DEV), y.to(DEV), sigma).cpu()
    ref = torch.from_numpy(od.coordinate_differences(raw.numpy(), y.numpy(), sigma)).float()
    assert got.shape == ref.shape
    assert (got - ref).abs().max().item() <= 2e-3 * max(ref.abs().max().item(), 1e-3)
