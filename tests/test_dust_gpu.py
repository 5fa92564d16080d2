"""DUST's head error on the GPU (noise_coordinate_differences through the C ABI) against the float64
oracle (oracle/dust.py). The kernel computes in fp32 as the reference's torch ops do; the moved logits'
differences z' - z (about sigma) carry fp32 rounding of the capped values (~2e-6), so entries agree to
5e-5 absolute (entries are O(1))."""
import numpy as np
import pytest
import torch

from oracle import dust as odust

pytestmark = pytest.mark.gpu
ATOL = 5e-5


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_head_error_matches_oracle(dtype):
    from noise_amd.dust import head_error
    g = torch.Generator().manual_seed(0)
    logits = (torch.randn(2, 512, 4096, generator=g) * 5).to(dtype)
    y = torch.randint(0, 4000, (2, 512), generator=g)
    y[0, :7] = -1
    y[1, 100] = 3999
    got = head_error(logits.cuda(), y.cuda(), 4000, 0.1).cpu().numpy()
    ref = odust.head_error(logits.float().numpy(), y.numpy(), 4000, 0.1)
    err = float(np.abs(got - ref).max())
    print(dtype, 'max abs err', err, flush=True)
    assert got.shape == (2, 512, 4096)
    assert np.all(got[..., 4000:] == 0) and np.all(got[0, :7] == 0)
    assert err <= ATOL


def test_coordinate_differences_sum_rule():
    # sum_j of the exact derivative (softmax - onehot) * cap' has no closed form, but a token whose logits
    # are all equal has cap' equal everywhere and softmax uniform: the row sums to 0 up to O(sigma^2)
    from noise_amd.dust import coordinate_differences
    raw = torch.full((64, 4096), 2.5, dtype=torch.float32)
    y = torch.arange(64) * 61
    got = coordinate_differences(raw.cuda(), y.cuda(), 0.01).cpu().double()
    assert float(got.sum(-1).abs().max()) < 1e-4
    ref = odust.coordinate_differences(raw.numpy(), y.numpy(), 0.01)
    assert float(np.abs(got.numpy() - ref).max()) <= ATOL
