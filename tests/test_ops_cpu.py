"""torch.library registrations: fake implementations give the real ops' shapes/dtypes (CPU, no kernels)."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode


def test_fake_shapes():
    import noise_amd.ops  # noqa: F401
    with FakeTensorMode():
        q = torch.empty(2, 256, 8, 64, dtype=torch.bfloat16)
        out = torch.ops.noise_amd.attention(q, q, q, 128)
        assert out.shape == q.shape and out.dtype == q.dtype
        x = torch.empty(4, 256, 512, dtype=torch.bfloat16)
        w = torch.empty(2048, 512)
        y = torch.ops.noise_amd.lowrank(x, w, torch.empty(2, 2048), torch.empty(2, 512), torch.empty(4), 2)
        assert y.shape == (4, 256, 2048) and y.dtype == torch.float32
        h = torch.ops.noise_amd.head_loss(torch.empty(3, 256, 512), torch.empty(4096, 512),
                                          torch.empty(3, 256, dtype=torch.long), 4096)
        assert h.shape == (768,) and h.dtype == torch.float32
