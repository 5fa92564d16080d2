"""HIP attention vs fp32 references (utils/model.py:24-31 semantics).

Tolerance (bf16 inputs, fp32 reference): relative Frobenius error ||out - ref|| / ||ref|| <= 2e-2 and
max |out - ref| <= 2e-2 * max |ref|.
"""
import math

import pytest
import torch

from oracle import model as om

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda', 0)


def rel_ok(out, ref, tol=2e-2):
    out, ref = out.float(), ref.float()
    fro = ((out - ref).norm() / ref.norm()).item()
    mx = ((out - ref).abs().max() / ref.abs().max()).item()
    assert fro <= tol and mx <= tol, f'rel fro {fro:.3e}, rel max {mx:.3e}'
    return fro, mx


def fp32_reference_gpu(q, k, v, window):
    """Dense masked softmax in fp32 on the GPU, one batch at a time (no bf16 batched products)."""
    B, T, H, D = q.shape
    i = torch.arange(T, device=q.device)[:, None]
    j = torch.arange(T, device=q.device)[None, :]
    visible = (i >= j) & (i - j <= window)
    out = torch.empty(B, T, H, D, device=q.device, dtype=torch.float32)
    for b in range(B):
        qh, kh, vh = (t[b].float().transpose(0, 1).contiguous() for t in (q, k, v))
        s = torch.matmul(qh, kh.transpose(-1, -2).contiguous()) / math.sqrt(D)
        s = s.masked_fill(~visible, float('-inf'))
        out[b] = torch.matmul(torch.softmax(s, -1), vh).transpose(0, 1)
    return out


def test_config_attention_causal():
    """bf16 q, k, v [B=16, H=8, T=2048, D=64] ~ N(0,1) from one CPU generator seed 0 (q, k, v in order),
    causal, passed as the [B, T, H, D] views the reference's attention() takes."""
    from noise_amd.model import attention
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(16, 8, 2048, 64, generator=g).bfloat16().to(DEV).transpose(1, 2) for _ in range(3))
    out = attention(q, k, v, 2048)
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    rel_ok(out, fp32_reference_gpu(q, k, v, 2048))


@pytest.mark.parametrize('B,T,H,window', [(2, 2048, 8, 1024), (1, 1000, 3, 300), (3, 64, 8, 0), (1, 130, 2, 5000),
                                          (2, 513, 8, 64)])
def test_windows_and_ragged_lengths_vs_oracle(B, T, H, window):
    """Against the CPU oracle (dense masked fp32): window edges, lengths not multiple of 64,
    heads not a multiple of 8, window 0 (each query sees only itself)."""
    from noise_amd.model import attention
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(B, T, H, 64, generator=g).bfloat16() for _ in range(3))
    out = attention(q.to(DEV), k.to(DEV), v.to(DEV), window).cpu()
    ref = om.attention(q.float(), k.float(), v.float(), window)
    rel_ok(out, ref)
    if window == 0:
        assert torch.equal(out, v), 'window 0: each query returns its own value row'


def test_strided_views_and_fp32_inputs():
    """[B, H, T, D] storage passed as transposed views (the reference's flex call layout), fp32 in -> fp32 out."""
    from noise_amd.model import attention
    g = torch.Generator().manual_seed(2)
    qh, kh, vh = (torch.randn(2, 8, 512, 64, generator=g).to(DEV) for _ in range(3))
    q, k, v = (t.transpose(1, 2) for t in (qh, kh, vh))
    out = attention(q, k, v, 200)
    assert out.dtype == torch.float32
    rel_ok(out, fp32_reference_gpu(q.bfloat16(), k.bfloat16(), v.bfloat16(), 200))


def _rms_normed(x):
    return (x.float() / torch.sqrt((x.float() ** 2).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps)).bfloat16()


@pytest.mark.parametrize('qk_normed', [False, True])
def test_transposed_v_and_fused_dot(qk_normed):
    """Population layout: q, k [B, H, T, D], v^T [B, H, D, T], fused x.b dot per head; with and without the
    RMS-normed promise (q, k are RMSNorm outputs, as utils/model.py:94 makes them)."""
    from noise_amd.model import attention_raw
    g = torch.Generator().manual_seed(3)
    B, H, T = 4, 8, 256
    q, k, v = (torch.randn(B, T, H, 64, generator=g).bfloat16().to(DEV) for _ in range(3))
    q, k = _rms_normed(q), _rms_normed(k)
    qh, kh = q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
    vt = v.permute(0, 2, 3, 1).contiguous()  # [B, H, D, T]
    out = torch.empty(B, T, H, 64, dtype=torch.bfloat16, device=DEV)
    dvec = torch.randn(B // 2, H * 64, generator=g).to(DEV)
    dot = torch.empty(B, T, H, device=DEV)
    attention_raw(qh.transpose(1, 2), kh.transpose(1, 2), vt, out, 100, v_transposed=True, dot_vec=dvec,
                  dot_div=2, dot_out=dot, qk_normed=qk_normed)
    rel_ok(out, fp32_reference_gpu(q, k, v, 100))
    expect = (out.float().view(B, T, H, 64) * dvec.repeat_interleave(2, 0).view(B, 1, H, 64)).sum(-1)
    assert torch.allclose(dot, expect, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize('window', [1024, 2048])
def test_transposed_v_population_shape(window):
    """[2 members, 8 heads, 2048 tokens], RMS-normed q, k (seed 5): the fixed-shift softmax and the
    running-max softmax of the transposed-V kernel both match the fp32 reference, and each other closely."""
    from noise_amd.model import attention_raw
    g = torch.Generator().manual_seed(5)
    B, H, T = 2, 8, 2048
    q, k = (_rms_normed(torch.randn(B, T, H, 64, generator=g)).to(DEV) for _ in range(2))
    v = torch.randn(B, T, H, 64, generator=g).bfloat16().to(DEV)
    vt = v.permute(0, 2, 3, 1).contiguous()
    ref = fp32_reference_gpu(q, k, v, window)
    outs = []
    for normed in (True, False):
        out = torch.empty(B, T, H, 64, dtype=torch.bfloat16, device=DEV)
        attention_raw(q, k, vt, out, window, v_transposed=True, qk_normed=normed)
        rel_ok(out, ref)
        outs.append(out.float())
    assert (outs[0] - outs[1]).abs().max().item() <= 2e-2 * ref.abs().max().item()


@pytest.mark.parametrize('qk_normed,window', [(False, 2048), (False, 300), (True, 1024), (True, 0)])
def test_natural_v_ring_kernel_equals_transposed(qk_normed, window):
    """The ring kernel on V in its natural layout (V^T fragments put together by transposing LDS reads) against
    the same kernel on V^T: the same bf16 operands in the same products, so the outputs are bit-identical. V
    is a [B, T, H, D] view of [B, H, T, D] storage (token stride 64, not heads * 64); 1024 tokens, 3 heads."""
    from noise_amd.model import attention_raw
    g = torch.Generator().manual_seed(8)
    B, H, T = 2, 3, 1024
    q, k = (torch.randn(B, T, H, 64, generator=g) for _ in range(2))
    q, k = (_rms_normed(t) if qk_normed else t.bfloat16() for t in (q, k))
    q, k = q.to(DEV), k.to(DEV)
    vh = torch.randn(B, H, T, 64, generator=g).bfloat16().to(DEV)
    v, vt = vh.transpose(1, 2), vh.transpose(2, 3).contiguous()
    outs = []
    for layout, vv in (('natural', v), ('transposed', vt)):
        out = torch.full((B, T, H, 64), float('nan'), dtype=torch.bfloat16, device=DEV)
        attention_raw(q, k, vv, out, window, v_transposed=layout == 'transposed', qk_normed=qk_normed)
        outs.append(out)
    assert torch.equal(outs[0], outs[1]), 'natural-V and V^T ring kernels differ'
    rel_ok(outs[0], fp32_reference_gpu(q, k, v, window))
    if window == 0:
        assert torch.equal(outs[0], v), 'window 0: each query returns its own value row'


def test_transposed_v_normed_promise_broken_stays_finite():
    """q, k of RMS 2.5 (scores up to ~6x the normed bound) under the fixed shift: still finite and right."""
    from noise_amd.model import attention_raw
    g = torch.Generator().manual_seed(6)
    B, H, T = 1, 8, 512
    q, k = ((2.5 * _rms_normed(torch.randn(B, T, H, 64, generator=g)).float()).bfloat16().to(DEV) for _ in range(2))
    v = torch.randn(B, T, H, 64, generator=g).bfloat16().to(DEV)
    out = torch.empty(B, T, H, 64, dtype=torch.bfloat16, device=DEV)
    attention_raw(q, k, v.permute(0, 2, 3, 1).contiguous(), out, 300, v_transposed=True, qk_normed=True)
    assert torch.isfinite(out.float()).all()
    rel_ok(out, fp32_reference_gpu(q, k, v, 300))


def test_transposed_v_ragged_length():
    """T = 300 (not a multiple of the 256-query tile) in the transposed layout takes the general kernel."""
    from noise_amd.model import attention_raw
    g = torch.Generator().manual_seed(7)
    B, H, T = 2, 3, 300
    q, k, v = (torch.randn(B, T, H, 64, generator=g).bfloat16().to(DEV) for _ in range(3))
    vt = torch.zeros(B, H, 64, 304, dtype=torch.bfloat16, device=DEV)  # token stride 304: 16 B aligned rows
    vt[..., :T] = v.permute(0, 2, 3, 1)
    out = torch.empty(B, T, H, 64, dtype=torch.bfloat16, device=DEV)
    attention_raw(q, k, vt, out, 77, v_transposed=True, qk_normed=False)
    rel_ok(out, fp32_reference_gpu(q, k, v, 77))


def test_deterministic():
    from noise_amd.model import attention
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(2, 1024, 8, 64, generator=g).bfloat16().to(DEV) for _ in range(3))
    assert torch.equal(attention(q, k, v, 1024), attention(q, k, v, 1024))


def test_invalid_head_dim_raises():
    from noise_amd.model import attention
    q = torch.zeros(1, 64, 2, 32, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match='head_dim must be 64'):
        attention(q, q, q, 10)


def test_v_transpose_layout_exact():
    """noise_v_transpose: V [B, T, H, D] (a strided view) -> [B, H, D, T], bit for bit; the drop-in on the
    same strided V (T a multiple of 256: the ring kernel on natural V) against the fp32 reference."""
    from noise_amd import _lib
    from noise_amd.model import attention
    g = torch.Generator().manual_seed(3)
    v = torch.randn(2, 3, 512, 64, generator=g).bfloat16().to(DEV).transpose(1, 2)  # [B, T, H, D] view
    vt = torch.empty(2, 3, 64, 512, dtype=torch.bfloat16, device=DEV)
    _lib.call('noise_v_transpose', v.data_ptr(), 2, 3, 512, 64, v.stride(0), v.stride(2), v.stride(1),
              vt.data_ptr(), _lib.stream_ptr(DEV))
    assert torch.equal(vt, v.permute(0, 2, 3, 1))
    with pytest.raises(RuntimeError, match='multiple of 64'):
        _lib.call('noise_v_transpose', v.data_ptr(), 2, 3, 500, 64, v.stride(0), v.stride(2), v.stride(1),
                  vt.data_ptr(), _lib.stream_ptr(DEV))
    q, k = (torch.randn(2, 512, 3, 64, generator=g).bfloat16().to(DEV) for _ in range(2))
    fast = attention(q, k, v, 200)
    ref = fp32_reference_gpu(q, k, v, 200)
    rel_ok(fast, ref)


@pytest.mark.parametrize('T', [1024, 600])
def test_running_max_rescales_as_scores_grow(T):
    """Scores that grow along the keys (k rows scaled by 1 .. 150 with the key position, q along the same
    direction): a query's maximum climbs to ~80 in log2 units, passing the stale reference maximum by more than 8
    again and again, so the lazy rescale runs in many tiles, of the ring kernel (T = 1024) and of the general
    kernel (T = 600). Against the fp32 reference."""
    from noise_amd.model import attention
    g = torch.Generator().manual_seed(9)
    B, H = 2, 3
    u = torch.randn(64, generator=g)
    u = u / u.norm()
    ramp = torch.linspace(1.0, 150.0, T).view(1, T, 1, 1)
    q = (3.0 * u + 0.3 * torch.randn(B, T, H, 64, generator=g)).bfloat16()
    k = (ramp * (u + 0.3 * torch.randn(B, T, H, 64, generator=g))).bfloat16()
    v = torch.randn(B, T, H, 64, generator=g).bfloat16()
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    out = attention(q, k, v, T)
    assert torch.isfinite(out.float()).all()
    rel_ok(out, fp32_reference_gpu(q, k, v, T))
