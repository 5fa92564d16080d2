"""Device noise vs torch-ROCm's own device generator on the same GPU: bit-exact.

The reference's buffer is torch.randn(2**28, generator=Generator('cuda').manual_seed(0)) (eggroll.py:114);
its offsets are torch.randint draws on a seeded device generator (eggroll.py:117-120).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().view(torch.int32)


@pytest.fixture(scope='module')
def dev():
    return torch.device('cuda', 0)


@pytest.mark.parametrize('numel', [1, 255, 1000, 65536 + 3, 2 ** 20 + 7, 2 ** 24])
def test_randn_bit_exact(dev, numel):
    from noise_amd.noise import DeviceGenerator
    ref = torch.randn(numel, device=dev, generator=torch.Generator(dev).manual_seed(0))
    out = DeviceGenerator(0, dev).randn(numel)
    assert torch.equal(bits(out), bits(ref))


def test_reference_buffer_bit_exact(dev):
    """The full 2^28 buffer the reference draws once, seed 0."""
    from noise_amd.noise import DeviceGenerator
    ref = torch.randn(2 ** 28, device=dev, generator=torch.Generator(dev).manual_seed(0))
    out = DeviceGenerator(0, dev).randn(2 ** 28)
    eq = bits(out) == bits(ref)
    assert bool(eq.all()), f'{(~eq).sum().item()} of 2^28 differ'


def test_randn_offsets_and_slices(dev):
    """Successive draws advance the offset as torch does; slices equal the same elements of the full draw."""
    from noise_amd.noise import DeviceGenerator
    g = torch.Generator(dev).manual_seed(1234)
    mine = DeviceGenerator(1234, dev)
    for numel in (3000, 2 ** 21 + 5, 77):
        ref = torch.randn(numel, device=dev, generator=g)
        draw = mine.take(numel)
        assert torch.equal(bits(draw.normal()), bits(ref))
        for first, n in ((0, 1), (numel // 3, min(500, numel - numel // 3)), (numel - 1, 1)):
            assert torch.equal(bits(draw.normal(first, n)), bits(ref[first:first + n]))


@pytest.mark.parametrize('seed', [0, 7, 2 ** 40 + 3])
def test_randint_bit_exact(dev, seed):
    from noise_amd.noise import DeviceGenerator
    g = torch.Generator(dev).manual_seed(seed)
    mine = DeviceGenerator(seed, dev)
    for n, high in ((512, 2 ** 28 - 2560), (131072, 2 ** 28 - 4608), (1, 5), (70000, 2 ** 27 + 1), (3, 2)):
        ref = torch.randint(0, high, (n,), device=dev, generator=g)
        assert torch.equal(mine.randint(0, high, n), ref)


def test_gather_slices(dev):
    """Eggroll.noise's gather buffer[offsets[directions, None] + arange(width)] (eggroll.py:126)."""
    from noise_amd.noise import DeviceGenerator
    numel = 2 ** 22
    buf = torch.randn(numel, device=dev, generator=torch.Generator(dev).manual_seed(0))
    draw = DeviceGenerator(0, dev).take(numel)
    offsets = torch.randint(0, numel - 3000, (300,), device=dev, generator=torch.Generator(dev).manual_seed(5))
    directions = torch.arange(10, 138, 2, device=dev) % 300
    ref = buf[offsets[directions, None] + torch.arange(2560, device=dev)]
    out = draw.gather(offsets, 2560, directions)
    assert torch.equal(bits(out), bits(ref))


def test_gather_many_equals_per_parameter_gathers(dev):
    """One noise_gather_slice_groups launch for several parameters' slices (the step's 48 block matrices in the
    population forward) gives each parameter's columns bit for bit what its own gather gives, over the 2^28
    buffer's draw layout, with repeated and unordered rows; a width that is not a multiple of 256 is rejected."""
    from noise_amd.noise import DeviceGenerator
    from noise_amd import _lib
    draw = DeviceGenerator(0, dev).take(2 ** 28)
    g = torch.Generator(dev).manual_seed(7)
    widths = [1024, 2560, 2560, 4608, 1024]
    offsets = [torch.randint(0, 2 ** 28 - w, (300,), device=dev, generator=g) for w in widths]
    rows = torch.tensor([5, 5, 299, 0, 17, 123, 123, 4], device=dev)
    out = draw.gather_many(offsets, widths, rows)
    assert out.shape == (8, sum(widths))
    col = 0
    for o, w in zip(offsets, widths):
        assert torch.equal(bits(out[:, col:col + w]), bits(draw.gather(o, w, rows)))
        col += w
    with pytest.raises(RuntimeError, match='multiple of 256'):
        draw.gather_many(offsets[:1], [1000], rows)
