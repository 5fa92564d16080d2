"""Pins the oracle's noise restatement (oracle/philox.c) without a GPU.

- Published Random123 known-answer vectors for Philox4x32-10 (Salmon et al., SC'11, kat_vectors).
- Two independent in-container implementations it was not derived from: torch's PhiloxRNGEngine.h and
  rocRAND's philox4x32_10 engine (the generator torch-ROCm's device draws use), driven through
  oracle/crosscheck/.
- The grid-stride layout closed form (torch: ATen/native/hip/DistributionTemplates.h:52-89) against a
  brute-force replay of the loop, and its known MI355X values.
"""
import subprocess

import numpy as np
import pytest

from oracle import noise as on

# Random123 kat_vectors: philox4x32 10 <counter x4> <key x2> <expected x4>
KATS = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff), (0xffffffff, 0xffffffff),
     (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.fixture(scope='module', autouse=True)
def built():
    on.build()


@pytest.mark.parametrize('ctr,key,expect', KATS)
def test_philox_kat(ctr, key, expect):
    assert tuple(int(x) for x in on.philox4x32(ctr, key)) == expect


def test_philox_round_count_matters():
    """A dropped or extra round changes the block (guards the round loop)."""
    ctr, key, expect = KATS[2]
    assert tuple(int(x) for x in on.philox4x32(ctr, key, rounds=9)) != expect
    assert tuple(int(x) for x in on.philox4x32(ctr, key, rounds=11)) != expect


def _run(driver, lines):
    res = subprocess.run([str(on.HERE / '_build' / driver)], input='\n'.join(lines) + '\n',
                         capture_output=True, text=True, check=True)
    return res.stdout.split('\n')


def _random_cases(n, seed=0):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        s = int(rng.integers(0, 2 ** 63)) * int(rng.integers(1, 3))
        sub = int(rng.integers(0, 2 ** 62))
        off = int(rng.integers(0, 2 ** 40))
        cases.append((s % 2 ** 64, sub, off))
    cases += [(0, 0, 0), (0, 524287, 1), (2 ** 64 - 1, 2 ** 64 - 1, 2 ** 64 - 1), (1, 2 ** 32, 2 ** 32 - 1)]
    return cases


def test_philox_matches_torch_engine():
    """torch's engine: counter = (block offset, subsequence), key = seed; first block."""
    cases = _random_cases(300)
    out = _run('torch_philox', [f'{s} {sub} {off} 1' for s, sub, off in cases])
    for (s, sub, off), line in zip(cases, out):
        ctr = (off & 0xffffffff, off >> 32, sub & 0xffffffff, sub >> 32)
        key = (s & 0xffffffff, s >> 32)
        assert ' '.join(f'{int(x):08x}' for x in on.philox4x32(ctr, key)) == line


def test_philox_matches_rocrand_engine_and_counter_carry():
    """rocRAND's engine with its offset in 32-bit words (hiprand_init's convention), several next4() calls
    per case so the 64-bit counter carry across word 0 -> 1 is exercised."""
    cases = [(s, sub, (off % 2 ** 34) * 4) for s, sub, off in _random_cases(100, seed=1)]
    cases.append((5, 9, (2 ** 32 - 2) * 4))  # crosses counter word 0 within the 3 blocks
    out = _run('rocrand_philox', [f'{s} {sub} {off} 3' for s, sub, off in cases])
    i = 0
    for s, sub, off in cases:
        for k in range(3):
            words = out[i].split()[:4]
            i += 1
            c = off // 4 + k
            ctr = (c & 0xffffffff, (c >> 32) & 0xffffffff, sub & 0xffffffff, sub >> 32)
            key = (s & 0xffffffff, s >> 32)
            assert [f'{int(x):08x}' for x in on.philox4x32(ctr, key)] == words


def test_host_box_muller_matches_rocrand_host_branch():
    """rocRAND's host Box-Muller (rocrand_normal.h:62-64) of a block's first two words vs the oracle's
    element with lane 0 / 1 of the same block."""
    out = _run('rocrand_philox', ['0 0 0 4', '77 12 40 4'])
    for line_no, (seed, sub, off) in enumerate([(0, 0, 0)] * 4 + [(77, 12, 40)] * 4):
        k = line_no % 4
        fields = out[line_no].split()
        threads = 2 ** 40  # one thread plane wider than any index used: element L = thread L, block k
        idx = np.array([sub + 4 * threads * k, sub + 4 * threads * k + threads])
        vals = on.randn(seed, off, threads, idx)
        assert np.float32(fields[4]) == vals[0]
        assert np.float32(fields[5]) == vals[1]


def test_grid_threads_known_values():
    """MI355X: 256 CUs x 2048 threads -> at most 2048 blocks of 256."""
    assert on.grid_threads(2 ** 28, 256, 2048) == 2 ** 19
    assert on.grid_threads(512, 256, 2048) == 512
    assert on.grid_threads(1, 256, 2048) == 256
    assert on.grid_threads(1000, 256, 2048) == 1024
    assert on.offset_increment(2 ** 28, 2 ** 19) == 512
    assert on.offset_increment(512, 512) == 4
    assert on.offset_increment(2 ** 21 + 1, 2 ** 19) == 8


def test_layout_matches_brute_force_grid_stride_loop():
    """Replays the kernel loop of DistributionTemplates.h:71-88 for a tiny grid and checks every element's
    (block, lane) against the closed form."""
    numel, threads, seed, offset = 3 * 4 * 256 + 77, 512, 99, 8
    expect = np.zeros(numel, dtype=np.uint32)
    rounded = ((numel - 1) // (threads * 4) + 1) * threads * 4
    for t in range(threads):
        k = 0
        for li0 in range(t, rounded, threads * 4):
            block = on.philox4x32((offset // 4 + k, 0, t, 0), (seed, 0))
            for lane in range(4):
                li = li0 + threads * lane
                if li < numel:
                    expect[li] = block[lane]
            k += 1
    got = on.draw_u32(seed, offset, threads, np.arange(numel))
    assert np.array_equal(got, expect)


def test_randint_is_mod_of_u32():
    idx = np.arange(1000)
    u = on.draw_u32(3, 4, 1024, idx).astype(np.int64)
    assert np.array_equal(on.randint(3, 4, 1024, 2 ** 28 - 2560, idx), u % (2 ** 28 - 2560))
    assert np.array_equal(on.randint(3, 4, 1024, 7, idx, base=-3), u % 7 - 3)


def test_randn_moments():
    """N(0,1) invariants over 2^20 draws of the reference buffer's layout."""
    x = on.randn(0, 0, 2 ** 19, np.arange(2 ** 20)).astype(np.float64)
    assert abs(x.mean()) < 5e-3
    assert abs(x.var() - 1) < 5e-3
    assert np.isfinite(x).all()


def test_generator_offsets_advance_like_torch():
    g = on.OracleGenerator(5)
    g.randint(0, 100, 512)
    assert g.offset == 4
    g.randn(2 ** 28)
    assert g.offset == 4 + 512
