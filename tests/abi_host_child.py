"""Drives the C ABI's host layer of a libnoise_amd build without a GPU (run by test_abi_sanitized_cpu.py in a child
process with the ASan runtime preloaded): every entry point with all-zero arguments, targeted invalid arguments,
long error messages, and concurrent calls from several threads (the error message is per host thread). Loads
noise_amd/abi.py by path, so that torch is never imported into the sanitized process."""
import ctypes
import importlib.util
import sys
import threading
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
spec = importlib.util.spec_from_file_location('noise_abi', ROOT / 'noise_amd' / 'abi.py')
abi = importlib.util.module_from_spec(spec)
spec.loader.exec_module(abi)

lib = abi.bind(ctypes.CDLL(sys.argv[1]))
QUERIES = {'noise_abi_version', 'noise_last_error', 'noise_dust_block_workspace_bytes',
           'noise_dust_block_static_max_bytes', 'noise_update_workspace_bytes'}


def zero(t):
    return abi.View(None, 0, 0) if t == 'View' else (None if t is ctypes.c_void_p else t(0))


def message():
    return lib.noise_last_error().decode()


assert lib.noise_abi_version() == 2
rejected = 0
for name, argtypes in abi.SIGNATURES.items():
    fn = getattr(lib, name)
    st = fn(*[zero(t) for t in argtypes])
    if name in QUERIES:
        continue
    assert st != 0, f'{name} accepted all-zero arguments'
    assert message(), f'{name} returned {st} without a message'
    rejected += 1
print(f'all-zero arguments: {rejected} entry points rejected them with a message', flush=True)

# targeted invalid arguments (values that pass the NULL checks)
pop = abi.Population(2, 300, None, 2, 0)
assert lib.noise_pop_block(ctypes.byref(pop), abi.View(16, 0, 512), 16, None, None, 0, abi.View(16, 0, 512), 16, None,
                           16, None, 16, 0, None, None, None, None, 0, abi.View(None, 0, 0), 16, 0, None, 0, None,
                           None) == -1
assert 'multiple of' in message()
assert lib.noise_pop_block_qkv(ctypes.byref(pop), abi.View(16, 0, 512), 16, None, None, 0, abi.View(16, 0, 512), 16,
                               None, 16, None, 16, 0, None, None, None, None, 0, abi.View(None, 0, 0), None, None, None,
                               None, None, 0, None, 0, None, None, None, None, None) == -1
assert 'multiple of' in message()
big = abi.Population(1 << 40, 1 << 40, None, 1, 0)
assert lib.noise_member_mean(16, 1 << 40, 1 << 40, 16, None) != 0
assert lib.noise_rank1_expand(ctypes.byref(big), 16, 4, 16, 0, None, 16, 1, None) == -1
r1 = abi.Rank1(16, None, 4, 0)
pop4 = abi.Population(4, 8, 16, 3, 0)
assert lib.noise_rank1_expand(ctypes.byref(pop4), 16, 4, 16, 1, ctypes.byref(r1), 16, 1, None) == -1
assert 'directions' in message()  # dots_stride 1 < 2 directions: the %lld message formatting
assert lib.noise_attention_fwd(16, 16, 16, 16, 1, 1, 64, 32, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 10, 0.1, None, 0, 1,
                               None, None) == -1
assert 'head_dim' in message()
# the allocation-free DUST block: a shape beyond its static scratch is rejected before any HIP call
cap, need = lib.noise_dust_block_static_max_bytes(), lib.noise_dust_block_workspace_bytes(64, 2048, 1)
assert need > cap
w7 = (ctypes.c_void_p * 7)(*([16] * 7))
assert lib.noise_dust_block_static(16, 16, 64, 2048, w7, 16, 16, 16, 1024, None, None, None, None, None) == -1
assert 'static array holds' in message()
# the grouped noise gather: the descriptor's group count, widths and packing, the rows per call and the row stride
sg = abi.SliceGroups()
gather = lambda nrows, ld: lib.noise_gather_slice_groups(16, nrows, ld, ctypes.byref(sg), None, 1 << 20, 0, 0, 1 << 19,
                                                         None)
for count in (0, abi.SLICE_GROUPS_MAX + 1):
    sg.count = count
    assert gather(4, 1 << 16) == -1 and f'got {count}' in message()
sg.count = 2
sg.offsets[0] = sg.offsets[1] = 16
sg.width[0], sg.width[1], sg.col[0], sg.col[1] = 256, 300, 0, 256
assert gather(4, 1 << 16) == -1 and 'group 1' in message()      # width not a multiple of 256
sg.width[1], sg.col[1] = 256, 200
assert gather(4, 1 << 16) == -1 and 'column 256' in message()   # not packed in order
sg.col[1] = 256
assert gather(4, 300) == -1 and 'row stride 300' in message()   # below the total width of 512
assert gather(70000, 1 << 16) == -1 and 'rows per call' in message()
# direct_errors' mask-and-scale pass and the rerun's row kernels
assert lib.noise_mask_scale(16, None, 2, 12, 0.1, 16, None) == -1 and 'multiple of 8' in message()
assert lib.noise_mask_scale(8, None, 2, 16, 0.1, 16, None) == -1 and '16 B aligned' in message()
assert lib.noise_block_entry(16, 4, 8, 4, 16, 16, None) == -1 and 'add must be 16 B aligned' in message()
assert lib.noise_add_bf16(16, 16, 12, None) == -1 and 'multiple of 8' in message()
assert lib.noise_rerun_mix_norm(16, 4, 16, 4, None, None, 4, 16, 16, None) == -1 and 'lambdas' in message()
# the jittered block kernel: no jitter, misaligned jitter rows, no zero row for a block without mlp.c_proj jitter
pop_j = abi.Population(2, 256, None, 1, 0)
y_j = abi.View(256, 256 * 512, 512)
for (fc, mlp, zero), text in (((None, None, None), 'NULL or empty'), ((8, None, 256), '16 B aligned'),
                              ((256, None, None), 'zero row')):
    jit = abi.BlockJitter(fc, mlp, zero)
    assert lib.noise_pop_block_jit(ctypes.byref(pop_j), y_j, 256, y_j, 256, 256, 0, None, None, abi.View(None, 0, 0),
                                   256, 1, ctypes.byref(jit), None) == -1
    assert text in message(), message()
print('targeted invalid arguments: rejected', flush=True)

# concurrent calls: each thread's message is its own call's
errors = []


def worker(k):
    try:
        for _ in range(200):
            p = abi.Population(2, 300 + 2 * k, None, 2, 0)
            st = lib.noise_pop_block(ctypes.byref(p), abi.View(16, 0, 512), 16, None, None, 0, abi.View(16, 0, 512), 16,
                                     None, 16, None, 16, 0, None, None, None, None, 0, abi.View(None, 0, 0), 16, 0,
                                     None, 0, None, None)
            assert st == -1 and f'({300 + 2 * k})' in message(), message()
    except AssertionError as e:
        errors.append(str(e))


threads = [threading.Thread(target=worker, args=(k,)) for k in range(8)]
for t in threads:
    t.start()
for t in threads:
    t.join()
assert not errors, errors[:3]
print('threads: per-thread messages intact', flush=True)
print('ok', flush=True)
