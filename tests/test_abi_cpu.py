"""The C ABI without a GPU: libnoise_amd.so loads, exports every entry point include/noise_amd.h declares,
and rejects invalid arguments with NOISE_EINVAL and a message (argument checks run before any HIP call)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / 'include' / 'noise_amd.h').read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(noise_[a-z0-9_]+)\s*\(', text)))


@pytest.fixture(scope='module')
def lib():
    from noise_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail(f'{_lib.LIB_PATH} is not built (run __graft_entry__.build())')
    return _lib.lib()


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), f'{n} declared in include/noise_amd.h but not exported'


def test_every_declared_symbol_has_a_ctypes_signature():
    from noise_amd import _lib
    missing = [n for n in declared() if n not in _lib.SIGNATURES]
    assert not missing, missing


def declarations():
    """name -> [parameter type] for every entry point of include/noise_amd.h (parameter names dropped)."""
    text = (ROOT / 'include' / 'noise_amd.h').read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    out = {}
    for name, args in re.findall(r'\b(noise_[a-z0-9_]+)\s*\(([^;()]*)\)\s*;', text, flags=re.S):
        params = []
        for a in args.split(','):
            a = ' '.join(a.split())
            if not a or a == 'void':
                continue
            m = re.match(r'(.*?)(\w+)(\s*\[\d*\])?$', a)
            params.append(m.group(1).strip() + (' []' if m.group(3) else ''))
        out[name] = params
    return out


def test_ctypes_signatures_match_the_header():
    """Each entry point's ctypes argtypes agree with its C declaration parameter by parameter (a ctypes call
    with a wrong argument list would not fail; it would pass the wrong bits)."""
    import ctypes
    import importlib.util
    spec = importlib.util.spec_from_file_location('noise_abi', ROOT / 'noise_amd' / 'abi.py')
    abi = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(abi)

    def expected(t):
        if '*' in t or t.endswith('[]') or t == 'noise_stream_t':
            return ctypes.c_void_p
        return {'noise_view_t': 'View', 'int64_t': ctypes.c_int64, 'uint64_t': ctypes.c_uint64, 'int': ctypes.c_int,
                'float': ctypes.c_float}[t]

    decl = declarations()
    assert set(decl) == set(abi.SIGNATURES), set(decl) ^ set(abi.SIGNATURES)
    for name, params in decl.items():
        want = [expected(t) for t in params]
        assert abi.SIGNATURES[name] == want, f'{name}: header {params}, ctypes {abi.SIGNATURES[name]}'


def test_struct_layouts_match_the_header(tmp_path):
    """The ctypes mirrors of noise_view_t, noise_rank1_t, noise_population_t, noise_update_param_t and
    noise_slice_groups_t have the
    sizes and field offsets a C compiler gives the header's structs (gcc on include/noise_amd.h)."""
    import ctypes
    import shutil
    import subprocess
    import importlib.util
    gcc = shutil.which('gcc')
    if gcc is None:
        pytest.skip('gcc not available')
    spec = importlib.util.spec_from_file_location('noise_abi', ROOT / 'noise_amd' / 'abi.py')
    abi = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(abi)
    structs = {'noise_view_t': abi.View, 'noise_rank1_t': abi.Rank1, 'noise_population_t': abi.Population,
               'noise_update_param_t': abi.UpdateParam, 'noise_slice_groups_t': abi.SliceGroups,
               'noise_block_jitter_t': abi.BlockJitter}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "noise_amd.h"', 'int main(void) {']
    for c_name, py in structs.items():
        lines.append(f'    printf("{c_name} size %zu\\n", sizeof({c_name}));')
        for field, _ in py._fields_:
            lines.append(f'    printf("{c_name} {field} %zu\\n", offsetof({c_name}, {field}));')
    lines += ['    return 0;', '}']
    src = tmp_path / 'layout.c'
    src.write_text('\n'.join(lines) + '\n')
    exe = tmp_path / 'layout'
    subprocess.run([gcc, '-std=c99', '-I', str(ROOT / 'include'), str(src), '-o', str(exe)], check=True)
    got = dict(line.rsplit(' ', 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                               check=True).stdout.splitlines())
    for c_name, py in structs.items():
        assert int(got[f'{c_name} size']) == ctypes.sizeof(py), c_name
        for field, _ in py._fields_:
            assert int(got[f'{c_name} {field}']) == getattr(py, field).offset, f'{c_name}.{field}'


def test_abi_version(lib):
    assert lib.noise_abi_version() == 2


def _err(lib):
    return lib.noise_last_error().decode()


def test_invalid_arguments_return_einval(lib):
    from noise_amd import _lib
    # attention: head_dim must be 64
    st = lib.noise_attention_fwd(1, 1, 1, 1, 1, 1, 64, 32, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 10, 0.1, None, 0, 1,
                                 None, None)
    assert st == -1 and 'head_dim' in _err(lib)
    # randint: range outside torch's 32-bit path
    st = lib.noise_randint(None, 4, 0, 0, 256, 2 ** 28, 0, None)
    assert st == -1 and 'range' in _err(lib)
    # normal fill: generator offset must be a multiple of 4
    st = lib.noise_normal_fill(None, 4, 0, 0, 2, 256, 0.0, 1.0, None)
    assert st == -1 and 'multiple of 4' in _err(lib)
    # population kernels: tokens must be a multiple of the tile
    pop = _lib.Population(2, 300, None, 2)
    st = lib.noise_pop_fc(ctypes.byref(pop), _lib.View(16, 0, 512), 16, None, None, 16, None, None, None)
    assert st == -1 and 'multiple of 256' in _err(lib)
    # missing population
    st = lib.noise_member_mean(None, 0, 10, None, None)
    assert st == -1
    # embedding entry: a vocabulary size is required (ids outside it become NaN rows on the device)
    pop = _lib.Population(2, 256, None, 1)
    st = lib.noise_pop_embed(ctypes.byref(pop), 0, 16, 0, 16, None, 16, 16, None, None, 0, 16, 16, 16, None)
    assert st == -1 and 'vocab' in _err(lib)
    # residual writer: mixing needs the device addresses of the mixing scalars
    st = lib.noise_pop_residual(ctypes.byref(pop), _lib.View(16, 0, 512), 16, 512, None, None, 0, 0,
                                _lib.View(16, 0, 512), None, 1, None, None, None, None, 0, _lib.View(16, 0, 512), 16,
                                0, None, 0, None, None)
    assert st == -1 and 'lam_r' in _err(lib)
    # generic lowrank: empty shapes rejected
    st = lib.noise_lowrank_rows(ctypes.byref(pop), _lib.View(16, 0, 32), 0, 16, 8, None, 16, None)
    assert st == -1


def test_python_raises_runtime_error_with_message():
    from noise_amd import _lib
    with pytest.raises(RuntimeError, match='invalid argument.*head_dim'):
        _lib.call('noise_attention_fwd', 1, 1, 1, 1, 1, 1, 64, 32, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 10, 0.1,
                  None, 0, 1, None, None)


def test_product_does_not_import_the_oracle():
    """The product package never routes through oracle/ (no CPU fallback)."""
    for f in (ROOT / 'noise_amd').rglob('*.py'):
        src = f.read_text()
        assert not re.search(r'^\s*(from|import)\s+oracle\b', src, re.M), f
