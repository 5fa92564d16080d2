"""Builds libnoise_amd.so (every HIP source under csrc/) in-tree for gfx950 with hipcc.

The library is the product's only compute path: noise_amd._lib loads it and raises if it is missing.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / 'csrc'
OUT = HERE / 'libnoise_amd.so'
OBJ = HERE / '_build'
ARCH = os.environ.get('NOISE_AMD_ARCH', 'gfx950')

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU instructions.
HIPFLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-Wall', '-Wno-unused-function',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-munsafe-fp-atomics',
]


def hipcc():
    exe = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not Path(exe).exists():
        raise RuntimeError('hipcc not found: the HIP toolchain is required to build libnoise_amd')
    return exe


# per-source additions: the fused MLP kernel (one wave per SIMD, 512 registers) needs the scheduler that keeps
# LDS fragment reads ahead of the matrix products; the default one serialises them at that register pressure
EXTRA = {'mlp.hip': ['-mllvm', '-amdgpu-sched-strategy=max-ilp']}


# host-side AddressSanitizer + UndefinedBehaviorSanitizer for the C-ABI layer (argument checks, error messages,
# struct handling); the device code is built as usual (GPU sanitizers are not used)
SANITIZE = ['-Xarch_host', '-fsanitize=address', '-Xarch_host', '-fsanitize=undefined',
            '-Xarch_host', '-fno-omit-frame-pointer', '-Xarch_host', '-fno-sanitize-recover=all']


def _compile(src: Path, obj_dir: Path = OBJ, extra=()) -> Path:
    obj = obj_dir / (src.stem + '.o')
    cmd = [hipcc(), *HIPFLAGS, *EXTRA.get(src.name, []), *extra, '-c', str(src), '-o', str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed on {src.name}:\n{res.stderr[-8000:]}')
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip and link libnoise_amd.so; always rebuilds."""
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob('*.hip'))
    workers = min(len(sources), int(os.environ.get('MAX_JOBS', '8')), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = OUT.with_suffix('.so.tmp')
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stderr[-8000:]}')
    os.replace(tmp, OUT)
    if verbose:
        print(f'built {OUT} from {len(sources)} sources', file=sys.stderr)
    return OUT


def build_sanitized(out_dir: Path) -> Path:
    """The library with the host code under ASan + UBSan, into out_dir (for tests that drive the C ABI's host
    layer on the CPU; load it with the sanitizer runtime preloaded: sanitizer_runtime())."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob('*.hip'))
    workers = min(len(sources), int(os.environ.get('MAX_JOBS', '8')), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objs = list(pool.map(lambda src: _compile(src, out_dir, SANITIZE), sources))
    out = out_dir / 'libnoise_amd_sanitized.so'
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *SANITIZE, '-o', str(out), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stderr[-8000:]}')
    return out


def sanitizer_runtime() -> Path:
    """The shared ASan runtime of the HIP toolchain's clang (to LD_PRELOAD into a host process)."""
    exe = Path(hipcc()).resolve()
    for root in (exe.parents[1] / 'llvm', exe.parents[1] / 'lib' / 'llvm', exe.parents[1]):
        hits = sorted(root.glob('lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so'))
        if hits:
            return hits[-1]
    raise RuntimeError('libclang_rt.asan-x86_64.so not found next to hipcc')


if __name__ == '__main__':
    build(verbose=True)
