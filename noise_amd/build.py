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


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + '.o')
    cmd = [hipcc(), *HIPFLAGS, *EXTRA.get(src.name, []), '-c', str(src), '-o', str(obj)]
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


if __name__ == '__main__':
    build(verbose=True)
