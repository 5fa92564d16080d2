"""The C ABI's host layer under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU: the library is built
with the host code instrumented (noise_amd.build.build_sanitized; device code as usual) and driven by
tests/abi_host_child.py in a child process with the sanitizer runtime preloaded: all-zero and invalid arguments
for every entry point, long formatted messages, concurrent callers. Any sanitizer report fails the child."""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope='module')
def sanitized(tmp_path_factory):
    if not shutil.which('hipcc') and not Path('/opt/rocm/bin/hipcc').exists():
        pytest.skip('hipcc not available')
    from noise_amd.build import build_sanitized
    return build_sanitized(tmp_path_factory.mktemp('sanitized'))


def test_host_layer_clean_under_asan_ubsan(sanitized):
    from noise_amd.build import sanitizer_runtime
    env = dict(os.environ, LD_PRELOAD=str(sanitizer_runtime()),
               ASAN_OPTIONS='detect_leaks=0:halt_on_error=1:abort_on_error=0',
               UBSAN_OPTIONS='halt_on_error=1:print_stacktrace=1', HIP_VISIBLE_DEVICES='')
    res = subprocess.run([sys.executable, str(ROOT / 'tests' / 'abi_host_child.py'), str(sanitized)],
                         capture_output=True, text=True, env=env, timeout=300)
    out = res.stdout + res.stderr
    assert 'ERROR: AddressSanitizer' not in out and 'runtime error:' not in out, out[-4000:]
    assert res.returncode == 0 and out.strip().splitlines()[-1] == 'ok', out[-4000:]
