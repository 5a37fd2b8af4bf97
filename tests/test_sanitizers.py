"""The host code of the native libraries under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU).

`make -C vectra_amd/csrc sanitize-test` builds libvectra_rbf.so,
libvectra_torch.so and libvectra_scan.so with their host code instrumented
(argument validation, kernel selection, the split top-k's workspace sizing,
the operator's checks and its CPU implementation; device code as usual) into
build/sanitize/lib, then runs tests/test_capi.py, tests/test_custom_op.py and
tests/test_scan_capi.py against them with clang's ASan runtime preloaded.
Any sanitizer report aborts that run, so this test fails on it.
"""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANGXX = '/opt/rocm/llvm/bin/clang++'


def _asan_runtime():
    if not os.path.exists(CLANGXX):
        return None
    path = subprocess.run([CLANGXX, '-print-file-name=libclang_rt.asan-x86_64.so'], capture_output=True,
                          text=True, check=False).stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


@pytest.mark.timeout(1800)
@pytest.mark.skipif(shutil.which('make') is None or _asan_runtime() is None,
                    reason='needs make and clang\'s shared ASan runtime')
def test_host_code_is_clean_under_asan_and_ubsan():
    jobs = str(min(8, os.cpu_count() or 1))
    env = dict(os.environ)
    env.pop('VECTRA_LIB_DIR', None)
    done = subprocess.run(['make', '-C', os.path.join(ROOT, 'vectra_amd', 'csrc'), '-j', jobs, 'sanitize-test'],
                          capture_output=True, text=True, timeout=1700, env=env, check=False)
    tail = (done.stdout + done.stderr)[-4000:]
    assert done.returncode == 0, tail
    assert 'passed' in done.stdout and 'failed' not in done.stdout, tail
    for marker in ('ERROR: AddressSanitizer', 'runtime error:'):
        assert marker not in done.stdout + done.stderr, tail
