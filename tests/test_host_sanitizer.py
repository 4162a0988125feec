"""The C ABI's host code (argument checks, the weight packer, the tree-column builder, engine creation without a GPU)
under AddressSanitizer and UndefinedBehaviorSanitizer: the library is rebuilt with both on the host side
(seedplane_amd.build.build_sanitized; the gfx950 code is unchanged) and the CPU tests of that code run against it in a
child process with the clang ASan runtime preloaded.  Any report aborts the child (halt_on_error), failing the test.
The build is cached in _build/ and redone when a source under seedplane_amd/csrc or include/ is newer."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

from seedplane_amd import build as B

ROOT = Path(__file__).resolve().parents[1]
SOURCES = list((ROOT / 'seedplane_amd' / 'csrc').glob('*')) + list((ROOT / 'include').glob('*.h'))


def _sanitized_lib():
    out = B.SAN_OUT
    if not out.is_file() or out.stat().st_mtime < max(p.stat().st_mtime for p in SOURCES):
        B.build_sanitized(out)
    return out


def test_host_code_is_clean_under_asan_and_ubsan():
    try:
        rt = B.asan_runtime()
    except FileNotFoundError as e:
        pytest.skip(str(e))
    lib = _sanitized_lib()
    env = dict(os.environ, LD_PRELOAD=str(rt), SEEDPLANE_HIP_LIB=str(lib),
               ASAN_OPTIONS='detect_leaks=0:halt_on_error=1:abort_on_error=1',
               UBSAN_OPTIONS='halt_on_error=1:print_stacktrace=1')
    r = subprocess.run([sys.executable, '-m', 'pytest', '-q', '-p', 'no:cacheprovider', '-m', 'not gpu',
                        str(ROOT / 'tests' / 'test_capi.py'), str(ROOT / 'tests' / 'test_pack_layout.py')],
                       cwd=str(ROOT), env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout or '')[-3000:] + (r.stderr or '')[-3000:]
    assert r.returncode == 0, tail
    assert 'ERROR: AddressSanitizer' not in tail and 'runtime error' not in tail, tail
    assert ' passed' in r.stdout
