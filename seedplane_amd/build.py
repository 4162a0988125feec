"""Build libseedplane_hip.so in-tree with hipcc for gfx950.

    python -m seedplane_amd.build
"""
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
SRC = PKG / 'csrc' / 'sp_engine.hip'
OUT = PKG / 'libseedplane_hip.so'
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')

FLAGS = ['--offload-arch=gfx950', '-O3', '-std=c++17', '-shared', '-fPIC',
         # packed fp32 instructions stay off (hipcc -O3 would otherwise form v_pk_* fp32 ops)
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
         '-Wno-pass-failed']


def build(verbose=False):
    tmp = OUT.with_suffix('.so.tmp')
    cmd = [HIPCC, *FLAGS, '-o', str(tmp), str(SRC)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = '\n'.join(l for l in (r.stderr or '').splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f'hipcc failed ({r.returncode}):\n{err}')
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == '__main__':
    print(build(verbose=True))
