"""Build libseedplane_hip.so in-tree with hipcc for gfx950.

    python -m seedplane_amd.build            # the library
    python -m seedplane_amd.build sanitized  # a host-sanitized copy for CPU tests (_build/, not shipped)
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


# Host code only under AddressSanitizer + UndefinedBehaviorSanitizer (-Xarch_host before each -fsanitize=; the gfx950
# code is built as usual).  CPU tests load it through SEEDPLANE_HIP_LIB with the clang ASan runtime preloaded.
SAN_OUT = PKG.parent / '_build' / 'libseedplane_hip_san.so'
SAN_FLAGS = ['--offload-arch=gfx950', '-O1', '-std=c++17', '-shared', '-fPIC',
             '-Xarch_host', '-g', '-Xarch_host', '-fno-omit-frame-pointer',
             '-Xarch_host', '-fsanitize=address', '-Xarch_host', '-fsanitize=undefined',
             '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops', '-Wno-pass-failed']


def asan_runtime():
    """The clang AddressSanitizer runtime that matches hipcc's compiler."""
    found = sorted(Path('/opt/rocm/lib/llvm/lib/clang').glob('*/lib/linux/libclang_rt.asan-x86_64.so'))
    if not found:
        raise FileNotFoundError('clang ASan runtime not found under /opt/rocm/lib/llvm/lib/clang')
    return found[-1]


def build_sanitized(out=SAN_OUT):
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_suffix('.so.tmp')
    r = subprocess.run([HIPCC, *SAN_FLAGS, '-o', str(tmp), str(SRC)], capture_output=True, text=True)
    if r.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = '\n'.join(l for l in (r.stderr or '').splitlines() if noise not in l)
        raise RuntimeError(f'hipcc (sanitized host) failed ({r.returncode}):\n{err}')
    os.replace(tmp, out)
    return out


if __name__ == '__main__':
    print(build_sanitized() if sys.argv[1:] == ['sanitized'] else build(verbose=True))
