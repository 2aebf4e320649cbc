"""Builds libxtier_amd.so from the HIP sources under csrc/ for gfx950 (hipcc cross-compiles; no GPU needed).

    python -m xtier_amd.build [--verbose]

Objects go to xtier_amd/_build/, the library to xtier_amd/libxtier_amd.so (both git-ignored).
"""
import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / 'csrc'
BUILD = PKG / '_build'
LIB = PKG / 'libxtier_amd.so'
ARCH = 'gfx950'
# Packed FP32 VALU instructions are kept out of the device code: the compiler would otherwise form them from float2
# arithmetic, and this hardware pool has produced silently wrong results with some of their forms.
DEVICE_FLAGS = ['-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops']
COMMON = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}', '-Wall', '-Wno-unused-function',
          '-Wno-unknown-pragmas']


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found: the HIP toolchain (ROCm) is required to build xtier_amd')
    return path


def _compile(src, verbose):
    obj = BUILD / (src.stem + '.o')
    cmd = [hipcc(), *COMMON, *DEVICE_FLAGS, '-c', str(src), '-o', str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the device feature flag; that warning is expected and dropped
    err = '\n'.join(l for l in r.stderr.splitlines() if 'packed-fp32-ops' not in l)
    if r.returncode != 0:
        raise RuntimeError(f'compiling {src.name} failed:\n{" ".join(cmd)}\n{err}')
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose=False):
    """Compiles every csrc/*.hip and links libxtier_amd.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob('*.hip'))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'linking failed:\n{" ".join(cmd)}\n{r.stderr}')
    os.replace(tmp, LIB)
    return LIB


if __name__ == '__main__':
    p = argparse.ArgumentParser()
    p.add_argument('--verbose', action='store_true')
    print(build(p.parse_args().verbose))
