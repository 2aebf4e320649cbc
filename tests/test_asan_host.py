"""The C-ABI host shim under AddressSanitizer, without a GPU: the library is rebuilt with ASan on its host code only
(the device code is unchanged; GPU sanitizers are not part of this build), then a subprocess with the ASan runtime
preloaded runs the host-side checks of test_abi, every exported function with all-zero arguments (null pointers,
zero sizes), and calls with valid-looking arguments that travel every host check up to the launch, which fails
without a device. Any heap, stack or global out-of-bounds access on the host aborts the subprocess."""
import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / 'xtier_amd' / 'csrc'


def _asan_runtime():
    found = sorted(glob.glob('/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so'))
    return found[-1] if found else None


@pytest.fixture(scope='module')
def asan_lib(tmp_path_factory):
    hipcc = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(hipcc) or _asan_runtime() is None:
        pytest.skip('hipcc or the clang ASan runtime is not installed')
    out = tmp_path_factory.mktemp('asan')
    flags = ['-O1', '-g', '-std=c++17', '-fPIC', '--offload-arch=gfx950', '-Xclang', '-target-feature', '-Xclang',
             '-packed-fp32-ops', '-Xarch_host', '-fsanitize=address', '-Xarch_host', '-fno-omit-frame-pointer']

    def compile_one(src):
        obj = out / (src.stem + '.o')
        r = subprocess.run([hipcc, *flags, '-c', str(src), '-o', str(obj)], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return str(obj)

    with concurrent.futures.ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(compile_one, sorted(CSRC.glob('*.hip'))))
    lib = out / 'libxtier_amd_asan.so'
    r = subprocess.run([hipcc, '--offload-arch=gfx950', '-shared', '-fPIC', '-Xarch_host', '-fsanitize=address',
                        '-o', str(lib), *objs], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return lib


_SCRIPT = r'''
import ctypes, sys
from pathlib import Path
sys.path.insert(0, sys.argv[2])
from xtier_amd import _lib
_lib.LIB_PATH = Path(sys.argv[1])
lib = _lib.lib()
import tests.test_abi as abi

for name in sorted(dir(abi)):
    if name.startswith('test_'):
        getattr(abi, name)(lib)

# every export with all-zero arguments: a status (or a size), never a host fault
for name, (res, args) in sorted(_lib.SIGNATURES.items()):
    vals = [0.0 if a is ctypes.c_float else None if a is ctypes.c_void_p or hasattr(a, 'contents') else 0
            for a in args]
    getattr(lib, name)(*vals)

# valid-looking calls: every host check passes and the launch reports that there is no device
P = 1 << 20                                   # aligned stand-in device addresses, never dereferenced on the host
ELAUNCH = _lib.XT_ELAUNCH
assert abi._decode(lib) == ELAUNCH, lib.xt_last_error()
assert lib.xt_varlen_decode_bf16(P, 4096, 128, P, 512, 128, P, 512, 128, P, P, 32, 32, 4, 128, 2048, 0.088, P, 4096,
                                 128, 0, 8, P, 1 << 30, None) == ELAUNCH, lib.xt_last_error()
stores = (_lib.KvStore * 2)()
for s in stores:
    s.src, s.src_row_stride, s.src_head_stride, s.heads, s.dim = P, 512, 128, 4, 128
    s.g, s.pay, s.scales = P, P, P
    s.pay_row_stride, s.pay_head_stride, s.sf_row_stride, s.sf_head_stride = 576, 128, 576, 16
assert lib.xt_nvfp4_store_kv(stores, 2, 4096, P, 69632, 1, 1, None) == ELAUNCH, lib.xt_last_error()
assert lib.xt_nvfp4_store_kv(stores, 5, 4096, P, 69632, 1, 1, None) == _lib.XT_EINVAL
cache = _lib.MlaCache(P, P, P, P, 1 << 20, 416, 416, 416)
keys = _lib.MlaKeys(P, 2048, 2048, None)
st = lib.xt_sparse_mla_nvfp4(P, 128 * 576, 576, 128, 512, 64, ctypes.byref(cache), ctypes.byref(keys), None, None,
                             None, 0.04, P, 128 * 512, 512, 0, P, 64, 4, P, 1 << 30, None)
assert st == ELAUNCH, (st, lib.xt_last_error())
assert lib.xt_qsa_gather_nvfp4(P, P, P, P, P, P, 1 << 20, 4, 128, P, 32768, P, P, 2048, P, P, P, P, 0, 32, 2048, 0,
                               None) == ELAUNCH, lib.xt_last_error()
print('asan host checks passed')
'''


def test_host_shim_under_address_sanitizer(asan_lib):
    env = dict(os.environ, LD_PRELOAD=_asan_runtime(), ASAN_OPTIONS='detect_leaks=0:halt_on_error=1:abort_on_error=0',
               HIP_VISIBLE_DEVICES='')
    r = subprocess.run([sys.executable, '-c', _SCRIPT, str(asan_lib), str(ROOT)], capture_output=True, text=True,
                       env=env, timeout=600, cwd=str(ROOT))
    assert r.returncode == 0 and 'asan host checks passed' in r.stdout, (r.stdout[-3000:], r.stderr[-6000:])
    assert 'AddressSanitizer' not in r.stderr, r.stderr[-6000:]
