"""The C ABI library without a GPU: it loads, exports every function include/xtier_amd.h declares, and rejects bad
arguments on the host before any device work (status codes and messages)."""
import ctypes

import pytest

from xtier_amd import _lib


@pytest.fixture(scope='module')
def lib():
    return _lib.lib()


def test_exports_every_declared_symbol(lib):
    names = _lib.declared_symbols()
    assert len(names) >= 8
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES)


def test_version(lib):
    assert lib.xt_version() >= 100


def _decode(lib, **kw):
    args = dict(q=1 << 20, q_rs=4096, q_hs=128, k_pay=1 << 20, v_pay=1 << 20, k_sf=1 << 20, v_sf=1 << 20,
                gk=1 << 20, gv=1 << 20, pool_slots=1024, pay_stride=0, sf_stride=0, pay_hs=0, sf_hs=0, kv_heads=4,
                q_heads=32, dim=128,
                table=1 << 20, table_stride=512, page_size=64, row_req=None, indices=1 << 20, idx_stride=2048, topk=2048,
                counts=None, seq_lens=1 << 20, query_pos=None, scale=0.088, out=1 << 20, o_rs=4096, o_hs=128,
                out_dtype=0, lse=None, rows=32, splits=8, ws=1 << 20, ws_bytes=1 << 30, stream=None)
    args.update(kw)
    return lib.xt_sparse_decode_nvfp4(*args.values())


def test_decode_rejects_bad_shapes_on_host(lib):
    assert _decode(lib, dim=96) == _lib.XT_EUNSUPPORTED
    assert b'head size 96' in lib.xt_last_error()
    assert _decode(lib, q_heads=30) == _lib.XT_EINVAL
    assert _decode(lib, q_heads=128) == _lib.XT_EUNSUPPORTED          # group 32 > 16
    assert _decode(lib, splits=0) == _lib.XT_EINVAL
    assert _decode(lib, q=None) == _lib.XT_EINVAL
    assert _decode(lib, q=(1 << 20) + 2) == _lib.XT_EINVAL            # misaligned rows
    assert _decode(lib, ws_bytes=16) == _lib.XT_EWORKSPACE
    assert _decode(lib, pay_stride=200) == _lib.XT_EINVAL              # not a multiple of 16 / too small
    assert _decode(lib, pay_hs=32) == _lib.XT_EINVAL                   # head rows overlap
    assert _decode(lib, pay_stride=576, sf_stride=576, pay_hs=72, sf_hs=16) == _lib.XT_EINVAL   # head stride % 16
    assert _decode(lib, rows=0) == _lib.XT_OK                          # nothing to do, no launch


def test_workspace_query(lib):
    need = lib.xt_sparse_decode_workspace_bytes(32, 32, 128, 8)
    assert need >= 32 * 8 * 32 * 130 * 4
    assert lib.xt_sparse_decode_workspace_bytes(-1, 32, 128, 8) == 0


def test_quantize_and_gather_reject_bad_layouts(lib):
    assert lib.xt_nvfp4_quantize_append(1 << 20, 4, 4, 100, 400, 100, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 64, 0, 0,
                                        0, 0, 1, None) == _lib.XT_EINVAL
    # head rows 8-byte aligned and not overlapping
    assert lib.xt_nvfp4_quantize_append(1 << 20, 4, 4, 128, 512, 128, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 64, 576,
                                        576, 60, 16, 1, None) == _lib.XT_EINVAL
    assert lib.xt_nvfp4_quantize_append(1 << 20, 4, 4, 128, 512, 128, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 64, 400,
                                        576, 128, 16, 1, None) == _lib.XT_EINVAL
    assert lib.xt_nvfp4_global_scale(1 << 20, 4, 4, 128, 512, 128, None, 1 << 20, None) == _lib.XT_EINVAL
    # non-power-of-2 head size: the reference's ValueError
    st = lib.xt_qsa_gather_nvfp4(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 64, 2, 96, 1 << 20, 10,
                                 1 << 20, 1 << 20, 10, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 0, 1, 10, 0, None)
    assert st == _lib.XT_EINVAL
    with pytest.raises(ValueError, match='power-of-2 head size'):
        _lib.check(st, 'gather')
    with pytest.raises(NotImplementedError):
        _lib.check(_decode(lib, dim=512), 'decode')
    assert isinstance(lib.xt_last_error(), bytes) and ctypes.sizeof(ctypes.c_void_p) == 8


def test_ceilings_reject_bad_arguments_on_host(lib):
    assert lib.xt_ceiling_launch(0, None) == _lib.XT_EINVAL
    merge = lib.xt_ceiling_split_merge
    assert merge(1 << 20, 4224, 1 << 20, 1 << 20, 3, 255, 0, None) == _lib.XT_EINVAL      # splits 2, 4 or 8
    assert merge(1 << 20, 4224, 1 << 20, 1 << 20, 2, 255, 0, None) == _lib.XT_EINVAL      # blocks % splits
    assert merge(1 << 20, 4220, 1 << 20, 1 << 20, 2, 256, 0, None) == _lib.XT_EINVAL      # bytes % 16
    assert merge(None, 4224, 1 << 20, 1 << 20, 2, 256, 0, None) == _lib.XT_EINVAL
    assert merge((1 << 20) + 8, 4224, 1 << 20, 1 << 20, 2, 256, 0, None) == _lib.XT_EINVAL   # part alignment
