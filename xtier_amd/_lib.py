"""ctypes binding of libxtier_amd.so (the C ABI declared in include/xtier_amd.h).

The library is built in-tree by ``python -m xtier_amd.build``; loading fails loudly when it is missing, and nothing in
this package falls back to another implementation.
"""
import ctypes
import re
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / 'libxtier_amd.so'
HEADER = Path(__file__).resolve().parent.parent / 'include' / 'xtier_amd.h'

XT_OK, XT_EINVAL, XT_EUNSUPPORTED, XT_ELAUNCH, XT_EWORKSPACE = 0, -1, -2, -3, -4
XT_DTYPE_BF16, XT_DTYPE_F16 = 0, 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_Z = ctypes.c_size_t



class KvStore(ctypes.Structure):
    """xt_kv_store: one tensor of a fused KV append (strides of the source in elements, of the pool in bytes)."""
    _fields_ = [('src', _P), ('src_row_stride', _L), ('src_head_stride', _L), ('heads', _I), ('dim', _I),
                ('g', _P), ('pay', _P), ('scales', _P), ('pay_page_stride', _L), ('pay_row_stride', _L),
                ('pay_head_stride', _L), ('sf_page_stride', _L), ('sf_row_stride', _L), ('sf_head_stride', _L)]


class MlaCache(ctypes.Structure):
    """xt_mla_cache: one NVFP4 latent + BF16 rope cache (strides in bytes, 0 = packed)."""
    _fields_ = [('pay', _P), ('scales', _P), ('rope', _P), ('g', _P), ('slots', _L), ('pay_stride', _L),
                ('sf_stride', _L), ('rope_stride', _L)]


class MlaKeys(ctypes.Structure):
    """xt_mla_keys: a key list (slots, -1 none) with an optional per-row length."""
    _fields_ = [('indices', _P), ('stride', _L), ('topk', _I), ('lengths', _P)]


class MlaFp8Cache(ctypes.Structure):
    """xt_mla_fp8_cache: DeepSeek V4 FP8 pages (page stride in bytes)."""
    _fields_ = [('pages', _P), ('num_pages', _L), ('page_size', _I), ('page_stride', _L)]


_CP, _KP, _FP = ctypes.POINTER(MlaCache), ctypes.POINTER(MlaKeys), ctypes.POINTER(MlaFp8Cache)
_SP = ctypes.POINTER(KvStore)

SIGNATURES = {
    'xt_version': (_I, []),
    'xt_last_error': (ctypes.c_char_p, []),
    'xt_nvfp4_global_scale': (_I, [_P, _L, _I, _I, _L, _L, _P, _P, _P]),
    'xt_nvfp4_quantize_append': (_I, [_P, _L, _I, _I, _L, _L, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _P]),
    'xt_nvfp4_store_kv': (_I, [_SP, _I, _L, _P, _L, _I, _I, _P]),
    'xt_qsa_gather_nvfp4': (_I, [_P, _P, _P, _P, _P, _P, _L, _I, _I, _P, _L, _P, _P, _L, _P, _P, _P, _P, _I, _I, _I,
                                 _I, _P]),
    'xt_qsa_pack_nvfp4': (_I, [_P, _P, _P, _P, _P, _P, _L, _I, _I, _P, _L, _L, _P, _I, _P, _I, _P, _P, _I, _P]),
    'xt_qsa_gather_fp8': (_I, [_P, _P, _L, _I, _I, _P, _L, _P, _P, _L, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    'xt_qsa_pack_fp8': (_I, [_P, _P, _L, _I, _I, _P, _L, _L, _P, _I, _P, _I, _P, _P, _I, _P]),
    'xt_qsa_valid_counts': (_I, [_P, _P, _L, _I, _I, _P, _P, _P]),
    'xt_sparse_decode_workspace_bytes': (_Z, [_I, _I, _I, _I]),
    'xt_sparse_decode_nvfp4': (_I, [_P, _L, _L, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _I, _P, _L, _I, _P,
                                    _P, _L, _I, _P, _P, _P, _F, _P, _L, _L, _I, _P, _I, _I, _P, _Z, _P]),
    'xt_sparse_decode_nvfp4_static': (_I, [_P, _L, _L, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _I, _P, _L,
                                           _I, _P, _P, _L, _I, _P, _P, _P, _F, _P, _L, _L, _I, _P, _I, _I, _P]),
    'xt_block_sparse_decode_nvfp4': (_I, [_P, _L, _L, _P, _P, _P, _P, _F, _L, _I, _I, _I, _I, _L, _L, _L, _L, _L, _L,
                                          _P, _L, _I, _P, _P, _L, _L, _I, _P, _F, _P, _L, _L, _I, _P, _I, _I, _P, _Z,
                                          _P]),
    'xt_block_sparse_prefill_nvfp4': (_I, [_P, _L, _L, _P, _P, _P, _P, _F, _L, _I, _I, _I, _I, _L, _L, _L, _L, _L,
                                           _L, _P, _L, _P, _P, _P, _P, _L, _L, _I, _P, _F, _P, _L, _L, _I, _P, _I,
                                           _I, _P, _Z, _P]),
    'xt_dequantize_context_nvfp4': (_I, [_P, _P, _L, _I, _I, _I, _L, _L, _L, _L, _L, _L, _P, _L, _P, _P, _I, _I, _P,
                                         _P]),
    'xt_varlen_decode_workspace_bytes': (_Z, [_I, _I, _I, _I]),
    'xt_varlen_decode_bf16': (_I, [_P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _P, _I, _I, _I, _I, _I, _F, _P, _L, _L, _I,
                                   _I, _P, _Z, _P]),
    'xt_sparse_mla_workspace_bytes': (_Z, [_I, _I, _I]),
    'xt_sparse_mla_fp8_workspace_bytes': (_Z, [_I, _I, _I]),
    'xt_sparse_mla_max_split_keys': (_I, [_I]),
    'xt_selftest_conversions_bytes': (_Z, []),
    'xt_selftest_conversions': (_I, [_P, _P]),
    'xt_ceiling_mfma': (_I, [_P, ctypes.c_int, ctypes.c_int, _P]),
    'xt_clock_probe': (_I, [_P, ctypes.c_int, _P]),
    'xt_decode_timeline': (_I, [_P, _Z]),
    'xt_mla_timeline': (_I, [_P, _Z]),
    'xt_ceiling_launch': (_I, [ctypes.c_int, _P]),
    'xt_ceiling_split_merge': (_I, [_P, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]),
    'xt_qsa_indexer_logits': (_I, [_P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P,
                                   ctypes.c_int64, ctypes.c_int, _P, _P, ctypes.c_float, ctypes.c_int, _P,
                                   ctypes.c_int64, _P]),
    'xt_dsa_mqa_logits': (_I, [_P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P,
                               ctypes.c_int64, _P, ctypes.c_int, _P, ctypes.c_int64, _P, _P, ctypes.c_int, _P,
                               ctypes.c_int64, _P]),
    'xt_dsa_paged_mqa_logits': (_I, [_P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P,
                                     ctypes.c_int64, ctypes.c_int64, ctypes.c_int, _P, ctypes.c_int64, ctypes.c_int, _P, _P,
                                     ctypes.c_int64, ctypes.c_int, ctypes.c_int, _P, ctypes.c_int64, _P]),
    'xt_topk_rows': (_I, [_P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P, ctypes.c_int64, _P]),
    'xt_minimax_decode_scores': (_I, [_P, _L, _L, _I, _I, _I, _I, _P, _L, _L, _P, _L, _L, _L, _P, _L, _P, _P, _I, _I,
                                      ctypes.c_float, _I, _I, _I, _I, _P, _I, _L, _L, _L, _I, _P]),
    'xt_minimax_prefill_scores': (_I, [_P, _L, _L, _I, _I, _I, _I, _I, _P, _L, _L, _P, _L, _L, _L, _P, _L, _P, _P, _P,
                                       _P, _I, _I, ctypes.c_float, _P, _I, _L, _L, _L, _P]),
    'xt_ceiling_gather': (_I, [_P, ctypes.c_int64, ctypes.c_int64, _P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, _P,
                               ctypes.c_int, ctypes.c_int, _P, _P]),
    'xt_ceiling_gather_sink_words': (_Z, [ctypes.c_int, ctypes.c_int]),
    'xt_ceiling_gather_pieces': (_I, [_P, _L, _P, _L, _I, _I, _P, _I, _I, _I, _I, _P, _P]),
    'xt_sparse_mla_fp8': (_I, [_P, _L, _L, _I, _FP, _KP, _FP, _KP, _P, _F, _P, _L, _L, _I, _P, _I, _I, _P, _Z, _P]),
    'xt_sparse_mla_nvfp4': (_I, [_P, _L, _L, _I, _I, _I, _CP, _KP, _CP, _KP, _P, _F, _P, _L, _L, _I, _P, _I, _I, _P,
                                 _Z, _P]),
}

_lock = threading.Lock()
_lib = None


class XTierError(RuntimeError):
    """A launch or runtime failure reported by the library."""


def declared_symbols():
    """Names of the functions include/xtier_amd.h declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r'^\s*(?:const\s+)?[\w\s\*]*?\b(xt_\w+)\s*\(', text, re.M)))


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise ImportError(f'{LIB_PATH} is missing: build it with `python -m xtier_amd.build` '
                                      '(no other implementation is used)')
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def check(status, what):
    """Raises the reference's exception type for a negative status (ValueError for bad layouts,
    NotImplementedError for unsupported shapes, XTierError otherwise)."""
    if status == XT_OK:
        return
    msg = lib().xt_last_error().decode(errors='replace') or f'{what} failed with status {status}'
    if status == XT_EINVAL or status == XT_EWORKSPACE:
        raise ValueError(msg)
    if status == XT_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise XTierError(msg)
