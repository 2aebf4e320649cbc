"""MiniMax sparse-attention hooks over an NVFP4 cache of head-major pages (xtier/packs/minimax_m3/kv_fp4.py:533-638),
running the block-sparse decode and prefill of this package.

A layer's payload views (main K, main V, index K) carry their scale bytes as the attribute ``_xtier_fp4``
(``attach_scales``); the decode hook takes the NVFP4 path only for such a view and otherwise calls ``original``. The
pool has unit outer scales: a k_scale / v_scale other than 1 is a ValueError, a sink or HiSparse slots are
NotImplementedError, as in the reference. The main-head decode, the main-head prefill and the sparse-prefill entry are
installed; the top-k indexers stay SGLang's.
"""
import logging
import os

from . import ops

logger = logging.getLogger(__name__)
PAGE = 128
OPS = 'sglang.srt.layers.attention.minimax_sparse_ops.minimax_sparse'
PREFILL_GB = float(os.environ.get('XTIER_MINIMAX_FP4_PREFILL_GB', '1.5'))


def attach_scales(pool):
    """kv_fp4.py:533-545: each layer's payload view of the main K, main V and index K buffers gets its scale bytes."""
    main, index = pool.main_pool, pool.index_k_pool
    for pays, scales in ((main.k_buffer, main.k_scale_buffer), (main.v_buffer, main.v_scale_buffer),
                         (index.k_buffer, index.k_scale_buffer)):
        for pay, sc in zip(pays, scales):
            pay._xtier_fp4 = sc
    logger.info('xtier_amd: MiniMax KV cache in NVFP4 (head-major pages, fused block-sparse decode): %d tokens',
                getattr(pool, 'size', -1))


def _scales(t):
    return getattr(t, '_xtier_fp4', None)


def _unit(kwargs, *names):
    for name in names:
        if kwargs.get(name) not in (None, 1.0):
            raise ValueError(f'xtier: the NVFP4 KV cache has unit outer scales, got {name}={kwargs[name]}')


def decode_main(original, *args, **kwargs):
    """AROUND hook of flash_decode_with_gqa_share_sparse (kv_fp4.py:579-590): the block-sparse NVFP4 decode when
    k_cache carries scale bytes, else ``original``."""
    k_sc = _scales(kwargs.get('k_cache'))
    if k_sc is None:
        return original(*args, **kwargs)
    _unit(kwargs, 'k_scale', 'v_scale')
    if kwargs.get('sink') is not None or kwargs.get('hisparse_slots') is not None:
        raise NotImplementedError('xtier: the NVFP4 KV sparse decode has no attention sink or HiSparse')
    q, v = kwargs['q'], kwargs['v_cache']
    sm_scale = kwargs.get('sm_scale')
    sm_scale = (q.shape[-1] ** -0.5 if sm_scale is None else sm_scale) * (kwargs.get('q_scale') or 1.0)
    return ops.fp4_sparse_decode(q, kwargs['k_cache'], k_sc, v, _scales(v), kwargs['req_to_token'],
                                 kwargs['slot_ids'], kwargs['topk_idx'], kwargs['seq_lens'], kwargs['block_size'],
                                 sm_scale=sm_scale)


def prefill_main(original, *args, **kwargs):
    """AROUND hook of flash_prefill_with_gqa_share_sparse (kv_fp4.py:593-598): the block-sparse NVFP4 prefill when
    k_cache carries scale bytes, else ``original``."""
    k_sc = _scales(kwargs.get('k_cache'))
    if k_sc is None:
        return original(*args, **kwargs)
    _unit(kwargs, 'k_scale', 'v_scale')
    return ops.fp4_prefill_gqa_share_sparse(**kwargs, k_sc=k_sc, v_sc=_scales(kwargs['v_cache']))


def sparse_prefill(original, q, k_cache, v_cache, sink, idx_q, idx_k_cache, idx_v_cache, idx_sink, req_to_token,
                   slot_ids, cu_seqlens, seq_lens, prefix_lens, max_seqlen_q, max_seqlen_k, *args, **kwargs):
    """AROUND hook of minimax_sparse_prefill (kv_fp4.py:601-629): on the NVFP4 cache, requests whose BF16 copies
    (main K, V and index K, each request's positions on consecutive rows, a request-local req_to_token) fit in
    XTIER_MINIMAX_FP4_PREFILL_GB run ``original`` on the copies; larger ones run ``original`` on the NVFP4 cache, which
    the prefill_main hook serves."""
    import torch
    if _scales(k_cache) is not None and idx_v_cache is None and kwargs.get('loc_mapping') is None:
        b = slot_ids.shape[0]
        rows = -(-int(max_seqlen_k) // PAGE) * PAGE
        width = 2 * k_cache.shape[1] * 2 * k_cache.shape[3] + 2 * idx_k_cache.shape[2]   # K, V and index K values
        if b * rows * width * 2 <= PREFILL_GB * 2 ** 30:
            dev = k_cache.device
            local = torch.arange(b, dtype=torch.int32, device=dev)
            r2t = local[:, None] * rows + torch.arange(rows, dtype=torch.int32, device=dev)[None, :]
            k, v, ik = (ops.dequantize_context(c, _scales(c), req_to_token, slot_ids, seq_lens, rows)
                        for c in (k_cache, v_cache, idx_k_cache))
            return original(q, k, v, sink, idx_q, ik, None, idx_sink, r2t, local, cu_seqlens, seq_lens, prefix_lens,
                            max_seqlen_q, max_seqlen_k, *args, **kwargs)
    return original(q, k_cache, v_cache, sink, idx_q, idx_k_cache, idx_v_cache, idx_sink, req_to_token, slot_ids,
                    cu_seqlens, seq_lens, prefix_lens, max_seqlen_q, max_seqlen_k, *args, **kwargs)


def install(registry, hook_type):
    """Registers the hooks AROUND SGLang's generic MiniMax sparse ops (kv_fp4.py:632-638): the main-head decode and
    prefill kernels by keyword, the prefill entry positionally."""
    registry.register(f'{OPS}.flash_decode_with_gqa_share_sparse', decode_main, hook_type.AROUND)
    registry.register(f'{OPS}.flash_prefill_with_gqa_share_sparse', prefill_main, hook_type.AROUND)
    registry.register(f'{OPS}.minimax_sparse_prefill', sparse_prefill, hook_type.AROUND)
