"""MiniMax M3.1 sparse attention over an NVFP4 cache of head-major pages (SGLang's MSA-v1 pool), run by this library's
block-sparse kernels through hooks AROUND SGLang's generic MiniMax sparse ops. The hook contract (names, keyword
arguments, which calls fall through, the exception types) is the one of xtier/packs/minimax_m3/kv_fp4.py:533-638.

Recognizing an NVFP4 call: SGLang passes the ops the pool's payload views. ``attach_scales`` tags every layer's main K,
main V and index K payload view with the view of its E4M3 scale bytes; a call whose ``k_cache`` carries the tag runs
here, any other call goes to ``original`` untouched.

What an NVFP4 call must satisfy: the pool is written with outer scales of 1, so a ``k_scale`` / ``v_scale`` other than
1 is a ValueError; these kernels have no attention sink and no HiSparse slot lists (NotImplementedError).

The KV store: ``enable_fused_store`` (kv_fp4.py:546-559) turns on the pool's fused store, and the hook on SGLang's
``nvfp4_store_kv_index`` runs it as one launch of this library's store (main K, V and index K).

The prefill entry: while BF16 copies of every request's context (main K, V and index K) fit in
``XTIER_MINIMAX_FP4_PREFILL_GB`` GiB (default 1.5), ``dequantize_context`` makes them and ``original`` runs SGLang's
BF16 kernels on the copies through a request-local token table; beyond that ``original`` gets the NVFP4 views and
the prefill-op hook below serves it.
"""
import logging
import math
import os

import torch

from . import ops

logger = logging.getLogger(__name__)
OPS = 'sglang.srt.layers.attention.minimax_sparse_ops.minimax_sparse'
PAGE = 128                    # tokens per page of the MSA-v1 pool
TAG = '_xt_nvfp4_scales'      # attribute of a payload view that holds its scale-byte view
PREFILL_GB = float(os.environ.get('XTIER_MINIMAX_FP4_PREFILL_GB', '1.5'))


def _payload_scale_pairs(pool):
    main, index = pool.main_pool, pool.index_k_pool
    yield from zip(main.k_buffer, main.k_scale_buffer)
    yield from zip(main.v_buffer, main.v_scale_buffer)
    yield from zip(index.k_buffer, index.k_scale_buffer)


def attach_scales(pool):
    """Tags each layer's payload views of the pool (main K, main V, index K, kv_fp4.py:533-545) with their scale-byte
    views, which routes the sparse ops on them to the NVFP4 kernels."""
    tagged = 0
    for pay, sc in _payload_scale_pairs(pool):
        setattr(pay, TAG, sc)
        tagged += 1
    logger.info('xtier_amd: %d NVFP4 payload views of the MiniMax pool (%s tokens) go to the block-sparse kernels',
                tagged, getattr(pool, 'size', '?'))


def scales_of(view):
    """The scale-byte view a payload view was tagged with, or None (not an NVFP4 view)."""
    return getattr(view, TAG, None)


def _check_unit_scales(kwargs):
    for name in ('k_scale', 'v_scale'):
        value = kwargs.get(name)
        if value is not None and value != 1.0:
            raise ValueError(f'xtier_amd.minimax: {name}={value}, but NVFP4 pages are stored with an outer scale of 1')


def decode_main(original, *args, **kwargs):
    """AROUND flash_decode_with_gqa_share_sparse (kv_fp4.py:579-590): the NVFP4 block-sparse decode on a tagged
    k_cache, ``original`` otherwise."""
    k_sc = scales_of(kwargs.get('k_cache'))
    if k_sc is None:
        return original(*args, **kwargs)
    _check_unit_scales(kwargs)
    missing = [name for name in ('sink', 'hisparse_slots') if kwargs.get(name) is not None]
    if missing:
        raise NotImplementedError(f'xtier_amd.minimax: the NVFP4 block-sparse decode takes no {" / ".join(missing)}')
    q, v = kwargs['q'], kwargs['v_cache']
    base = kwargs.get('sm_scale')
    sm_scale = (q.shape[-1] ** -0.5 if base is None else base) * (kwargs.get('q_scale') or 1.0)
    return ops.fp4_sparse_decode(q, kwargs['k_cache'], k_sc, v, scales_of(v), kwargs['req_to_token'],
                                 kwargs['slot_ids'], kwargs['topk_idx'], kwargs['seq_lens'], kwargs['block_size'],
                                 sm_scale=sm_scale)


def prefill_main(original, *args, **kwargs):
    """AROUND flash_prefill_with_gqa_share_sparse (kv_fp4.py:593-598): the NVFP4 causal block-sparse prefill on a
    tagged k_cache, ``original`` otherwise."""
    k_sc = scales_of(kwargs.get('k_cache'))
    if k_sc is None:
        return original(*args, **kwargs)
    _check_unit_scales(kwargs)
    return ops.fp4_prefill_gqa_share_sparse(**kwargs, k_sc=k_sc, v_sc=scales_of(kwargs['v_cache']))


def _copy_rows(k_cache, idx_k_cache, idx_v_cache, slot_ids, max_seqlen_k, kwargs):
    """Rows per request of the BF16 context copies, or None when the call stays on the NVFP4 views: an untagged
    cache, a separate index V cache or a loc_mapping (forms the copy does not cover), or copies over the budget."""
    if scales_of(k_cache) is None or idx_v_cache is not None or kwargs.get('loc_mapping') is not None:
        return None
    rows = PAGE * math.ceil(int(max_seqlen_k) / PAGE)
    main_values = 2 * k_cache.shape[1] * (2 * k_cache.shape[3])     # K and V: heads x head size per position
    index_values = 2 * idx_k_cache.shape[2]                          # the index K head per position
    copy_bytes = slot_ids.shape[0] * rows * (main_values + index_values) * 2
    return rows if copy_bytes <= PREFILL_GB * 2 ** 30 else None


def sparse_prefill(original, q, k_cache, v_cache, sink, idx_q, idx_k_cache, idx_v_cache, idx_sink, req_to_token,
                   slot_ids, cu_seqlens, seq_lens, prefix_lens, max_seqlen_q, max_seqlen_k, *args, **kwargs):
    """AROUND minimax_sparse_prefill (kv_fp4.py:601-629): SGLang's BF16 prefill on dequantized copies of the
    contexts while they fit the budget, else ``original`` on the NVFP4 views."""
    rows = _copy_rows(k_cache, idx_k_cache, idx_v_cache, slot_ids, max_seqlen_k, kwargs)
    if rows is None:
        return original(q, k_cache, v_cache, sink, idx_q, idx_k_cache, idx_v_cache, idx_sink, req_to_token, slot_ids,
                        cu_seqlens, seq_lens, prefix_lens, max_seqlen_q, max_seqlen_k, *args, **kwargs)
    batch = slot_ids.shape[0]
    copies = [ops.dequantize_context(c, scales_of(c), req_to_token, slot_ids, seq_lens, rows)
              for c in (k_cache, v_cache, idx_k_cache)]
    # request b's positions sit on copy rows b * rows .. b * rows + rows - 1
    local_table = torch.arange(batch * rows, dtype=torch.int32, device=k_cache.device).view(batch, rows)
    local_ids = torch.arange(batch, dtype=torch.int32, device=k_cache.device)
    return original(q, copies[0], copies[1], sink, idx_q, copies[2], None, idx_sink, local_table, local_ids,
                    cu_seqlens, seq_lens, prefix_lens, max_seqlen_q, max_seqlen_k, *args, **kwargs)


STORE = 'sglang.kernels.ops.kvcache.nvfp4_store_kv_index.nvfp4_store_kv_index'


def store_kv_index(original, k, v, ik, kpay, ksc, vpay, vsc, ipay, isc, loc, global_scale, page_size=PAGE,
                   **kwargs):
    """AROUND SGLang's fused MiniMax NVFP4 store (called as tests/minimax_kv_fp4_check.py:173 calls it): main K, V
    and index K quantized into their head-major pages in one launch of this library's store, ``original`` for
    anything else (CPU tensors, extra options)."""
    if kwargs or not (torch.is_tensor(k) and k.is_cuda):
        return original(k, v, ik, kpay, ksc, vpay, vsc, ipay, isc, loc, global_scale, page_size=page_size, **kwargs)
    ops.nvfp4_store_kv_index(k, v, ik, kpay, ksc, vpay, vsc, ipay, isc, loc, global_scale, page_size=page_size)


def enable_fused_store(pool):
    """kv_fp4.py:546-559: the pool writes K, V and the index K through the one-launch store (the hook above) instead
    of quantizing each buffer and scattering it. Taken when not disabled (XTIER_MINIMAX_FP4_FUSED_STORE=0), not
    already on, and the main and index pools share head size, page size and global scale. Returns whether it is on."""
    main, index = pool.main_pool, pool.index_k_pool
    if os.environ.get('XTIER_MINIMAX_FP4_FUSED_STORE', '1') == '0':
        return bool(pool.use_nvfp4_fused_quantize_store)
    compatible = (main.head_dim == index.INDEX_HEAD_DIM and main.page_size == index.page_size
                  and torch.equal(main.global_scale, index.global_scale))
    if compatible and not pool.use_nvfp4_fused_quantize_store:
        pool.use_nvfp4_fused_quantize_store = True
        logger.info('xtier_amd: MiniMax NVFP4 KV store through the one-launch K / V / index K store')
    return bool(pool.use_nvfp4_fused_quantize_store)


HOOKS = ((f'{OPS}.flash_decode_with_gqa_share_sparse', decode_main),
         (f'{OPS}.flash_prefill_with_gqa_share_sparse', prefill_main),
         (f'{OPS}.minimax_sparse_prefill', sparse_prefill),
         (STORE, store_kv_index))


def install(registry, hook_type):
    """Registers every hook of HOOKS AROUND its target: SGLang's generic MiniMax sparse ops (kv_fp4.py:632-638) and
    its fused NVFP4 store."""
    for target, hook in HOOKS:
        registry.register(target, hook, hook_type.AROUND)
