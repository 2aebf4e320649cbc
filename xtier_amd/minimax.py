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

The pool: ``kv_pool``, AROUND SGLang's builder of the MiniMax sparse KV pool (minimax_m3/__init__.py:93-100), calls
both on an NVFP4 main pool as it is built. ``install`` registers it and the op hooks unless XTIER_MINIMAX_KV_FP4=0
(minimax_m3/__init__.py:176-181), the reference's switch for the NVFP4 KV cache.

The prefill entry: while BF16 copies of every request's context (main K, V and index K) fit in
``XTIER_MINIMAX_FP4_PREFILL_GB`` GiB (default 1.5), ``dequantize_context`` makes them and ``original`` runs SGLang's
BF16 kernels on the copies through a request-local token table; beyond that ``original`` gets the NVFP4 views and
the prefill-op hook below serves it.
"""
import logging
import math
import os
import sys

import torch

from . import ops

logger = logging.getLogger(__name__)
OPS = 'sglang.srt.layers.attention.minimax_sparse_ops.minimax_sparse'
KV_POOL = 'sglang.srt.mem_cache.kv_cache_configurator.KVCacheConfigurator._build_minimax_sparse_kv_pool'
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


class _DecodeScores:
    """Takes the place of SGLang's _decode_score_kernel for one flash_decode_with_topk_idx call: ``kernel[grid](...)``
    with that kernel's launch arguments (the argument list the shim of kv_fp4.py:225-244 receives) runs
    xt_minimax_decode_scores on the NVFP4 index pool. The BF16 cache SGLang was handed is a shape-only stand-in."""

    def __init__(self, pay, sc):
        self.pay, self.sc = pay, sc

    def __getitem__(self, grid):
        def launch(q, _k, req_to_token, score, seq_lens, slot_ids, _max_slots, batch_size, gqa_group_size, _head_dim,
                   block_size, topk, sm_scale, k_scale, init_blocks, local_blocks, sq0, sq1, sq2, _sk0, _sk1, _sk2,
                   sr0, ss0, ss1, ss2, NUM_KV_CHUNKS=1, SCORE_TYPE='max', SKIP_TRIVIAL_TOPK_SCORE=False,
                   IS_FP8=False, **_):
            if IS_FP8:
                raise NotImplementedError('xtier_amd.minimax: the NVFP4 index scores read no FP8 index cache')
            g = grid({'NUM_KV_CHUNKS': NUM_KV_CHUNKS}) if callable(grid) else grid
            ops.minimax_decode_scores(q, self.pay, self.sc, req_to_token, score, seq_lens, slot_ids, block_size,
                                      sm_scale, k_scale, init_blocks, local_blocks, SCORE_TYPE,
                                      skip_topk=topk if SKIP_TRIVIAL_TOPK_SCORE else None,
                                      heads=g[1] * gqa_group_size, batch=batch_size, q_strides=(sq0, sq1, sq2),
                                      r2t_stride=sr0, score_strides=(ss0, ss1, ss2))
        return launch


class _PrefillScores:
    """Takes the place of SGLang's _flash_attn_fwd_with_block_score_kernel for one flash_prefill_with_topk_index call
    (score only: no index value, no sink, no output; the argument list of the shim at kv_fp4.py:449-472): runs
    xt_minimax_prefill_scores on the NVFP4 index pool, 64 query rows per grid row as that kernel's grid counts."""

    BLOCK_Q = 64

    def __init__(self, pay, sc):
        self.pay, self.sc = pay, sc

    def __getitem__(self, grid):
        def launch(q, _k, _v, sink, o, score, req_to_token, cu_seqlens, seq_lens, prefix_lens, slot_ids, _max_slots,
                   num_heads, _gqa_group_size, _qk_head_dim, _v_head_dim, block_size_k, sm_scale, k_scale, _v_scale,
                   _gumbel, _one, sq0, sq1, sq2, *rest, SCORE_TYPE='max', DISABLE_INDEX_VALUE=True, IS_FP8=False,
                   **_):
            if IS_FP8 or not DISABLE_INDEX_VALUE or SCORE_TYPE != 'max' or sink is not None or o is not None:
                raise NotImplementedError('xtier_amd.minimax: the NVFP4 prefill index scores compute the max score '
                                          'only (no index value, sink or FP8 index cache)')
            ss0, ss1, ss2, sr0 = rest[-4:]
            g = grid({'BLOCK_SIZE_Q': self.BLOCK_Q}) if callable(grid) else grid
            ops.minimax_prefill_scores(q, self.pay, self.sc, req_to_token, score, cu_seqlens, seq_lens, prefix_lens,
                                       slot_ids, block_size_k, sm_scale, k_scale, max_q_len=g[0] * self.BLOCK_Q,
                                       heads=num_heads, q_strides=(sq0, sq1, sq2), r2t_stride=sr0,
                                       score_strides=(ss0, ss1, ss2))
        return launch


def _run_with_scores(run, kernel_name, scores, q, pay, kwargs):
    """Calls SGLang's ``run`` (its own chunking, score buffer and top-k) with ``kernel_name`` of its module replaced by
    ``scores`` for the call, and a shape-only BF16 stand-in of the index cache [slots, 1, dim]."""
    module = sys.modules[run.__module__]
    stand_in = torch.empty((1, 1, 1), dtype=q.dtype, device=q.device).expand(pay.shape[0] * pay.shape[1], 1,
                                                                                pay.shape[2] * 2)
    kept = getattr(module, kernel_name)
    setattr(module, kernel_name, scores)
    try:
        return run(q=q, k_cache=stand_in, **kwargs)
    finally:
        setattr(module, kernel_name, kept)


def _index_call(kwargs, what):
    if not kwargs.get('disable_index_value') or kwargs.get('sink') is not None:
        raise NotImplementedError(f'xtier_amd.minimax: {what} on the NVFP4 index cache computes scores only '
                                  '(disable_index_value, no sink)')
    q, pay = kwargs.pop('q'), kwargs.pop('k_cache')
    return q, pay


def decode_topk(original, *args, **kwargs):
    """AROUND flash_decode_with_topk_idx (kv_fp4.py:572-576, :247-265): on a tagged index cache, SGLang's own call
    with the index scores from xt_minimax_decode_scores; ``original`` untouched otherwise."""
    sc = scales_of(kwargs.get('k_cache'))
    if sc is None:
        return original(*args, **kwargs)
    q, pay = _index_call(kwargs, 'flash_decode_with_topk_idx')
    return _run_with_scores(original, '_decode_score_kernel', _DecodeScores(pay, sc), q, pay, kwargs)


def prefill_topk(original, *args, **kwargs):
    """AROUND flash_prefill_with_topk_index (kv_fp4.py:593-598, :475-494): as ``decode_topk``, with the prefill
    scores from xt_minimax_prefill_scores."""
    sc = scales_of(kwargs.get('k_cache'))
    if sc is None:
        return original(*args, **kwargs)
    q, pay = _index_call(kwargs, 'flash_prefill_with_topk_index')
    return _run_with_scores(original, '_flash_attn_fwd_with_block_score_kernel', _PrefillScores(pay, sc), q, pay,
                            kwargs)


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


HOOKS = ((f'{OPS}.flash_decode_with_topk_idx', decode_topk),
         (f'{OPS}.flash_decode_with_gqa_share_sparse', decode_main),
         (f'{OPS}.flash_prefill_with_topk_index', prefill_topk),
         (f'{OPS}.flash_prefill_with_gqa_share_sparse', prefill_main),
         (f'{OPS}.minimax_sparse_prefill', sparse_prefill),
         (STORE, store_kv_index))


def kv_pool(original, *args, **kwargs):
    """AROUND KVCacheConfigurator._build_minimax_sparse_kv_pool (minimax_m3/__init__.py:93-100): the pool as SGLang
    builds it; when its main pool is the NVFP4 MSA-v1 pool, its payload views are tagged with their scale views
    (attach_scales) and its stores go through the one-launch store (enable_fused_store). Any other pool is returned
    untouched."""
    pool = original(*args, **kwargs)
    if getattr(getattr(pool, 'main_pool', None), 'is_minimax_m3_nvfp4_main', False):
        attach_scales(pool)
        enable_fused_store(pool)
    return pool


def kv_fp4_enabled():
    """The reference's switch for the NVFP4 KV cache (minimax_m3/__init__.py:67-68): on unless XTIER_MINIMAX_KV_FP4=0."""
    return os.environ.get('XTIER_MINIMAX_KV_FP4', '1') != '0'


def install(registry, hook_type):
    """Unless XTIER_MINIMAX_KV_FP4=0 (minimax_m3/__init__.py:176-181): the pool hook, then every hook of HOOKS AROUND
    its target (SGLang's generic MiniMax sparse ops, kv_fp4.py:632-638, and its fused NVFP4 store)."""
    if not kv_fp4_enabled():
        return
    registry.register(KV_POOL, kv_pool, hook_type.AROUND)
    for target, hook in HOOKS:
        registry.register(target, hook, hook_type.AROUND)
