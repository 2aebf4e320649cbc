"""MiniMax sparse-decode hook over an NVFP4 cache of head-major pages (xtier/packs/minimax_m3/kv_fp4.py:533-590 and
:632-638), running the block-sparse decode of this package.

A layer's payload views (main K, main V, index K) carry their scale bytes as the attribute ``_xtier_fp4``
(``attach_scales``); the decode hook takes the NVFP4 path only for such a view and otherwise calls ``original``. The
pool has unit outer scales: a k_scale / v_scale other than 1 is a ValueError, a sink or HiSparse slots are
NotImplementedError, as in the reference. Only the main-head decode (SGLang's flash_decode_with_gqa_share_sparse) is
installed; the top-k indexers and the prefill entry points stay SGLang's.
"""
import logging

from . import ops

logger = logging.getLogger(__name__)
PAGE = 128
OPS = 'sglang.srt.layers.attention.minimax_sparse_ops.minimax_sparse'


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


def install(registry, hook_type):
    """Registers decode_main AROUND SGLang's main-head sparse decode (kv_fp4.py:632-638, its decode entry)."""
    registry.register(f'{OPS}.flash_decode_with_gqa_share_sparse', decode_main, hook_type.AROUND)
