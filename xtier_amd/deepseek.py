"""DeepSeek V4 sparse-attention hooks over this library's sparse MLA (xtier/packs/deepseek_v4/sparse_mla.py:220-236,
registered as in xtier/packs/deepseek_v4/__init__.py:89-90, :491-494).

flash_mla_with_kvcache takes the backend's sparse FP8 calls on DeepSeek V4 pages ([pages, page_size, 1, 584]: 448
E4M3 values with UE8M0 scales per 64, then 64 BF16 rope values) and leaves every other call to ``original``, with the
reference's conditions; no_sparse_prefill keeps prefill on the paged caches.
"""
from . import ops

FLASH_MLA = 'sglang.kernels.ops.attention.flash_mla_interface.flash_mla_with_kvcache'
SPARSE_PREFILL = 'sglang.srt.layers.attention.deepseek_v4_backend.DeepseekV4AttnBackend._use_sparse_prefill'
DIM = 512


def flash_mla_with_kvcache(original, *args, **kwargs):
    """AROUND flash_mla_interface.flash_mla_with_kvcache (sparse_mla.py:220-231): keyword calls with indices on an
    FP8 V4 cache and head_dim_v 512 run ops.sparse_mla; anything else calls ``original``."""
    cache = kwargs.get('k_cache')
    if (args or kwargs.get('indices') is None or not kwargs.get('is_fp8_kvcache') or cache is None
            or not ops.is_v4_cache(cache) or kwargs.get('head_dim_v', DIM) != DIM):
        return original(*args, **kwargs)
    scale = kwargs.get('softmax_scale')
    q = kwargs['q']
    return ops.sparse_mla(q, cache, kwargs['indices'], kwargs.get('topk_length'), kwargs.get('attn_sink'),
                          scale if scale is not None else q.shape[-1] ** -0.5, kwargs.get('extra_k_cache'),
                          kwargs.get('extra_indices_in_kvcache'), kwargs.get('extra_topk_length'))


def no_sparse_prefill(original, self, *args, **kwargs):
    """AROUND DeepseekV4AttnBackend._use_sparse_prefill (sparse_mla.py:234-236): prefill stays on the paged caches."""
    return False


def install(registry, hook_type):
    """Registers both hooks AROUND their targets (the reference registers them below SM90; here on every GPU)."""
    registry.register(FLASH_MLA, flash_mla_with_kvcache, hook_type.AROUND)
    registry.register(SPARSE_PREFILL, no_sparse_prefill, hook_type.AROUND)
