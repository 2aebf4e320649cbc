"""The MiniMax decode hook without a GPU: fall-through to `original` for caches without scale bytes, the unit-scale and
sink / HiSparse checks (kv_fp4.py:562-590), attach_scales and the registration (:632-638)."""
from types import SimpleNamespace

import pytest
import torch

from xtier_amd import minimax


def _original(*args, **kwargs):
    return ('original', args, kwargs)


def test_falls_through_without_scale_bytes():
    k = torch.zeros(2, 4, 128, 64, dtype=torch.uint8)
    got = minimax.decode_main(_original, 1, q=torch.zeros(1, 16, 128), k_cache=k, v_cache=k)
    assert got[0] == 'original' and got[1] == (1,) and got[2]['k_cache'] is k


def test_unit_scales_and_unsupported_features():
    k = torch.zeros(2, 4, 128, 64, dtype=torch.uint8)
    setattr(k, minimax.TAG, torch.zeros(2, 4, 128, 8, dtype=torch.uint8))
    base = dict(q=torch.zeros(1, 16, 128), k_cache=k, v_cache=k)
    with pytest.raises(ValueError):
        minimax.decode_main(_original, **base, k_scale=0.5)
    with pytest.raises(NotImplementedError):
        minimax.decode_main(_original, **base, sink=torch.zeros(16))
    with pytest.raises(NotImplementedError):
        minimax.decode_main(_original, **base, k_scale=1.0, hisparse_slots=torch.zeros(1))


def test_attach_scales_and_install():
    pays = [torch.zeros(1), torch.zeros(1)]
    scs = [torch.ones(1), torch.ones(1)]
    pool = SimpleNamespace(main_pool=SimpleNamespace(k_buffer=pays, k_scale_buffer=scs, v_buffer=pays[::-1],
                                                     v_scale_buffer=scs[::-1]),
                           index_k_pool=SimpleNamespace(k_buffer=[], k_scale_buffer=[]), size=7)
    minimax.attach_scales(pool)
    assert minimax.scales_of(pays[0]) is scs[0] and minimax.scales_of(pays[1]) is scs[1]
    seen = []
    registry = SimpleNamespace(register=lambda name, fn, kind: seen.append((name, fn, kind)))
    minimax.install(registry, SimpleNamespace(AROUND='around'))
    assert seen == [(f'{minimax.OPS}.flash_decode_with_gqa_share_sparse', minimax.decode_main, 'around'),
                    (f'{minimax.OPS}.flash_prefill_with_gqa_share_sparse', minimax.prefill_main, 'around'),
                    (f'{minimax.OPS}.minimax_sparse_prefill', minimax.sparse_prefill, 'around'),
                    (minimax.STORE, minimax.store_kv_index, 'around')]
    # caches without scale bytes fall through
    assert minimax.prefill_main(_original, k_cache=torch.zeros(1))[0] == 'original'
    got = minimax.sparse_prefill(_original, *range(16), flag=1)
    assert got[0] == 'original' and got[1] == tuple(range(16)) and got[2] == {'flag': 1}


def test_deepseek_hook_falls_through_and_installs():
    from xtier_amd import deepseek
    seen = []
    original = lambda *a, **k: ('original', a, k)
    assert deepseek.flash_mla_with_kvcache(original, 1, k_cache=None)[0] == 'original'          # positional call
    cache = torch.zeros(2, 64, 1, 584, dtype=torch.uint8)
    assert deepseek.flash_mla_with_kvcache(original, k_cache=cache, indices=None, is_fp8_kvcache=True)[0] == 'original'
    assert deepseek.flash_mla_with_kvcache(original, k_cache=torch.zeros(2, 64, 1, 656, dtype=torch.uint8),
                                           indices=torch.zeros(1), is_fp8_kvcache=True)[0] == 'original'
    assert deepseek.no_sparse_prefill(original, None) is False
    registry = SimpleNamespace(register=lambda name, fn, kind: seen.append((name, fn, kind)))
    deepseek.install(registry, SimpleNamespace(AROUND='around'))
    assert [s[1] for s in seen] == [deepseek.flash_mla_with_kvcache, deepseek.no_sparse_prefill]


def test_enable_fused_store_conditions(monkeypatch):
    def pool(head_dim=128, index_dim=128, pages=(128, 128), scales=(1.0, 1.0), on=False):
        main = SimpleNamespace(head_dim=head_dim, page_size=pages[0], global_scale=torch.tensor([scales[0]]))
        index = SimpleNamespace(INDEX_HEAD_DIM=index_dim, page_size=pages[1], global_scale=torch.tensor([scales[1]]))
        return SimpleNamespace(main_pool=main, index_k_pool=index, use_nvfp4_fused_quantize_store=on)
    p = pool()
    assert minimax.enable_fused_store(p) and p.use_nvfp4_fused_quantize_store
    for bad in (pool(index_dim=64), pool(pages=(128, 64)), pool(scales=(1.0, 0.5))):
        assert not minimax.enable_fused_store(bad) and not bad.use_nvfp4_fused_quantize_store
    monkeypatch.setenv('XTIER_MINIMAX_FP4_FUSED_STORE', '0')
    off = pool()
    assert not minimax.enable_fused_store(off) and not off.use_nvfp4_fused_quantize_store
