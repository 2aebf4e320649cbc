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
    assert seen == [(minimax.KV_POOL, minimax.kv_pool, 'around'),
                    (f'{minimax.OPS}.flash_decode_with_topk_idx', minimax.decode_topk, 'around'),
                    (f'{minimax.OPS}.flash_decode_with_gqa_share_sparse', minimax.decode_main, 'around'),
                    (f'{minimax.OPS}.flash_prefill_with_topk_index', minimax.prefill_topk, 'around'),
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


def _fake_sglang(kernel_name, launch_args, launch_kwargs, grid):
    """A stand-in for the SGLang module whose score kernel the top-k hooks replace: its entry launches
    ``kernel_name`` of its own module with the given arguments and returns what it saw."""
    import sys
    import types
    mod = types.ModuleType('xt_fake_sglang_topk')

    class Real:
        def __getitem__(self, g):
            raise AssertionError('the real score kernel ran')
    setattr(mod, kernel_name, Real())

    def run(q, k_cache, **kwargs):
        getattr(mod, kernel_name)[grid](q, k_cache, *launch_args, **launch_kwargs)
        return 'topk', k_cache.shape, kwargs
    run.__module__ = mod.__name__
    sys.modules[mod.__name__] = mod
    return mod, run


def test_decode_topk_hook_routes_the_score_launch(monkeypatch):
    seen = {}
    monkeypatch.setattr(minimax.ops, 'minimax_decode_scores', lambda *a, **k: seen.update(args=a, kw=k))
    pay = torch.zeros(3, 128, 64, dtype=torch.uint8)
    sc = torch.zeros(3, 128, 8, dtype=torch.uint8)
    setattr(pay, minimax.TAG, sc)
    q = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    r2t, score, seq, sid = torch.zeros(2, 9), torch.zeros(8, 2, 4), torch.zeros(2), torch.zeros(2)
    # the launch arguments of SGLang's _decode_score_kernel, as the reference's shim takes them (kv_fp4.py:233-236)
    args = (r2t, score, seq, sid, 999, 2, 4, 128, 64, 16, 0.1, 1.0, 0, 1, 1024, 128, 1, 0, 0, 0, 9, 8, 4, 1)
    mod, run = _fake_sglang('_decode_score_kernel', args, dict(NUM_KV_CHUNKS=2, SCORE_TYPE='lse',
                                                               SKIP_TRIVIAL_TOPK_SCORE=True), (4, 2))
    kept = mod._decode_score_kernel
    got = minimax.decode_topk(run, q=q, k_cache=pay, disable_index_value=True, sink=None, topk=16)
    assert got[0] == 'topk' and got[1] == (384, 1, 128) and got[2] == dict(disable_index_value=True, sink=None,
                                                                              topk=16)
    assert mod._decode_score_kernel is kept                        # restored after the call
    a, k = seen['args'], seen['kw']
    assert a[:4] == (q, pay, sc, r2t) and a[4] is score and a[7:13] == (64, 0.1, 1.0, 0, 1, 'lse')
    assert k == dict(skip_topk=16, heads=2 * 4, batch=2, q_strides=(1024, 128, 1), r2t_stride=9,
                     score_strides=(8, 4, 1))
    with pytest.raises(NotImplementedError):
        minimax.decode_topk(run, q=q, k_cache=pay, disable_index_value=False)
    assert minimax.decode_topk(_original, q=q, k_cache=torch.zeros(1))[0] == 'original'


def test_prefill_topk_hook_routes_the_score_launch(monkeypatch):
    seen = {}
    monkeypatch.setattr(minimax.ops, 'minimax_prefill_scores', lambda *a, **k: seen.update(args=a, kw=k))
    pay = torch.zeros(3, 128, 64, dtype=torch.uint8)
    sc = torch.zeros(3, 128, 8, dtype=torch.uint8)
    setattr(pay, minimax.TAG, sc)
    q = torch.zeros(70, 4, 128, dtype=torch.bfloat16)
    score, r2t, cu, seq, pre, sid = (torch.zeros(1) for _ in range(6))
    # SGLang's _flash_attn_fwd_with_block_score_kernel arguments (kv_fp4.py:459-462), the score strides and the
    # req_to_token stride last
    args = (None, None, score, r2t, cu, seq, pre, sid, 999, 4, 4, 128, 128, 64, 0.2, 1.0, 1.0, None, None, 512, 128,
            1, 'x', 'y', 300, 75, 1, 77)
    mod, run = _fake_sglang('_flash_attn_fwd_with_block_score_kernel', (None,) + args,
                            dict(SCORE_TYPE='max', DISABLE_INDEX_VALUE=True), lambda meta: (2, 4))
    got = minimax.prefill_topk(run, q=q, k_cache=pay, disable_index_value=True)
    assert got[0] == 'topk'
    a, k = seen['args'], seen['kw']
    assert a[:5] == (q, pay, sc, r2t, score) and a[5:12] == (cu, seq, pre, sid, 64, 0.2, 1.0)
    assert k == dict(max_q_len=128, heads=4, q_strides=(512, 128, 1), r2t_stride=77, score_strides=(300, 75, 1))


def _msa_pool(nvfp4=True, same_scale=True):
    pays = [torch.zeros(1), torch.zeros(1)]
    scs = [torch.ones(1), torch.ones(1)]
    main = SimpleNamespace(k_buffer=pays, k_scale_buffer=scs, v_buffer=pays[::-1], v_scale_buffer=scs[::-1],
                           head_dim=128, page_size=128, global_scale=torch.ones(1), is_minimax_m3_nvfp4_main=nvfp4)
    index = SimpleNamespace(k_buffer=[torch.zeros(1)], k_scale_buffer=[torch.ones(1)], INDEX_HEAD_DIM=128,
                            page_size=128, global_scale=torch.ones(1) * (1.0 if same_scale else 2.0))
    return SimpleNamespace(main_pool=main, index_k_pool=index, use_nvfp4_fused_quantize_store=False, size=256)


def test_kv_pool_hook_tags_nvfp4_pools_and_turns_on_the_fused_store(monkeypatch):
    """AROUND _build_minimax_sparse_kv_pool (minimax_m3/__init__.py:93-100): an NVFP4 MSA-v1 pool comes back with its
    payload views tagged and the one-launch store on; the builder's arguments pass through unchanged."""
    monkeypatch.delenv('XTIER_MINIMAX_FP4_FUSED_STORE', raising=False)
    pool = _msa_pool()
    calls = []

    def build(*args, **kwargs):
        calls.append((args, kwargs))
        return pool
    assert minimax.kv_pool(build, 'cfg', dtype='nvfp4') is pool
    assert calls == [(('cfg',), {'dtype': 'nvfp4'})]
    assert minimax.scales_of(pool.main_pool.k_buffer[0]) is pool.main_pool.k_scale_buffer[0]
    assert minimax.scales_of(pool.index_k_pool.k_buffer[0]) is pool.index_k_pool.k_scale_buffer[0]
    assert pool.use_nvfp4_fused_quantize_store
    # the pools' global scales differ: tagged, but the stores stay SGLang's
    other = _msa_pool(same_scale=False)
    minimax.kv_pool(lambda: other)
    assert minimax.scales_of(other.main_pool.k_buffer[0]) is not None and not other.use_nvfp4_fused_quantize_store


def test_kv_pool_hook_leaves_other_pools_alone():
    for pool in (_msa_pool(nvfp4=False), SimpleNamespace(size=3)):
        assert minimax.kv_pool(lambda p=pool: p) is pool
    plain = _msa_pool(nvfp4=False)
    minimax.kv_pool(lambda: plain)
    assert minimax.scales_of(plain.main_pool.k_buffer[0]) is None and not plain.use_nvfp4_fused_quantize_store


def test_install_off_switch(monkeypatch):
    """XTIER_MINIMAX_KV_FP4=0 (minimax_m3/__init__.py:176-181) registers neither the pool hook nor the op hooks."""
    monkeypatch.setenv('XTIER_MINIMAX_KV_FP4', '0')
    seen = []
    minimax.install(SimpleNamespace(register=lambda *a: seen.append(a)), SimpleNamespace(AROUND='around'))
    assert seen == []
