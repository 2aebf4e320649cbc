"""Causal block-sparse prefill over head-major NVFP4 pages (kv_fp4.py:293-404) and the BF16 context copy
(kv_fp4.py:496-530) on the GPU against the oracle: MiniMax shapes (64 query heads over 4 KV heads, d 128, 128-token
blocks), ragged query lengths with prefixes, query blocks of 1 and 64 sharing a list, lists in any order with blocks
in the queries' future and -1 padding, per-token slot lookups (tokens off their block's page), strided pools, kv_scale,
key splits; the copy bit-exact, with the one-head index cache and untouched rows; and the two prefill hooks."""
import numpy as np
import pytest
import torch

from oracle import attention
from tests._attn import check
from xtier_amd import minimax, ops, workloads

pytestmark = pytest.mark.gpu

KH, GROUP, D, BLOCK = 4, 16, 128, 128


def _pages(seed, pages, heads=KH, extra_heads=0):
    """Head-major K and V pages [pages, heads, BLOCK, D/2] / [.., D/16] quantized with a unit global scale on the
    GPU; with extra_heads the views skip them (a larger page stride)."""
    gen = workloads.generator('cuda', seed)
    slots = pages * BLOCK
    one = torch.ones(1, dtype=torch.float32, device='cuda')
    out = []
    for _ in range(2):
        x = workloads.kv_tensor(slots, heads + extra_heads, D, gen, 'cuda')
        pay = torch.empty(slots, heads + extra_heads, D // 2, dtype=torch.uint8, device='cuda')
        sc = torch.empty(slots, heads + extra_heads, D // 16, dtype=torch.uint8, device='cuda')
        ops.quantize_append(x, torch.arange(slots, device='cuda'), one, pay, sc)
        p, s = workloads.head_major_pages(pay, sc, BLOCK)
        out += [p[:, :heads], s[:, :heads]]
    return out


def _case(seed, q_lens, prefix, bq, topk, pages=48):
    """Queries, a per-token req_to_token over random slots, and per-(KV head, query block) lists of distinct block ids
    in random order (blocks past a query's position included), some padded with -1."""
    rng = np.random.default_rng(seed)
    b = len(q_lens)
    seq = np.array([p + n for p, n in zip(prefix, q_lens)], dtype=np.int32)
    ctx = int(seq.max())
    r2t = np.stack([rng.permutation(pages * BLOCK)[:ctx] for _ in range(b + 1)]).astype(np.int32)
    sid = rng.permutation(b + 1)[:b].astype(np.int64)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    nqb = [-(-n // bq) for n in q_lens]
    cu_blk = np.concatenate([[0], np.cumsum(nqb)]).astype(np.int32)
    ids = np.full((KH, cu_blk[-1], topk), -1, dtype=np.int32)
    for h in range(KH):
        for r in range(b):
            nb = -(-int(seq[r]) // BLOCK)
            for j in range(nqb[r]):
                n = min(topk, nb) - (j + h) % 3 // 2
                ids[h, cu_blk[r] + j, :n] = rng.permutation(nb)[:n]
    q = (torch.from_numpy(rng.standard_normal((int(cu[-1]), KH * GROUP, D))).float()).to(torch.bfloat16)
    cuda = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return dict(q=q.cuda(), r2t=cuda(r2t), sid=cuda(sid), ids=cuda(ids), cu=cuda(cu), cu_blk=cuda(cu_blk),
                seq=cuda(seq), prefix=cuda(np.array(prefix, dtype=np.int32)), bq=bq)


def _run(c, pool, **kw):
    k_pay, k_sc, v_pay, v_sc = pool
    return ops.fp4_prefill_gqa_share_sparse(
        c['q'], k_pay, v_pay, None, c['r2t'], c['sid'], c['ids'], c['bq'], BLOCK, c['cu'], c['seq'], c['prefix'],
        int((c['cu'][1:] - c['cu'][:-1]).max()), cu_seqblocks_q=c['cu_blk'], k_sc=k_sc, v_sc=v_sc, **kw)


def _ref(c, pool, scale, kv_scale=1.0):
    host = [t.cpu().numpy() for t in pool]
    k_pay, k_sc, v_pay, v_sc = host
    args = (c['q'].float().cpu().numpy(), k_pay, k_sc, v_pay, v_sc, c['r2t'].cpu().numpy(), c['sid'].cpu().numpy(),
            c['ids'].cpu().numpy(), c['cu'].cpu().numpy(), c['cu_blk'].cpu().numpy(), c['seq'].cpu().numpy(),
            c['prefix'].cpu().numpy(), c['bq'], BLOCK, scale, kv_scale)
    ref = attention.block_sparse_prefill(*args)
    flash = attention.block_sparse_prefill(*args, attend=attention.flash_precision_attention)
    return ref, flash


@pytest.mark.parametrize('bq,splits', [(1, None), (64, 1), (64, 3)])
def test_minimax_prefill_against_oracle(bq, splits):
    print(f'block-sparse prefill bq={bq} splits={splits}', flush=True)
    c = _case(20261201 + bq, q_lens=(150, 1, 77), prefix=(900, 2000, 0), bq=bq, topk=6)
    pool = _pages(3, 48)
    out = _run(c, pool, splits=splits)
    assert out.shape == c['q'].shape and out.dtype == torch.bfloat16
    ref, flash = _ref(c, pool, D ** -0.5)
    check(out, ref, flash)


def test_strided_pool_kv_scale_and_queries_without_keys():
    print('block-sparse prefill: strided pool, kv_scale, empty rows', flush=True)
    c = _case(77, q_lens=(40, 70), prefix=(300, 129), bq=16, topk=3)
    ids = c['ids'].clone()
    ids[:, 0] = -1
    ids[:, 0, 0] = 3                      # positions 384..511: past every query of request 0's first block
    c['ids'] = ids
    pool = _pages(8, 48, extra_heads=1)
    assert not pool[0].is_contiguous()
    out = _run(c, pool, sm_scale=0.07, kv_scale=0.625)
    ref, flash = _ref(c, pool, 0.07, 0.625)
    assert torch.all(out[:16] == 0)
    check(out, ref, flash)


def test_context_copy_bit_exact_main_and_index():
    print('dequantize_context', flush=True)
    c = _case(5, q_lens=(10, 10, 10), prefix=(1000, 37, 300), bq=1, topk=1)
    pool = _pages(12, 48)
    rows = 1024
    sentinel = -7.0
    for pay, sc in ((pool[0], pool[1]), (pool[2][:, 2], pool[3][:, 2])):
        out = torch.full((3 * rows,) + ((KH,) if pay.dim() == 4 else (1,)) + (D,), sentinel, dtype=torch.bfloat16,
                         device='cuda')
        got = ops.dequantize_context(pay, sc, c['r2t'], c['sid'], c['seq'], rows, out=out)
        assert got is out
        want = attention.dequantize_context(pay.cpu().numpy(), sc.cpu().numpy(), c['r2t'].cpu().numpy(),
                                            c['sid'].cpu().numpy(), c['seq'].cpu().numpy(), rows)
        g = out.float().cpu().numpy()
        written = ~np.isnan(want)
        np.testing.assert_array_equal(g[written], want[written])
        assert np.all(g[~written] == sentinel)
    fresh = ops.dequantize_context(pool[0], pool[1], c['r2t'], c['sid'], c['seq'], rows)
    assert fresh.shape == (3 * rows, KH, D) and fresh.dtype == torch.bfloat16


class _Keep:
    def __init__(self):
        self.calls = []

    def __call__(self, *args, **kwargs):
        self.calls.append((args, kwargs))
        return 'original'


def test_prefill_hooks(monkeypatch):
    print('minimax prefill hooks', flush=True)
    c = _case(9, q_lens=(20, 5), prefix=(200, 400), bq=1, topk=4, pages=16)
    k_pay, k_sc, v_pay, v_sc = _pages(4, 16)
    ik_pay, ik_sc = _pages(6, 16, heads=1)[:2]
    ik_pay, ik_sc = ik_pay[:, 0], ik_sc[:, 0]
    for view, sc in ((k_pay, k_sc), (v_pay, v_sc), (ik_pay, ik_sc)):
        setattr(view, minimax.TAG, sc)
    # prefill_main: keyword call -> the NVFP4 prefill
    kw = dict(q=c['q'], k_cache=k_pay, v_cache=v_pay, sink=None, req_to_token=c['r2t'], slot_ids=c['sid'],
              topk_idx=c['ids'], block_size_q=1, block_size_k=BLOCK, cu_seqlens=c['cu'], seq_lens=c['seq'],
              prefix_lens=c['prefix'], max_seqlen_q=20, cu_seqblocks_q=c['cu_blk'], k_scale=1.0)
    got = minimax.prefill_main(_Keep(), **kw)
    want = _run(c, (k_pay, k_sc, v_pay, v_sc))
    assert torch.equal(got, want)
    with pytest.raises(ValueError):
        minimax.prefill_main(_Keep(), **dict(kw, v_scale=0.5))
    # sparse_prefill: BF16 copies with a request-local table when they fit, the caches themselves otherwise
    orig = _Keep()
    args = (c['q'], k_pay, v_pay, None, 'idx_q', ik_pay, None, None, c['r2t'], c['sid'], c['cu'], c['seq'],
            c['prefix'], 20, 405)
    assert minimax.sparse_prefill(orig, *args, 'extra', flag=2) == 'original'
    a, kwargs = orig.calls[-1]
    assert kwargs == {'flag': 2} and a[15] == 'extra' and a[6] is None
    k, v, ik, r2t, local = a[1], a[2], a[5], a[8], a[9]
    assert k.shape == (2 * 512, KH, D) and ik.shape == (2 * 512, 1, D)
    assert torch.equal(r2t, torch.arange(2 * 512, dtype=torch.int32, device='cuda').view(2, 512))
    assert torch.equal(local, torch.arange(2, dtype=torch.int32, device='cuda'))
    for got_t, (pay, sc) in ((k, (k_pay, k_sc)), (v, (v_pay, v_sc)), (ik, (ik_pay, ik_sc))):
        want_t = ops.dequantize_context(pay, sc, c['r2t'], c['sid'], c['seq'], 512)
        for b in range(2):
            n = int(c['seq'][b])
            assert torch.equal(got_t[b * 512:b * 512 + n], want_t[b * 512:b * 512 + n])
    monkeypatch.setattr(minimax, 'PREFILL_GB', 1e-6)
    minimax.sparse_prefill(orig, *args)
    a, _ = orig.calls[-1]
    assert a[1] is k_pay and a[5] is ik_pay and a[8] is c['r2t']


def test_prefill_chunk_workload_on_sampled_rows():
    """The benchmarked chunk (4096 queries after 61440 tokens, MiniMax heads, 16 blocks per query) at full size,
    checked against the oracle on sampled query rows."""
    w = workloads.BLOCK_PREFILL_WORKLOADS['minimax_prefill_chunk4096']
    print(f'{w.name}: full size, sampled rows', flush=True)
    inp = workloads.block_prefill_inputs(w, 20261202, 'cuda')
    shape = workloads.BlockDecodeWorkload(w.name, 1, w.q_heads, w.kv_heads, w.dim, w.ctx, w.topk_blocks, w.block)
    gen = workloads.generator('cuda', 31)
    pool = []
    one = torch.ones(1, dtype=torch.float32, device='cuda')
    for _ in range(2):
        x = workloads.kv_tensor(w.ctx, w.kv_heads, w.dim, gen, 'cuda')
        pay = torch.empty(w.ctx, w.kv_heads, w.dim // 2, dtype=torch.uint8, device='cuda')
        sc = torch.empty(w.ctx, w.kv_heads, w.dim // 16, dtype=torch.uint8, device='cuda')
        ops.quantize_append(x, torch.arange(w.ctx, device='cuda'), one, pay, sc)
        pool += list(workloads.head_major_pages(pay, sc, shape.block))
    k_pay, k_sc, v_pay, v_sc = pool
    out = ops.fp4_prefill_gqa_share_sparse(inp.q, k_pay, v_pay, None, inp.req_to_token, inp.slot_ids, inp.topk_idx, 1,
                                           w.block, inp.cu_seqlens, inp.seq_lens, inp.prefix_lens, w.q_len,
                                           k_sc=k_sc, v_sc=v_sc)
    rows = np.array([0, 1, 127, 128, 1000, 2047, 2048, 3000, 4094, 4095])
    n = len(rows)
    host = [t.cpu().numpy() for t in pool]
    args = (inp.q.float().cpu().numpy()[rows], host[0], host[1], host[2], host[3], inp.req_to_token.cpu().numpy(),
            np.zeros(n, np.int64), inp.topk_idx.cpu().numpy()[:, rows], np.arange(n + 1), np.arange(n + 1),
            np.full(n, w.ctx), w.prefix + rows, 1, w.block, w.dim ** -0.5)
    ref = attention.block_sparse_prefill(*args)
    flash = attention.block_sparse_prefill(*args, attend=attention.flash_precision_attention)
    check(out[torch.from_numpy(rows).cuda()], ref, flash)
