"""Block-sparse decode over head-major NVFP4 pages (kv_fp4.py:119-153) on the GPU against the oracle: MiniMax shapes
(64 query heads over 4 KV heads, 128-token blocks), per-KV-head block lists padded with -1, partial last blocks,
lengths clamped to the table, strided pools, kv_scale, key splits, LSE, rows without keys, graph replay equal to
eager, and the full 32-request workload on sampled rows."""
import math

import numpy as np
import pytest
import torch

from oracle import attention
from tests._attn import check
from xtier_amd import ops, workloads

pytestmark = pytest.mark.gpu


def _pool(w, seed, b, extra_heads=0):
    """Head-major pages [pages, kh (+ extra_heads), block, d/2] / [.., d/16] quantized with a unit global scale on the
    GPU; with extra_heads the returned views skip them (a pool with a larger page stride)."""
    gen = workloads.generator('cuda', seed)
    slots = b * w.ctx
    one = torch.ones(1, dtype=torch.float32, device='cuda')
    bufs = []
    for _ in range(2):
        x = workloads.kv_tensor(slots, w.kv_heads + extra_heads, w.dim, gen, 'cuda')
        pay = torch.empty(slots, w.kv_heads + extra_heads, w.dim // 2, dtype=torch.uint8, device='cuda')
        sc = torch.empty(slots, w.kv_heads + extra_heads, w.dim // 16, dtype=torch.uint8, device='cuda')
        ops.quantize_append(x, torch.arange(slots, device='cuda'), one, pay, sc)
        p, s = workloads.head_major_pages(pay, sc, w.block)
        bufs += [p[:, :w.kv_heads], s[:, :w.kv_heads]]
    k_pay, k_sc, v_pay, v_sc = bufs
    return k_pay, k_sc, v_pay, v_sc


def _ref(q, pool, inp, seq, scale, kv_scale, rows=None):
    """FP64 and flash-precision references (and LSE) from the pool bytes the GPU holds, for `rows` (default all)."""
    k_pay, k_sc, v_pay, v_sc = (t.cpu().numpy() for t in pool)
    rows = np.arange(q.shape[0]) if rows is None else np.asarray(rows)
    args = (k_pay, k_sc, v_pay, v_sc, inp.req_to_token.cpu().numpy(), inp.slot_ids.cpu().numpy()[rows],
            inp.topk_idx.cpu().numpy()[:, rows], seq.cpu().numpy()[rows], inp.workload.block, scale, kv_scale)
    qh = q.float().cpu().numpy()[rows]
    ref, lse = attention.block_sparse_decode(qh, *args)
    flash, _ = attention.block_sparse_decode(qh, *args, attend=attention.flash_precision_attention)
    return ref, flash, lse


def _small(seed, b=4, q_heads=64, ctx=4096, topk=16):
    w = workloads.BlockDecodeWorkload('block_test', b, q_heads, 4, 128, ctx, topk)
    return w, workloads.block_decode_inputs(w, seed, 'cuda')


@pytest.mark.parametrize('splits', [None, 1, 3])
def test_minimax_shape_against_oracle(splits):
    w, inp = _small(20261101)
    pool = _pool(w, 5, w.batch)
    idx = inp.topk_idx.clone()
    idx[1, 2, 9:] = -1                                   # a shorter list for one (KV head, row)
    seq = inp.seq_lens.clone()
    seq[1] = w.ctx - 50                                  # a partial last block
    seq[3] = 10 ** 6                                     # clamped to req_to_token.shape[1]
    inp.topk_idx = idx
    lse = torch.empty(w.batch, w.q_heads, dtype=torch.float32, device='cuda')
    out = ops.fp4_sparse_decode(inp.q, pool[0], pool[1], pool[2], pool[3], inp.req_to_token, inp.slot_ids, idx, seq,
                                w.block, lse=lse, splits=splits)
    assert out.shape == (w.batch, w.q_heads, w.dim) and out.dtype == torch.bfloat16
    ref, flash, ref_lse = _ref(inp.q, pool, inp, seq, w.dim ** -0.5, 1.0)
    check(out, ref, flash)
    assert np.abs(lse.cpu().numpy() - ref_lse).max() < 2e-3


def test_group8_strided_pool_kv_scale_and_empty_row():
    w, inp = _small(7, b=5, q_heads=32, ctx=2048, topk=6)
    pool = _pool(w, 9, w.batch, extra_heads=1)
    assert pool[0].stride(0) == 5 * 128 * 64 and not pool[0].is_contiguous()
    idx = inp.topk_idx.clone()
    idx[:, 4] = -1                                       # row 4: no block for any KV head
    inp.topk_idx = idx
    slot_ids = torch.tensor([4, 3, 2, 1, 0], dtype=torch.int32, device='cuda')   # int32 ids, reversed
    inp.slot_ids = slot_ids
    lse = torch.empty(w.batch, w.q_heads, dtype=torch.float32, device='cuda')
    out = ops.fp4_sparse_decode(inp.q, pool[0], pool[1].view(torch.float8_e4m3fn), pool[2],
                                pool[3].view(torch.float8_e4m3fn), inp.req_to_token, slot_ids, idx, inp.seq_lens,
                                w.block, sm_scale=0.07, kv_scale=0.5, lse=lse)
    ref, flash, ref_lse = _ref(inp.q, pool, inp, inp.seq_lens, 0.07, 0.5)
    o = out.float().cpu()
    assert torch.equal(o[4], torch.zeros_like(o[4])) and torch.isneginf(lse[4]).all()
    check(out[:4], ref[:4], flash[:4])
    assert np.abs(lse[:4].cpu().numpy() - ref_lse[:4]).max() < 2e-3


def test_bad_layouts_raise():
    w, inp = _small(3, b=2, ctx=1024, topk=4)
    pool = _pool(w, 2, w.batch)
    with pytest.raises(AssertionError):
        ops.fp4_sparse_decode(inp.q, *pool[:1], pool[1], pool[2], pool[3], inp.req_to_token, inp.slot_ids,
                              inp.topk_idx, inp.seq_lens, 64)
    q80 = torch.zeros(2, 64, 80, dtype=torch.bfloat16, device='cuda')
    with pytest.raises(ValueError):
        ops.fp4_sparse_decode(q80, *pool, inp.req_to_token, inp.slot_ids, inp.topk_idx, inp.seq_lens, 128)


def test_graph_replay_equals_eager():
    w, inp = _small(11, b=3, ctx=2048, topk=8)
    pool = _pool(w, 4, w.batch)
    splits = 2
    ws = ops.new_workspace('cuda', w.batch, w.q_heads, w.dim, splits)
    q = inp.q.clone()
    out = torch.empty_like(q)
    args = (pool[0], pool[1], pool[2], pool[3], inp.req_to_token, inp.slot_ids, inp.topk_idx, inp.seq_lens, w.block)
    ops.fp4_sparse_decode(q, *args, out=out, splits=splits, ws=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.fp4_sparse_decode(q, *args, out=out, splits=splits, ws=ws)
    gen = torch.Generator(device='cuda').manual_seed(3)
    for _ in range(3):
        q.copy_(torch.randn(q.shape, generator=gen, device='cuda').to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = ops.fp4_sparse_decode(q, *args, splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16))


def test_full_workload_sampled_rows():
    """The 32-request, 32768-token workload (4 KV heads x 16 blocks of 128 per row) with the default splits; six
    rows checked against the oracle from the bytes the GPU holds."""
    w = workloads.BLOCK_WORKLOADS['minimax_decode_b32']
    inp = workloads.block_decode_inputs(w, 20261102, 'cuda')
    pool = _pool(w, 6, w.batch)
    out = ops.fp4_sparse_decode(inp.q, *pool, inp.req_to_token, inp.slot_ids, inp.topk_idx, inp.seq_lens, w.block)
    rows = [0, 5, 13, 21, 30, 31]
    sel = torch.tensor(rows, device='cuda')
    # only the pages the sampled rows read travel to the host: remap them to a compact pool
    used = torch.unique(inp.req_to_token[sel][:, ::w.block].long() // w.block)
    remap = torch.full((w.pages,), -1, dtype=torch.int64, device='cuda')
    remap[used] = torch.arange(used.numel(), device='cuda')
    r2t = inp.req_to_token.clone()
    r2t[sel] = (remap[r2t[sel].long() // w.block] * w.block + r2t[sel].long() % w.block).to(torch.int32)
    small = tuple(t[used] for t in pool)
    sub = workloads.BlockDecodeInputs(w, inp.q, r2t, inp.slot_ids, inp.topk_idx, inp.seq_lens)
    ref, flash, _ = _ref(inp.q, small, sub, inp.seq_lens, w.dim ** -0.5, 1.0, rows=rows)
    check(out[sel], ref, flash)
    assert math.isfinite(out.float().abs().max().item())


def test_decode_main_hook_equals_direct_call():
    """The hook (kv_fp4.py:579-590) with the keyword call SGLang makes, q_scale folded into sm_scale."""
    from xtier_amd import minimax
    w, inp = _small(13, b=2, ctx=1024, topk=4)
    k_pay, k_sc, v_pay, v_sc = _pool(w, 8, w.batch)
    k_view, v_view = k_pay[:], v_pay[:]
    setattr(k_view, minimax.TAG, k_sc)
    setattr(v_view, minimax.TAG, v_sc)
    got = minimax.decode_main(None, q=inp.q, k_cache=k_view, v_cache=v_view, req_to_token=inp.req_to_token,
                              slot_ids=inp.slot_ids, topk_idx=inp.topk_idx, seq_lens=inp.seq_lens,
                              block_size=w.block, sm_scale=0.1, q_scale=0.5, k_scale=1.0)
    want = ops.fp4_sparse_decode(inp.q, k_pay, k_sc, v_pay, v_sc, inp.req_to_token, inp.slot_ids, inp.topk_idx,
                                 inp.seq_lens, w.block, sm_scale=0.05)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
