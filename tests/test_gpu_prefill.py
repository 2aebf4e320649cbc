"""Chunked sparse prefill on the GPU: the chunk's K/V rows quantized into the pool (bit-exact against the oracle),
then every query token attends to its own causal top-k positions (query_pos = its position; the reference's causal
mask q_pos >= key, xtier/packs/minimax_m3/kv_fp4.py:330-331, :345) through the fused kernel, against the FP64 oracle
on the pool bytes. The full-size workload (4096 queries at context 65536, top-2048) is checked on sampled rows."""
import math

import numpy as np
import pytest
import torch

from oracle import nvfp4
from tests._attn import check, oracle
from tests._pools import bf16_numpy
from xtier_amd import ops, workloads
from xtier_amd.pool import KVPool

pytestmark = pytest.mark.gpu


def _run_prefill(w, inp, layout='split'):
    """Pool of w.ctx slots: context rows quantized up front, the chunk's rows appended by quantize_append; then the
    attention of the chunk's queries. Returns (pool, out, slots of the chunk rows)."""
    dev = 'cuda'
    k, v = inp.k.to(dev), inp.v.to(dev)
    pool = KVPool(w.slots, w.kv_heads, w.dim, dev, layout=layout)
    pool.set_global_scales(k, v)          # per-layer scales fixed before the chunk arrives
    pt = inp.page_table.to(dev)
    pos = torch.arange(w.ctx, device=dev)
    slot_of = (pt[0, pos // w.page].long() * w.page + pos % w.page)
    ctx_slots, chunk_slots = slot_of[:w.ctx0], slot_of[w.ctx0:]
    pool.append(k[:w.ctx0], v[:w.ctx0], ctx_slots, saturate=False)
    pool.append(k[w.ctx0:], v[w.ctx0:], chunk_slots, saturate=False)      # the step's quantize-on-append
    rows = w.chunk
    out = ops.sparse_decode(inp.q.to(dev), pool.raw, pt, inp.indices.to(dev),
                            torch.full((rows,), w.ctx, dtype=torch.int32, device=dev), 1.0 / math.sqrt(w.dim),
                            page_size=w.page, row_req=torch.zeros(rows, dtype=torch.int64, device=dev),
                            query_pos=inp.q_pos.to(dev))
    return pool, out, chunk_slots


@pytest.mark.parametrize('layout', ['split', 'interleaved'])
def test_prefill_chunk_small(layout):
    w = workloads.PrefillWorkload('prefill_small', 32, 4, 128, 4096, 256, 512)
    inp = workloads.prefill_inputs(w, seed=20261023)
    pool, out, chunk_slots = _run_prefill(w, inp, layout)
    # the appended rows: the oracle's bytes under the pool's global scales
    s = chunk_slots.cpu().numpy()
    for x, pay, sc, g in ((inp.k, pool.k_pay, pool.k_sf, pool.gk), (inp.v, pool.v_pay, pool.v_sf, pool.gv)):
        opay, osc = nvfp4.quantize_blocks(bf16_numpy(x[w.ctx0:]), np.float32(g.item()))
        assert np.array_equal(pay.cpu().numpy()[s], opay) and np.array_equal(sc.cpu().numpy()[s], osc)
    ref, flash, _ = oracle(pool.raw, bf16_numpy(inp.q), inp.page_table.numpy(), w.page, np.zeros(w.chunk, np.int64),
                           inp.indices.numpy(), None, np.full(w.chunk, w.ctx, np.int32), 1 / math.sqrt(w.dim),
                           inp.q_pos.numpy())
    check(out, ref, flash)


def test_prefill_causal_limit_masks_later_positions():
    """Positions after a query's own position are masked even when listed: the last 16 positions of the context
    written into every query's list (future ones for all queries but the last few) against the oracle on the same
    lists."""
    w = workloads.PrefillWorkload('prefill_mask', 32, 4, 128, 2048, 64, 256)
    inp = workloads.prefill_inputs(w, seed=7)
    pool, out, _ = _run_prefill(w, inp)
    idx = inp.indices.clone()
    idx[:, :16] = torch.arange(w.ctx - 16, w.ctx, dtype=torch.int32)[None, :]     # future for every query but none
    idx = torch.sort(idx, dim=1).values
    dev = 'cuda'
    got = ops.sparse_decode(inp.q.to(dev), pool.raw, inp.page_table.to(dev), idx.to(dev),
                            torch.full((w.chunk,), w.ctx, dtype=torch.int32, device=dev), 1.0 / math.sqrt(w.dim),
                            page_size=w.page, row_req=torch.zeros(w.chunk, dtype=torch.int64, device=dev),
                            query_pos=inp.q_pos.to(dev))
    ref, flash, _ = oracle(pool.raw, bf16_numpy(inp.q), inp.page_table.numpy(), w.page, np.zeros(w.chunk, np.int64),
                           idx.numpy(), None, np.full(w.chunk, w.ctx, np.int32), 1 / math.sqrt(w.dim),
                           inp.q_pos.numpy())
    check(got, ref, flash)


def test_prefill_full_chunk_sampled_rows():
    """The full workload: 4096 queries appended at 65536, top-2048 causal each. All rows run; 48 sampled rows (first,
    last and random) are checked against the FP64 oracle."""
    w = workloads.PREFILL_WORKLOADS['gqa_prefill_chunk4096']
    inp = workloads.prefill_inputs(w, seed=20261029, device='cuda')
    pool, out, _ = _run_prefill(w, inp)
    gen = np.random.default_rng(5)
    rows = np.unique(np.concatenate([[0, 1, w.chunk - 1], gen.choice(w.chunk, 45, replace=False)]))
    q = bf16_numpy(inp.q.cpu()[rows])
    ref, flash, _ = oracle(pool.raw, q, inp.page_table.cpu().numpy(), w.page, np.zeros(len(rows), np.int64),
                           inp.indices.cpu().numpy()[rows], None, np.full(len(rows), w.ctx, np.int32),
                           1 / math.sqrt(w.dim), inp.q_pos.cpu().numpy()[rows])
    check(out[torch.from_numpy(rows).cuda()], ref, flash, strict=True)
