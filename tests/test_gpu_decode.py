"""Fused NVFP4 sparse GQA decode on the GPU against the oracle: FP64 softmax on the dequantized KV with the
tolerance max-abs 2e-2 / mean-abs 2e-3 in BF16, the precision class of the flash kernels
(tests/qsa_decode_check.py:82: max error <= 1.5x and mean <= 1.25x the flash-precision reference's), closed-form
special cases bit for bit, and HIP-graph replay equal to eager bit for bit (tests/qsa_decode_check.py:94-108)."""
import math

import numpy as np
import pytest
import torch

from oracle import attention, nvfp4
from tests._attn import MAX_ABS, MEAN_ABS, check as _check, oracle as _oracle
from tests._pools import Pool, bf16_numpy
from xtier_amd import ops, workloads
from xtier_amd.pool import KVPool

pytestmark = pytest.mark.gpu


def _dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def _gpu_pool(inp):
    k_pay, k_sf, gk = ops.nvfp4_encode(inp.k.cuda())
    v_pay, v_sf, gv = ops.nvfp4_encode(inp.v.cuda())
    return (k_pay, v_pay, k_sf, v_sf, gk, gv)


@pytest.mark.parametrize('name,batch', [('cpu_ref_decode', None), ('gqa_decode_b32', 4)])
def test_decode_workload(name, batch):
    w = workloads.WORKLOADS[name]
    inp = workloads.decode_inputs(w, seed=20261029, batch=batch)
    raw = _gpu_pool(inp)
    scale = 1.0 / math.sqrt(w.dim)
    lse = torch.empty(inp.q.shape[:2], dtype=torch.float32, device='cuda')
    out = ops.sparse_decode(inp.q.cuda(), raw, inp.page_table.cuda(), inp.indices.cuda(), inp.seq_lens.cuda(),
                            scale, page_size=w.page, lse=lse)
    b = inp.q.shape[0]
    ref, flash, lse_ref = _oracle(raw, bf16_numpy(inp.q), inp.page_table.numpy(), w.page, np.arange(b),
                                  inp.indices.numpy(), None, inp.seq_lens.numpy(), scale)
    _check(out, ref, flash, strict=True)
    assert np.abs(lse.cpu().numpy() - lse_ref).max() < 2e-3


def _small_case(seed=3, batch=6, ctx=3008, heads=4, qh=32, topk=700, page=64, dim=128):
    gen = workloads.generator('cpu', seed)
    ctx_p = -(-ctx // page) * page
    k = workloads.kv_tensor(batch * ctx_p, heads, dim, gen, 'cpu')
    v = workloads.kv_tensor(batch * ctx_p, heads, dim, gen, 'cpu')
    pool = Pool(k, v)
    pt = workloads.page_table(batch, ctx_p, page, gen, 'cpu')
    idx = workloads.index_lists(batch, ctx_p, topk, gen, 'cpu')
    q = (torch.randn(batch, qh, dim, generator=gen) * 2).to(torch.bfloat16)
    return pool, pt, idx, q


@pytest.mark.parametrize('dim,heads,qh,batch,splits', [
    (64, 2, 16, 6, 1), (64, 4, 32, 40, 4), (64, 1, 8, 5, 3),
    (256, 2, 24, 6, 1), (256, 2, 24, 6, 5), (256, 4, 32, 80, 4), (256, 1, 4, 3, 2), (256, 2, 16, 128, 2),
])
def test_decode_head_sizes(dim, heads, qh, batch, splits):
    """Head sizes 64 and 256 (the reference's Qwen3.8 QSA shape is 2 KV heads x 256) against the oracle, with -1
    holes, short rows and key splits; 80 rows x 4 KV heads x 4 splits takes 4 KV heads per workgroup, 40 rows x 4 KV
    heads x 4 splits (head size 64) and 128 rows x 2 KV heads x 2 splits (head size 256) take 2."""
    pool, pt, idx, q = _small_case(seed=dim + heads * 10 + batch, batch=batch, heads=heads, qh=qh, dim=dim)
    idx = idx.numpy().copy()
    idx[0, ::9] = -1
    seq = np.full(batch, 3008, np.int32)
    seq[-1] = 1200
    scale = dim ** -0.5
    lse = torch.empty(batch, qh, dtype=torch.float32, device='cuda')
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), _dev(idx), _dev(seq), scale, page_size=64, lse=lse,
                            splits=splits)
    ref, flash, lse_ref = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(batch), idx, None, seq, scale)
    _check(out, ref, flash)
    # the query enters the MFMA exactly (q * 2^-e per head), so the LSE carries only FP32 rounding
    assert np.abs(lse.cpu().numpy() - lse_ref).max() < 2e-3


@pytest.mark.parametrize('mag', [1e-4, 1e3, 1e6, 'mixed'])
def test_decode_query_magnitudes(mag):
    """Queries far from unit size: |q| ~ 1e-4 (q * scale * log2(e) would sit among FP16's subnormals), 1e3, 1e6
    (beyond FP16's range once scaled) and rows whose heads span seven decades (1e-4 .. 1e3). Each head's query enters
    the MFMA as q * 2^-e, exactly, with 2^e from its own largest magnitude: every row within tolerance of the FP64
    oracle, the LSE within FP32 rounding of the scores."""
    pool, pt, idx, q = _small_case(seed=77, batch=4, topk=500)
    if mag == 'mixed':
        heads = torch.arange(q.shape[1])
        q = (q.float() * (10.0 ** ((heads % 8) - 4)).view(1, -1, 1)).to(torch.bfloat16)
    else:
        q = (q.float() * mag).to(torch.bfloat16)
    seq = np.full(4, 3008, np.int32)
    scale = 128 ** -0.5
    lse = torch.empty(4, q.shape[1], dtype=torch.float32, device='cuda')
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), idx.cuda(), _dev(seq), scale, page_size=64, lse=lse,
                            splits=2)
    ref, flash, lse_ref = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(4), idx.numpy(), None, seq, scale)
    _check(out, ref, flash)
    got = lse.cpu().numpy()
    assert np.isfinite(got).all()
    assert (np.abs(got - lse_ref) <= 2e-3 + 1e-6 * np.abs(lse_ref)).all()


@pytest.mark.parametrize('dim', [64, 256])
def test_decode_head_sizes_single_key_and_empty_rows(dim):
    """One valid key gives that V row (bit for bit after BF16 rounding); no valid key gives exact zeros."""
    pool, pt, idx, q = _small_case(seed=7, batch=3, heads=2, qh=8, dim=dim, topk=64)
    counts = np.array([0, 1, 64], np.int32)
    seq = np.full(3, 3008, np.int32)
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), idx.cuda(), _dev(seq), dim ** -0.5, page_size=64,
                            counts=_dev(counts), splits=2)
    assert not out[0].any()
    pos = int(idx[1, 0])
    slot = int(pt[1, pos // 64]) * 64 + pos % 64
    v = nvfp4.dequant(pool.v_pay[slot], pool.v_sf[slot], pool.gv)          # [heads, dim]
    want = torch.from_numpy(np.repeat(v, 4, axis=0)).to(torch.bfloat16)
    assert torch.equal(out[1].cpu().view(torch.int16), want.view(torch.int16))


def test_decode_edge_rows():
    """Row 0: no valid key (count 0) -> exact zeros and LSE -inf. Row 1: one valid key -> that value exactly.
    Row 2: -1 holes and positions past the row's length. Row 3: a causal limit. Rows 4, 5: plain."""
    pool, pt, idx, q = _small_case()
    batch, topk = idx.shape
    idx = idx.numpy().copy()
    seq = np.full(batch, 3008, np.int32)
    counts = np.full(batch, topk, np.int32)
    counts[0] = 0
    counts[1] = 1
    idx[2, ::7] = -1
    seq[2] = 1500
    qpos = np.full(batch, 1 << 30, np.int32)
    qpos[3] = 1000
    scale = 1 / math.sqrt(128)
    lse = torch.empty(batch, 32, dtype=torch.float32, device='cuda')
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), _dev(idx), _dev(seq), scale, page_size=64,
                            counts=_dev(counts), query_pos=_dev(qpos), lse=lse, splits=3)
    ref, flash, _ = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(batch), idx, counts, seq, scale,
                            qpos)
    # rows with many keys against the tolerances; row 0 (empty) and row 1 (one key: the output is a raw V value, up
    # to ~30 with the outlier channels, whose BF16 rounding alone exceeds 2e-2) are checked bit for bit below
    _check(out, ref, flash, nonempty=np.arange(batch) >= 2)
    o = out.cpu()
    assert torch.equal(o[0], torch.zeros_like(o[0])) and torch.isneginf(lse[0]).all()
    # one key: P = 1, so the output is (e2m1 * e4m3) * g of that key's V, rounded to BF16
    slot = int(pt[1, idx[1, 0] // 64]) * 64 + idx[1, 0] % 64
    v1 = nvfp4.bf16_bits(nvfp4.dequant(pool.v_pay[slot], pool.v_sf[slot], pool.gv))
    want = np.repeat(v1, 8, axis=0)
    assert np.array_equal(o[1].view(torch.int16).numpy().view(np.uint16), want)


def test_decode_lengths_past_the_table_width():
    """Positions at or past a table row's pitch (table_stride * page_size) are skipped keys even when seq_lens reaches
    beyond: the table is a contiguous [batch, 30] view into a longer buffer whose next entries (the next row, and after
    the last row a tail) are valid page ids, so a read past a row would pick up real keys and change the output."""
    pool, pt, idx, q = _small_case(seed=11)
    batch, width = idx.shape[0], 30
    buf = torch.zeros(batch * width + 64, dtype=torch.int32)
    buf[:batch * width] = pt[:, :width].reshape(-1)
    buf[batch * width:] = pt[0, :64] if pt.shape[1] >= 64 else pt[0, torch.arange(64) % pt.shape[1]]
    table = buf.cuda()[:batch * width].view(batch, width)
    assert table.stride(0) == width
    seq = np.full(batch, 3008, np.int32)                     # past the 30 * 64 = 1920 positions the table holds
    scale = 0.0884
    out = ops.sparse_decode(q.cuda(), pool.raw, table, idx.cuda(), _dev(seq), scale, page_size=64, splits=2)
    clamped = np.full(batch, width * 64, np.int32)
    ref, flash, _ = _oracle(pool.raw, bf16_numpy(q), pt[:, :width].numpy(), 64, np.arange(batch), idx.numpy(), None,
                            clamped, scale)
    _check(out, ref, flash)


@pytest.mark.parametrize('splits', [1, 2, 7, 22, 64])
def test_decode_splits(splits):
    pool, pt, idx, q = _small_case(seed=splits)
    seq = np.full(idx.shape[0], 3008, np.int32)
    scale = 0.0884
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), idx.cuda(), _dev(seq), scale, page_size=64,
                            splits=splits)
    ref, flash, _ = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(idx.shape[0]), idx.numpy(), None,
                            seq, scale)
    _check(out, ref, flash)


def test_decode_token_table_equals_page_table_and_row_map():
    """page_size 1 through the token-granular table gives the same bits as page_size 64; rows may share a request
    (row_req, as verify rows do); strided q; FP16 output."""
    pool, pt, idx, q = _small_case(seed=11, batch=4)
    tt = workloads.token_table(pt, 64)
    seq = torch.full((4,), 3008, dtype=torch.int32)
    a = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), idx.cuda(), seq.cuda(), 0.09, page_size=64)
    b = ops.sparse_decode(q.cuda(), pool.raw, tt.cuda(), idx.cuda(), seq.cuda(), 0.09, page_size=1)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # 8 rows over the 4 requests, q a strided view, FP16 out
    rows_req = torch.tensor([0, 0, 1, 2, 3, 3, 2, 1])
    big = torch.zeros(8, 40, 136, dtype=torch.bfloat16, device='cuda')
    qv = big[:, 4:36, :128]
    qv.copy_(torch.cat([q, q.flip(0)]).cuda() * 0.5)
    assert not qv.is_contiguous()
    idx8 = idx[rows_req]
    out = torch.empty(8, 32, 128, dtype=torch.float16, device='cuda')
    ops.sparse_decode(qv, pool.raw, pt.cuda(), idx8.cuda(), seq[rows_req].cuda(), 0.09, page_size=64,
                      row_req=rows_req.cuda(), out=out)
    ref, flash, _ = _oracle(pool.raw, bf16_numpy(qv), pt.numpy(), 64, rows_req.numpy(), idx8.numpy(), None,
                            seq[rows_req].numpy(), 0.09)
    _check(out, ref, flash)


def test_graph_replay_equals_eager():
    pool, pt, idx, q = _small_case(seed=5, batch=8)
    seq = torch.full((8,), 3008, dtype=torch.int32, device='cuda')
    splits = 4
    ws = ops.new_workspace('cuda', 8, 32, 128, splits)
    qs = q.cuda().clone()
    out = torch.empty(8, 32, 128, dtype=torch.bfloat16, device='cuda')
    args = (pool.raw, pt.cuda(), idx.cuda(), seq, 0.0884)
    ops.sparse_decode(qs, *args, page_size=64, out=out, splits=splits, ws=ws)   # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.sparse_decode(qs, *args, page_size=64, out=out, splits=splits, ws=ws)
    gen = torch.Generator().manual_seed(99)
    for _ in range(4):
        q2 = (torch.randn(8, 32, 128, generator=gen) * 2).to(torch.bfloat16).cuda()
        qs.copy_(q2)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = ops.sparse_decode(q2, *args, page_size=64, splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16), eager.view(torch.int16))


@pytest.mark.parametrize('heads,qh,batch,ctx,topk,splits', [
    (1, 16, 5, 3008, 700, 3),    # one KV head, group 16: 8-wave workgroups of 1 KV head x 8 slices
    (1, 4, 6, 3008, 700, 3),     # group 4: a partial block of 4 heads, so 128-B lines straddle splits and rows
    (2, 32, 4, 3008, 700, 1),    # 1 KV head x 8 slices, no partials
    (6, 24, 3, 3008, 700, 2),    # KV heads not a multiple of 4: 1 KV head x 8 slices
    (8, 64, 40, 512, 300, 8),    # 640 units of 4 KV heads: past one round, 4-wave workgroups of 4 heads x 1 slice
    (12, 48, 32, 512, 300, 8),   # 768 units of 4 KV heads, 3 head groups per row: 4-wave, 4 heads x 1 slice
    (4, 32, 64, 512, 300, 4),    # exactly 256 units: 8-wave workgroups of 4 KV heads x 2 slices, with partials
])
def test_decode_head_layouts(heads, qh, batch, ctx, topk, splits):
    """KV head counts and GQA groups over the workgroup shapes (on 256 CUs: 4 KV heads x 2 slices at one round of
    workgroups, 4 heads x 1 slice in 4-wave workgroups past it, 1 KV head x 8 slices for few rows), with or without
    key splits."""
    pool, pt, idx, q = _small_case(seed=heads * 100 + batch, batch=batch, ctx=ctx, heads=heads, qh=qh, topk=topk)
    seq = np.full(batch, ctx, np.int32)
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), idx.cuda(), _dev(seq), 0.0884, page_size=64,
                            splits=splits)
    ref, flash, _ = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(batch), idx.numpy(), None, seq,
                            0.0884)
    _check(out, ref, flash)


@pytest.mark.parametrize('splits', [1, 8])
def test_decode_full_gqa_workload(splits):
    """Batch 32, 32 q / 4 KV heads, context 32768, top-2048 over a 1M-slot pool built on the GPU: every row against
    the oracle on the pool bytes the GPU wrote (one key split: 1 KV head per workgroup, 8 slices merged in LDS; 8
    splits: 4 KV heads per workgroup and cross-workgroup partials)."""
    w = workloads.WORKLOADS['gqa_decode_b32']
    gen = workloads.generator('cuda', 20261029)
    k = workloads.kv_tensor(w.slots, w.kv_heads, w.dim, gen, 'cuda')
    k_pay, k_sf, gk = ops.nvfp4_encode(k)
    del k
    v = workloads.kv_tensor(w.slots, w.kv_heads, w.dim, gen, 'cuda')
    v_pay, v_sf, gv = ops.nvfp4_encode(v)
    del v
    raw = (k_pay, v_pay, k_sf, v_sf, gk, gv)
    q = (torch.randn(w.batch, w.q_heads, w.dim, generator=gen, device='cuda')).to(torch.bfloat16)
    pt = workloads.page_table(w.batch, w.ctx, w.page, gen, 'cuda')
    idx = workloads.index_lists(w.batch, w.ctx, w.topk, gen, 'cuda')
    seq = torch.full((w.batch,), w.ctx, dtype=torch.int32, device='cuda')
    scale = 1 / math.sqrt(w.dim)
    out = ops.sparse_decode(q, raw, pt, idx, seq, scale, page_size=w.page, splits=splits)
    ref, flash, _ = _oracle(raw, bf16_numpy(q), pt.cpu().numpy(), w.page, np.arange(w.batch), idx.cpu().numpy(),
                            None, seq.cpu().numpy(), scale)
    _check(out, ref, flash, strict=True)


def test_decode_long_context_workload():
    """Batch 4 at context 524288 (a 2M-slot pool, 1.2 GB of NVFP4 K/V, far beyond the MALL), top-2048 with half the
    keys in the last 4096 positions, at the default key splits and at 8 and 16: every row against the oracle."""
    w = workloads.WORKLOADS['long_ctx_decode_b4']
    gen = workloads.generator('cuda', 20261106)
    k = workloads.kv_tensor(w.slots, w.kv_heads, w.dim, gen, 'cuda')
    k_pay, k_sf, gk = ops.nvfp4_encode(k)
    del k
    v = workloads.kv_tensor(w.slots, w.kv_heads, w.dim, gen, 'cuda')
    v_pay, v_sf, gv = ops.nvfp4_encode(v)
    del v
    raw = (k_pay, v_pay, k_sf, v_sf, gk, gv)
    q = torch.randn(w.batch, w.q_heads, w.dim, generator=gen, device='cuda').to(torch.bfloat16)
    pt = workloads.page_table(w.batch, w.ctx, w.page, gen, 'cuda')
    idx = workloads.index_lists(w.batch, w.ctx, w.topk, gen, 'cuda', w.index_mode)
    seq = torch.full((w.batch,), w.ctx, dtype=torch.int32, device='cuda')
    scale = 1 / math.sqrt(w.dim)
    assert ops.default_splits(w.batch, w.kv_heads, w.topk) == 4
    ref, flash, _ = _oracle(raw, bf16_numpy(q), pt.cpu().numpy(), w.page, np.arange(w.batch), idx.cpu().numpy(),
                            None, seq.cpu().numpy(), scale)
    for splits in (None, 8, 16):   # the default, and the split counts a caller may still ask for
        out = ops.sparse_decode(q, raw, pt, idx, seq, scale, page_size=w.page, splits=splits)
        _check(out, ref, flash, strict=True)


@pytest.mark.parametrize('batch,splits', [(96, 1), (40, 3)])
def test_decode_past_one_round_of_workgroups(batch, splits):
    """Unit counts beyond one round of 8-wave workgroups (384 and 480 at 4 KV heads) run 4-wave workgroups, two per
    CU: every row matches the oracle. Outputs here reach magnitude 22, where one BF16 step is 0.125, so the absolute
    bound applies beyond the BF16 rounding of the reference value (the flash-precision reference errs as much)."""
    pool, pt, idx, q = _small_case(seed=50 + batch, batch=batch, ctx=1024, topk=400)
    seq = np.full(batch, 1024, np.int32)
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), idx.cuda(), torch.from_numpy(seq).cuda(), 0.09,
                            page_size=64, splits=splits)
    ref, flash, _ = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(batch), idx.numpy(), None, seq, 0.09)
    _check(out, ref, flash)


@pytest.mark.parametrize('splits', [4, 5])
def test_decode_two_kv_heads_per_workgroup(splits):
    """32 rows x 4 KV heads with 4 or 5 key splits fill the CUs with workgroups of 2 KV heads (8 waves at 256
    workgroups, 4 at 320), with -1 holes, a short row, a short and an empty key list and a causal limit: every row
    against the oracle on SGLang's split pool, and the interleaved pool's bits equal to the split pool's."""
    pool, pt, idx, q = _small_case(seed=50 + splits, batch=32)
    idx = idx.numpy().copy()
    idx[3, ::5] = -1
    seq = np.full(32, 3008, np.int32)
    seq[7] = 900
    counts = np.full(32, idx.shape[1], np.int32)
    counts[11] = 150                      # a short list: its last splits hold no key
    counts[12] = 0                        # no key at all: zeros, LSE -inf
    qpos = np.full(32, 1 << 30, np.int32)
    qpos[13] = 1200                       # a causal limit
    scale = 128 ** -0.5
    lse = torch.empty(32, 32, dtype=torch.float32, device='cuda')
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), _dev(idx), _dev(seq), scale, page_size=64, lse=lse,
                            counts=_dev(counts), query_pos=_dev(qpos), splits=splits)
    ref, flash, lse_ref = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(32), idx, counts, seq, scale,
                                  qpos)
    live = np.arange(32) != 12
    _check(out, ref, flash, nonempty=live)
    assert not out[12].any() and torch.isneginf(lse[12]).all()
    assert np.abs(lse.cpu().numpy()[live] - lse_ref[live]).max() < 2e-3
    il = KVPool(pool.raw[0].shape[0], 4, 128, layout='interleaved', gk=pool.raw[4].clone(), gv=pool.raw[5].clone())
    for dst, src in zip((il.k_pay, il.v_pay, il.k_sf, il.v_sf), pool.raw[:4]):
        dst.copy_(src)
    out2 = ops.sparse_decode(q.cuda(), il.raw, pt.cuda(), _dev(idx), _dev(seq), scale, page_size=64,
                             counts=_dev(counts), query_pos=_dev(qpos), splits=splits)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


@pytest.mark.parametrize('kv,qh,batch', [(4, 16, 32), (2, 16, 64), (8, 64, 16), (4, 8, 32)])
def test_decode_paired_waves_head_layouts(kv, qh, batch):
    """Launches of 256 workgroups of 2 KV heads (8 waves each, one wave per pair of KV heads): GQA groups of 8, 4 and 2
    (columns past the group are padding), one pair (2 KV heads) and four pairs (8 KV heads), with -1 holes and a
    short row: every row against the oracle, on SGLang's split pool and on the interleaved pool bit for bit."""
    pool, pt, idx, q = _small_case(seed=kv * 100 + qh, batch=batch, heads=kv, qh=qh)
    assert ops.decode_shape(batch, kv, 4)[:3] == (2, 8, 256)
    idx = idx.numpy().copy()
    idx[1, ::6] = -1
    seq = np.full(batch, 3008, np.int32)
    seq[2] = 1100
    scale = 128 ** -0.5
    lse = torch.empty(batch, qh, dtype=torch.float32, device='cuda')
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), _dev(idx), _dev(seq), scale, page_size=64, lse=lse,
                            splits=4)
    ref, flash, lse_ref = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(batch), idx, None, seq, scale)
    _check(out, ref, flash)
    assert np.abs(lse.cpu().numpy() - lse_ref).max() < 2e-3
    il = KVPool(pool.raw[0].shape[0], kv, 128, layout='interleaved', gk=pool.raw[4].clone(), gv=pool.raw[5].clone())
    for dst, src in zip((il.k_pay, il.v_pay, il.k_sf, il.v_sf), pool.raw[:4]):
        dst.copy_(src)
    out2 = ops.sparse_decode(q.cuda(), il.raw, pt.cuda(), _dev(idx), _dev(seq), scale, page_size=64, splits=4)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


@pytest.mark.parametrize('splits', [4, 5])
def test_decode_nan_scales_stay_in_their_head(splits):
    """A NaN E4M3 scale byte (0x7F / 0xFF) in a live key's row reaches exactly the outputs the oracle makes NaN: a K
    scale the whole of its KV head's query heads, a V scale the 16 dims of its block in those heads, in every row
    that reads the key. With 4 splits one wave covers the two KV heads of a pair (its zero blocks must not carry the
    NaN to the other head), with 5 one wave per KV head; on both pool layouts."""
    pool, pt, idx, q = _small_case(seed=71, batch=32)
    idx = idx.numpy()
    seq = np.full(32, 3008, np.int32)
    table = pt.numpy()
    slot = lambda r, c: int(attention.slots_of(table, r, idx[r, c:c + 1], 64)[0])
    k_sf, v_sf = pool.raw[2], pool.raw[3]      # [slots, 4 heads, 8 blocks]
    k_sf[slot(5, 17), 1, 3] = 0x7F             # K scale, KV head 1: query heads 8..15 of the rows reading it
    v_sf[slot(9, 300), 2, 5] = 0xFF            # V scale, KV head 2, dims 80..95 of query heads 16..23
    k_sf[slot(20, 611), 0, 0] = 0xFF           # K scale, KV head 0 (a pair's first head), the last split
    scale = 128 ** -0.5
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), _dev(idx), _dev(seq), scale, page_size=64, splits=splits)
    ref, flash, _ = _oracle(pool.raw, bf16_numpy(q), table, 64, np.arange(32), idx, None, seq, scale)
    got = out.float().cpu().numpy()
    nan = np.isnan(ref)
    assert nan[5, 8:16].all() and nan[9, 16:24, 80:96].all() and not nan[9, 16:24, :80].any() and nan[20, :8].all()
    assert np.array_equal(np.isnan(got), nan)
    _check(torch.nan_to_num(out.float(), nan=0.0), np.where(nan, 0.0, ref), np.where(nan, 0.0, flash),
           nonempty=~nan)
    il = KVPool(pool.raw[0].shape[0], 4, 128, layout='interleaved', gk=pool.raw[4].clone(), gv=pool.raw[5].clone())
    for dst, src in zip((il.k_pay, il.v_pay, il.k_sf, il.v_sf), pool.raw[:4]):
        dst.copy_(src)
    out2 = ops.sparse_decode(q.cuda(), il.raw, pt.cuda(), _dev(idx), _dev(seq), scale, page_size=64, splits=splits)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


@pytest.mark.parametrize('splits', [2, 4, 7])
def test_decode_partials_at_the_value_limit(splits):
    """Every V value at +-6 x 448 (E2M1 code +-6.0 under the largest finite E4M3 scale byte, 0x7E): a split's output
    normalized by its own sum, which its FP16 partial holds before the V global scale is applied, reaches 2688 in
    magnitude (dims 0..63 are +2688 in every key, so every split's partial and the output are exactly that times
    the global scale, 1/4096 here; the other dims have random signs). Against the oracle, with 2, 4 and 7 key
    splits."""
    pool, pt, idx, q = _small_case(seed=83, batch=8)
    v_pay, v_sf = pool.raw[1], pool.raw[3]          # [slots, 4 heads, 64] payload bytes, [slots, 4 heads, 8] scales
    gen = torch.Generator().manual_seed(5)
    signs = torch.randint(0, 2, (v_pay.shape[0], v_pay.shape[1], 128), generator=gen, dtype=torch.uint8)
    signs[:, :, :64] = 0
    nib = (7 | (signs << 3)).to(torch.uint8)        # 0x7: +6.0, 0xF: -6.0
    v_pay.copy_((nib[:, :, 0::2] | (nib[:, :, 1::2] << 4)).cuda())
    v_sf.fill_(0x7E)
    pool.raw[5].fill_(1.0 / 4096)                   # applied after the merge: outputs up to 0.65625, partials 2688
    seq = np.full(8, 3008, np.int32)
    scale = 128 ** -0.5
    out = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), idx.cuda(), _dev(seq), scale, page_size=64, splits=splits)
    ref, flash, _ = _oracle(pool.raw, bf16_numpy(q), pt.numpy(), 64, np.arange(8), idx.numpy(), None, seq, scale)
    gv = float(pool.raw[5].item())
    assert np.allclose(ref[:, :, :64], 2688.0 * gv)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    assert np.array_equal(got[:, :, :64], np.full_like(got[:, :, :64], float(torch.tensor(2688.0 * gv).bfloat16())))
    _check(out, ref, flash)


@pytest.mark.parametrize('batch,splits', [(32, 4), (6, 3)])
def test_decode_timeline(batch, splits):
    """The per-wave timeline (xt_decode_timeline) of a launch of paired waves (32 rows x 4 KV heads x 4 splits) and of
    one with 1 KV head per workgroup: every wave of every workgroup stamps its phases in order, exactly one workgroup
    per (row, KV head group) merges the splits, and the outputs are those of the same launch without the timeline."""
    pool, pt, idx, q = _small_case(seed=90 + batch, batch=batch)
    seq = np.full(batch, 3008, np.int32)
    args = (q.cuda(), pool.raw, pt.cuda(), idx.cuda(), _dev(seq), 128 ** -0.5)
    plain = ops.sparse_decode(*args, page_size=64, splits=splits)
    hpw, waves, units = ops.decode_shape(batch, 4, splits)
    with ops.decode_timeline(units * waves + 16) as tl:
        timed = ops.sparse_decode(*args, page_size=64, splits=splits)
    assert torch.equal(plain.view(torch.int16), timed.view(torch.int16))
    st = tl.stamps
    assert not st[units * waves:].any()                        # nothing past the launch's waves
    st = st[:units * waves].reshape(units, waves, 8)
    reached = st[:, :, :7]                                      # every wave reaches phases 0..6 (splits > 1)
    assert (reached > 0).all()
    assert (np.diff(reached, axis=2) >= 0).all()
    last = st[:, :, 7] > 0
    assert (last.all(1) | ~last.any(1)).all()                   # all waves of a workgroup, or none
    assert last.all(1).sum() == batch * (4 // hpw)              # one last arriver per (row, KV head group)
    assert (st[:, :, 7][last] >= st[:, :, 6][last]).all()


def test_interleaved_pool_equals_split_pool():
    """The same bytes in the interleaved layout (one buffer; per slot each head's [K row | V row], then each head's
    [K scales | V scales]) and in SGLang's four buffers give the same bits."""
    pool, pt, idx, q = _small_case(seed=21, batch=4)
    slots = pool.raw[0].shape[0]
    il = KVPool(slots, 4, 128, layout='interleaved', gk=pool.raw[4].clone(), gv=pool.raw[5].clone())
    for dst, src in zip((il.k_pay, il.v_pay, il.k_sf, il.v_sf), pool.raw[:4]):
        dst.copy_(src)
    assert il.k_pay.stride()[:2] == (576, 128) and il.v_sf.stride()[:2] == (576, 16) and not il.k_pay.is_contiguous()
    seq = torch.full((4,), 3008, dtype=torch.int32, device='cuda')
    a = ops.sparse_decode(q.cuda(), pool.raw, pt.cuda(), idx.cuda(), seq, 0.09, page_size=64)
    b = ops.sparse_decode(q.cuda(), il.raw, pt.cuda(), idx.cuda(), seq, 0.09, page_size=64)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize('heads,qh', [(1, 16), (2, 16), (8, 64)])
def test_interleaved_pool_any_head_count(heads, qh):
    """KVPool's interleaved layout at 1, 2 and 8 KV heads (head strides of the pairs and of the scales through the
    ABI, the single-head default, the paired-scale load): quantize-on-append into it gives the split pool's bytes,
    and the decode gives the split pool's bits, for 1 and 3 key splits."""
    gen = workloads.generator('cpu', 40 + heads)
    batch, ctx, page, topk = 3, 1024, 64, 300
    k = workloads.kv_tensor(batch * ctx, heads, 128, gen, 'cpu').cuda()
    v = workloads.kv_tensor(batch * ctx, heads, 128, gen, 'cpu').cuda()
    slots = torch.arange(batch * ctx, device='cuda')
    pools = {}
    for layout in ('split', 'interleaved'):
        pool = KVPool(batch * ctx, heads, 128, layout=layout)
        pool.set_global_scales(k, v)
        pool.append(k, v, slots)
        pools[layout] = pool
    for a_, b_ in zip(pools['split'].raw[:4], pools['interleaved'].raw[:4]):
        assert torch.equal(a_, b_)
    pt = workloads.page_table(batch, ctx, page, gen, 'cpu').cuda()
    idx = workloads.index_lists(batch, ctx, topk, gen, 'cpu').cuda()
    q = (torch.randn(batch, qh, 128, generator=gen) * 2).to(torch.bfloat16).cuda()
    seq = torch.full((batch,), ctx, dtype=torch.int32, device='cuda')
    for splits in (1, 3):
        a_ = ops.sparse_decode(q, pools['split'].raw, pt, idx, seq, 0.09, page_size=page, splits=splits)
        b_ = ops.sparse_decode(q, pools['interleaved'].raw, pt, idx, seq, 0.09, page_size=page, splits=splits)
        assert torch.equal(a_.view(torch.int16), b_.view(torch.int16)), splits


def test_one_workspace_serves_calls_of_any_shape():
    """A workspace left by a call with few rows (its partials written just past the counters) serves a later call
    with more rows and a sparse-MLA call: every result equals the one from a fresh workspace, bit for bit."""
    pool, pt, idx, q = _small_case(seed=31, batch=8)
    seq = torch.full((8,), 3008, dtype=torch.int32, device='cuda')
    ws = torch.zeros(ops.decode_workspace_bytes(8, 32, 128, 16), dtype=torch.uint8, device='cuda')
    runs = [(2, 16), (8, 3), (5, 7), (8, 2)]
    for rows, splits in runs:
        got = ops.sparse_decode(q[:rows].cuda(), pool.raw, pt[:rows].cuda(), idx[:rows].cuda(), seq[:rows], 0.09,
                                page_size=64, splits=splits, ws=ws)
        fresh = ops.sparse_decode(q[:rows].cuda(), pool.raw, pt[:rows].cuda(), idx[:rows].cuda(), seq[:rows], 0.09,
                                  page_size=64, splits=splits,
                                  ws=ops.new_workspace('cuda', rows, 32, 128, splits))
        assert torch.equal(got.view(torch.int16), fresh.view(torch.int16)), (rows, splits)
    assert not ws[:65536].any()   # the counters are left zero


def test_graph_survives_a_grown_workspace():
    """A graph captured on the cached per-device workspace keeps replaying correctly after a larger eager call has
    grown that workspace: the old buffer stays allocated (the graph holds its address), so a tensor allocated and
    filled afterwards is untouched by the replays and every replay equals the eager result."""
    pool, pt, idx, q = _small_case(seed=41, batch=8)
    seq = torch.full((8,), 3008, dtype=torch.int32, device='cuda')
    args = (pool.raw, pt.cuda(), idx.cuda(), seq, 0.0884)
    qs = q.cuda().clone()
    out = torch.empty(8, 32, 128, dtype=torch.bfloat16, device='cuda')
    ops.workspace('cuda', ops.decode_workspace_bytes(8, 32, 128, 4))
    ops.sparse_decode(qs, *args, page_size=64, out=out, splits=4)   # the cached workspace, warm-up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.sparse_decode(qs, *args, page_size=64, out=out, splits=4)
    # an eager call that needs more bytes than the cached workspace holds replaces it
    before = ops._cached_workspace_bytes(torch.device('cuda'))
    ops.workspace('cuda', before + (1 << 20))
    ops.sparse_decode(qs, *args, page_size=64, splits=48)
    assert ops._cached_workspace_bytes(torch.device('cuda')) > before
    torch.cuda.synchronize()
    canary = torch.full((before // 4 + 4096,), 1234567, dtype=torch.int32, device='cuda')
    eager = ops.sparse_decode(qs, *args, page_size=64, splits=4, ws=ops.new_workspace('cuda', 8, 32, 128, 4))
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        assert bool((canary == 1234567).all())
