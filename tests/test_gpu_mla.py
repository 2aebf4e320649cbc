"""Sparse MLA on the GPU against the FP64 oracle (tests/ds_sparse_mla_check.py:44-67 restated for an NVFP4 latent +
BF16 rope cache): errors measured as the reference measures them (max |err| / max |ref| < 1e-2, rms err / rms ref <
4e-3, tests/ds_sparse_mla_check.py:70-75, :160), plus the absolute bound max 2e-2 / mean 2e-3; rows without keys
exactly 0 with LSE -inf; two key lists; sink; key splits; graph replay equal to eager; the decode and prefill
workloads at their full sizes (64 rows at context 131072, a 2048-row causal chunk, top-2048) and latents whose
per-token magnitudes span three decades (tests/qsa_fp4_check.py:26-34)."""
import math

import numpy as np
import pytest
import torch

from oracle import attention
from xtier_amd import ops, workloads
from xtier_amd.pool import LatentPool

pytestmark = pytest.mark.gpu


def _pool(w, seed, layout='interleaved', slots=None):
    slots = slots or w.slots
    gen = workloads.generator('cuda', seed)
    lat, rope = workloads.mla_cache_rows(w, gen, 'cuda', 0, slots)
    pool = LatentPool(slots, w.latent, w.rope, 'cuda', layout=layout)
    pool.set_global_scale(lat)
    pool.append(lat, rope, torch.arange(slots, device='cuda'), saturate=False)
    return pool


def _host(pool):
    return (pool.pay.cpu().numpy(), pool.scales.cpu().numpy(), pool.rope.float().cpu().numpy(),
            np.float32(pool.g.item()))


def _ref(q, pool, idx, lengths, sink, scale, extra=None):
    pay, sc, rope, g = _host(pool)
    ex = None
    if extra is not None:
        p2, i2, l2 = extra
        ex = _host(p2) + (i2.cpu().numpy(), None if l2 is None else l2.cpu().numpy())
    return attention.sparse_mla(q.float().cpu().numpy(), pay, sc, rope, g, idx.cpu().numpy(),
                                None if lengths is None else lengths.cpu().numpy(),
                                None if sink is None else sink.cpu().numpy(), scale, extra=ex)


def _check(out, lse, ref, ref_lse, nonempty=None, bf16_slack=False):
    """bf16_slack: the absolute max bound applies beyond the BF16 rounding of the reference value (for outputs that
    are single latent values of magnitude up to ~30, where one BF16 step is 0.125)."""
    o = out.reshape(ref.shape).float().cpu().numpy().astype(np.float64)
    sel = slice(None) if nonempty is None else nonempty
    o_s, r_s = o[sel], ref[sel]
    assert np.isfinite(o_s).all()
    d = o_s - r_s
    max_rel = np.abs(d).max() / np.abs(r_s).max()
    rms_rel = np.sqrt((d ** 2).mean()) / np.sqrt((r_s ** 2).mean())
    assert max_rel < 1e-2 and rms_rel < 4e-3, (max_rel, rms_rel)
    slack = np.exp2(np.floor(np.log2(np.maximum(np.abs(r_s), 1e-30))) - 8) if bf16_slack else 0.0
    assert (np.abs(d) - slack).max() <= 2e-2 and np.abs(d).mean() <= 2e-3, (np.abs(d).max(), np.abs(d).mean())
    if lse is not None:
        l_ = lse.reshape(ref_lse.shape).cpu().numpy()
        fin = np.isfinite(ref_lse)
        assert (np.isfinite(l_) == fin).all()
        assert np.abs(l_[fin] - ref_lse[fin]).max() < 2e-3


def _case(seed, rows=5, heads=128, ctx=4096, topk=300, causal=False):
    w = workloads.MlaWorkload('mla_test', rows, heads, ctx, topk, causal=causal)
    inp = workloads.mla_inputs(w, seed, 'cuda')
    return w, inp


@pytest.mark.parametrize('splits', [1, 3])
@pytest.mark.parametrize('use_sink', [False, True])
def test_mla_small(splits, use_sink):
    w, inp = _case(20261023 + splits)
    pool = _pool(w, 7)
    idx = inp.slots.clone()
    idx[1, ::4] = -1                                   # holes
    lengths = torch.full((w.rows,), w.topk, dtype=torch.int32, device='cuda')
    lengths[2] = 100                                   # a shorter list
    sink = (torch.randn(w.heads, device='cuda') * 2) if use_sink else None
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q[:, None], pool, idx[:, None], lengths, sink, scale, splits=splits)
    assert out.shape == (w.rows, 1, w.heads, 512) and lse.shape == (w.rows, w.heads, 1)
    ref, ref_lse = _ref(inp.q, pool, idx, lengths, sink, scale)
    _check(out, lse, ref, ref_lse)


@pytest.mark.parametrize('splits', [1, 3])
def test_mla_fp16_output(splits):
    """An FP16 output tensor (the one-split epilogue's swizzled LDS stage and the split merge's, both converting by
    RNE): within the tolerance of the oracle, and within an FP16 plus a BF16 rounding (bounded by 2^-7 of the larger
    magnitude, 2^-25 below FP16's normal range) of the same call's BF16 output, with the same LSE."""
    w, inp = _case(20261107 + splits, rows=6, heads=72)    # 72 heads: a wave with 8 padding heads
    pool = _pool(w, 11)
    scale = 1 / math.sqrt(576)
    out16 = torch.empty(w.rows, w.heads, 512, dtype=torch.float16, device='cuda')
    o16, lse16 = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale, out=out16, splits=splits)
    ob, lseb = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale, splits=splits)
    ref, ref_lse = _ref(inp.q, pool, inp.slots, None, None, scale)
    _check(o16, lse16, ref, ref_lse)
    a, b = o16.float(), ob.float()
    assert torch.equal(lse16, lseb)
    assert ((a - b).abs() <= torch.maximum(a.abs(), b.abs()) * 2.0 ** -7 + 2.0 ** -25).all()


@pytest.mark.parametrize('mag', [1e-4, 1e3, 1e6, 'mixed'])
def test_mla_query_magnitudes(mag):
    """Queries far from unit size (|q| ~ 1e-4, 1e3, 1e6, beyond FP16's range once scaled by scale * log2(e), and rows
    whose 128 heads span seven decades): the query enters the MFMA as q * 2^-e per head, exactly; outputs within the
    reference's tolerance of the FP64 oracle, the LSE within FP32 rounding of the scores."""
    w, inp = _case(31, rows=4)
    pool = _pool(w, 5)
    q = inp.q.float()
    if mag == 'mixed':
        q = q * (10.0 ** ((torch.arange(w.heads, device='cuda') % 8) - 4)).view(1, -1, 1)
    else:
        q = q * mag
    q = q.to(torch.bfloat16)
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(q[:, None], pool, inp.slots[:, None], None, None, scale, splits=2)
    ref, ref_lse = _ref(q, pool, inp.slots, None, None, scale)
    _check(out, None, ref, ref_lse, bf16_slack=True)
    got = lse.reshape(ref_lse.shape).cpu().numpy()
    assert np.isfinite(got).all()
    assert (np.abs(got - ref_lse) <= 2e-3 + 1e-6 * np.abs(ref_lse)).all()


def test_mla_rope_beyond_fp16_range():
    """Rope values of ~1e5 (beyond FP16's range; BF16 holds them) against a rope query scaled by 1e-5: the rope
    chunks run the BF16 MFMA on the cache's own BF16 values, so the scores stay finite and exact in their products."""
    w, inp = _case(13, rows=4)
    gen = workloads.generator('cuda', 6)
    lat, rope = workloads.mla_cache_rows(w, gen, 'cuda', 0, w.slots)
    rope = (rope.float() * 1e5).to(torch.bfloat16)
    pool = LatentPool(w.slots, w.latent, w.rope, 'cuda')
    pool.set_global_scale(lat)
    pool.append(lat, rope, torch.arange(w.slots, device='cuda'), saturate=False)
    q = inp.q.float()
    q[:, :, w.latent:] *= 1e-5
    q = q.to(torch.bfloat16)
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(q[:, None], pool, inp.slots[:, None], None, None, scale, splits=2)
    ref, ref_lse = _ref(q, pool, inp.slots, None, None, scale)
    _check(out, lse, ref, ref_lse, bf16_slack=True)


def test_mla_two_lists_empty_and_single_key_rows():
    """A window list in one cache followed by compressed keys in another (sparse_mla.py:109-118); row 0 has no valid
    key in either list (zeros, LSE -inf), row 1 a single key (its latent, rounded once to FP16 then BF16)."""
    w, inp = _case(11, rows=6)
    pool = _pool(w, 3)
    pool2 = _pool(w, 4, layout='split', slots=2048)
    gen = torch.Generator(device='cuda').manual_seed(5)
    idx2 = torch.randint(0, 2048, (w.rows, 64), generator=gen, device='cuda', dtype=torch.int32)
    len2 = torch.full((w.rows,), 64, dtype=torch.int32, device='cuda')
    idx = inp.slots.clone()
    lengths = torch.full((w.rows,), w.topk, dtype=torch.int32, device='cuda')
    lengths[0] = 0
    len2[0] = 0
    lengths[1] = 1
    len2[1] = 0
    sink = torch.randn(w.heads, device='cuda')
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q[:, None], pool, idx[:, None], lengths, sink, scale, extra_k_cache=pool2,
                              extra_indices=idx2[:, None], extra_topk_length=len2)
    ref, ref_lse = _ref(inp.q, pool, idx, lengths, sink, scale, extra=(pool2, idx2, len2))
    o = out[:, 0].float().cpu()
    assert torch.equal(o[0], torch.zeros_like(o[0])) and torch.isneginf(lse[0]).all()
    rows = np.arange(w.rows) >= 2
    _check(out[:, 0], lse[:, :, 0], ref, ref_lse, nonempty=rows)
    # one key: p = 1, so out = latent / (1 + exp(sink - s)), a raw latent value up to ~30 in size (outlier channels):
    # within the FP16 rounding of the dequantized latent and the BF16 rounding of the output, relative to the value
    d = np.abs(o[1].numpy().astype(np.float64) - ref[1])
    assert np.all(d <= np.abs(ref[1]) * (2.0 ** -8 + 2.0 ** -10) + 1e-6), d.max()


@pytest.mark.parametrize('heads', [100, 72, 64, 16])
def test_mla_fewer_heads(heads):
    """Head counts on both sides of the 64-head boundary between the two kernel forms, including waves of 32 heads
    that are partly or wholly padding."""
    w, inp = _case(31, rows=3, heads=heads)
    pool = _pool(w, 9)
    out, lse = ops.sparse_mla(inp.q, pool, inp.slots, None, None, 0.05)
    ref, ref_lse = _ref(inp.q, pool, inp.slots, None, None, 0.05)
    _check(out, lse, ref, ref_lse)


@pytest.mark.parametrize('heads,splits', [(128, 8), (128, 10), (100, 9), (16, 4), (64, 3)])
def test_mla_split_merge_head_and_split_counts(heads, splits):
    """Key splits with head counts that pad the last 16-head wave, more splits than 16-head waves, and splits that
    hold no key (700 keys over 10 splits of 96): every row against the oracle, and a second launch on the same
    workspace gives the same bits."""
    w, inp = _case(61 + splits, rows=6, heads=heads, topk=700)
    pool = _pool(w, 15)
    scale = 1 / math.sqrt(576)
    ws = torch.zeros(ops.mla_workspace_bytes(w.rows, heads, splits), dtype=torch.uint8, device='cuda')
    out, lse = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale, splits=splits, ws=ws)
    ref, ref_lse = _ref(inp.q, pool, inp.slots, None, None, scale)
    _check(out, lse, ref, ref_lse)
    out2, _ = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale, splits=splits, ws=ws)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


def test_mla_split_layout_equals_interleaved():
    w, inp = _case(41)
    a = _pool(w, 12, layout='interleaved')
    b = _pool(w, 12, layout='split')
    assert torch.equal(a.pay, b.pay) and torch.equal(a.scales, b.scales)
    oa, _ = ops.sparse_mla(inp.q, a, inp.slots, None, None, 0.05)
    ob, _ = ops.sparse_mla(inp.q, b, inp.slots, None, None, 0.05)
    assert torch.equal(oa.view(torch.int16), ob.view(torch.int16))


def test_mla_decode_batch64_all_rows():
    """64 rows at context 16384 (a 1M-token cache), top-2048 each, the decode workload's shape with a smaller context:
    every row against the oracle."""
    w = workloads.MlaWorkload('mla_decode_b64_ctx16k', 64, 128, 16384, 2048)
    inp = workloads.mla_inputs(w, 20261029, 'cuda')
    pool = _pool(w, 13)
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q[:, None], pool, inp.slots[:, None], None, None, scale)
    ref, ref_lse = _ref(inp.q, pool, inp.slots, None, None, scale)
    _check(out, lse, ref, ref_lse)


def test_mla_causal_prefill_rows():
    w, inp = _case(51, rows=96, ctx=4096, topk=512, causal=True)
    pool = _pool(w, 14)
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale)
    ref, ref_lse = _ref(inp.q, pool, inp.slots, None, None, scale)
    _check(out, lse, ref, ref_lse)


def test_mla_long_key_list_takes_enough_splits():
    """A key list longer than one split's LDS slot list holds (4000 keys) over many rows: the default split count
    rises to fit (2 here, where the one-per-CU heuristic alone gives 1), and the result matches the oracle on sampled
    rows."""
    from xtier_amd import _lib
    limit = _lib.lib().xt_sparse_mla_max_split_keys(0)
    assert 2048 < limit < 4000
    assert ops.default_mla_splits(288, 4000) == 2 and ops.default_mla_splits(288, 2048) == 1
    w, inp = _case(71, rows=288, ctx=8192, topk=4000)
    pool = _pool(w, 16)
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale)
    rows = torch.tensor([0, 1, 143, 286, 287], device='cuda')
    ref, ref_lse = _ref(inp.q[rows], pool, inp.slots[rows], None, None, scale)
    _check(out[rows], lse[rows], ref, ref_lse)
    with pytest.raises(NotImplementedError):
        ops.sparse_mla(inp.q[:2], pool, inp.slots[:2], None, None, scale, splits=1)


def test_mla_graph_replay_equals_eager():
    w, inp = _case(61, rows=8)
    pool = _pool(w, 15)
    splits = 2
    ws = torch.zeros(ops.mla_workspace_bytes(w.rows, w.heads, splits), dtype=torch.uint8, device='cuda')
    qs = inp.q.clone()
    out = torch.empty(w.rows, w.heads, 512, dtype=torch.bfloat16, device='cuda')
    lse = torch.empty(w.rows, w.heads, dtype=torch.float32, device='cuda')
    ops.sparse_mla(qs, pool, inp.slots, None, None, 0.05, out=out, lse=lse, splits=splits, ws=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.sparse_mla(qs, pool, inp.slots, None, None, 0.05, out=out, lse=lse, splits=splits, ws=ws)
    gen = torch.Generator(device='cuda').manual_seed(3)
    for _ in range(3):
        qs.copy_((torch.randn(qs.shape, generator=gen, device='cuda') * 0.5).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager, _ = ops.sparse_mla(qs, pool, inp.slots, None, None, 0.05, splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16))


def _compact_ref(q, pool, idx, scale):
    """The oracle on host copies of only the cache rows the lists name (a full-size cache stays on the GPU)."""
    flat = idx.reshape(-1).long()
    ok = flat >= 0
    uniq, inv = torch.unique(flat[ok], return_inverse=True)
    host = (pool.pay[uniq].cpu().numpy(), pool.scales[uniq].cpu().numpy(), pool.rope[uniq].float().cpu().numpy(),
            np.float32(pool.g.item()))
    local = torch.full_like(flat, -1)
    local[ok] = inv
    return attention.sparse_mla(q.float().cpu().numpy(), *host, local.reshape(idx.shape).cpu().numpy(), None, None,
                                scale)


def test_mla_decode_workload_full_size():
    """The decode workload as measured: 64 rows at context 131072 (an 8.4M-token cache), 128 heads, top-2048, default
    splits; every row against the oracle."""
    w = workloads.MLA_WORKLOADS['mla_decode_b64']
    inp = workloads.mla_inputs(w, 20261029, 'cuda')
    pool = _pool(w, 13)
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q[:, None], pool, inp.slots[:, None], None, None, scale)
    ref, ref_lse = _compact_ref(inp.q, pool, inp.slots, scale)
    _check(out, lse, ref, ref_lse)


def test_mla_prefill_chunk_full_size_sampled_rows():
    """The prefill workload as measured: a 2048-row causal chunk at the end of a 131072-token context, top-2048 per
    query (the 128 most recent included); the whole chunk runs, 64 rows spread over it are checked."""
    w = workloads.MLA_WORKLOADS['mla_prefill_2048']
    inp = workloads.mla_inputs(w, 20261029, 'cuda')
    pool = _pool(w, 14)
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale)
    rows = torch.cat([torch.arange(0, 2048, 33, device='cuda')[:62], torch.tensor([2046, 2047], device='cuda')])
    ref, ref_lse = _compact_ref(inp.q[rows], pool, inp.slots[rows], scale)
    _check(out[rows], lse[rows], ref, ref_lse)


def _scaled_pool(w, seed, mag, slots, layout='interleaved'):
    gen = workloads.generator('cuda', seed)
    lat, rope = workloads.mla_cache_rows(w, gen, 'cuda', 0, slots)
    lat, rope = (lat.float() * mag).to(torch.bfloat16), (rope.float() * mag).to(torch.bfloat16)
    pool = LatentPool(slots, w.latent, w.rope, 'cuda', layout=layout)
    pool.set_global_scale(lat)
    pool.append(lat, rope, torch.arange(slots, device='cuda'), saturate=False)
    return pool


@pytest.mark.parametrize('splits', [1, 2])
@pytest.mark.parametrize('mag0,mag1', [(1e-3, 1e-3), (1e-3, 10.0), (10.0, 3e-2)])
def test_mla_two_caches_of_different_scales(mag0, mag1, splits):
    """Two key lists over caches whose latents differ in size (global scales g0, g1 from ~4e-6 to ~0.1): P enters
    the value MFMA as FP16(p * g / max(g0, g1)), so neither a small g (P * g below FP16's normal range) nor a large
    one (P * g beyond FP16's range) costs precision; held to the reference's scale-free measures and the LSE to
    2e-3."""
    w, inp = _case(41, rows=6)
    pool = _scaled_pool(w, 8, mag0, w.slots)
    pool2 = _scaled_pool(w, 9, mag1, 2048, layout='split')
    gen = torch.Generator(device='cuda').manual_seed(6)
    idx2 = torch.randint(0, 2048, (w.rows, 96), generator=gen, device='cuda', dtype=torch.int32)
    len2 = torch.full((w.rows,), 96, dtype=torch.int32, device='cuda')
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q[:, None], pool, inp.slots[:, None], None, None, scale, extra_k_cache=pool2,
                              extra_indices=idx2[:, None], extra_topk_length=len2, splits=splits)
    ref, ref_lse = _ref(inp.q, pool, inp.slots, None, None, scale, extra=(pool2, idx2, len2))
    d = out[:, 0].float().cpu().numpy().astype(np.float64) - ref
    assert np.isfinite(d).all()
    max_rel = np.abs(d).max() / np.abs(ref).max()
    rms_rel = np.sqrt((d ** 2).mean()) / np.sqrt((ref ** 2).mean())
    assert max_rel < 1e-2 and rms_rel < 4e-3, (max_rel, rms_rel)
    got = lse[:, :, 0].cpu().numpy()
    assert np.all(np.abs(got - ref_lse) <= 2e-3 + 2.0 ** -20 * np.abs(ref_lse))


@pytest.mark.parametrize('top', [10.0, 1e-3, 3e3])
def test_mla_latent_magnitudes_over_three_decades(top):
    """Per-token latent and rope magnitudes spread over three decades, 10^U(-3, 0) * top: top 10 is the spread of
    tests/qsa_fp4_check.py:26-34; top 1e-3 makes g = amax / 2688 small enough that the small tokens' (e2m1 * e4m3) * g
    falls below FP16's normal range; top 3e3 puts the largest latents (~1e5) beyond FP16's range, which the FP16 split
    partials (normalized before g) must not reach. Outputs then span the data's own scale, so they are held to the
    reference test's scale-free measures (max |err| / max |ref| < 1e-2, rms err / rms ref < 4e-3,
    tests/ds_sparse_mla_check.py:70-75) and the LSE to 2e-3."""
    w = workloads.MlaWorkload('mla_spread', 16, 128, 8192, 2048)
    inp = workloads.mla_inputs(w, 20261023, 'cuda')
    gen = workloads.generator('cuda', 77)
    lat, rope = workloads.mla_cache_rows(w, gen, 'cuda', 0, w.slots)
    mag = top * 10 ** torch.empty(w.slots, 1, device='cuda').uniform_(-3, 0, generator=gen)
    lat = (lat.float() * mag).to(torch.bfloat16)
    rope = (rope.float() * mag).to(torch.bfloat16)
    pool = LatentPool(w.slots, w.latent, w.rope, 'cuda')
    pool.set_global_scale(lat)
    pool.append(lat, rope, torch.arange(w.slots, device='cuda'), saturate=False)
    scale = 1 / math.sqrt(576)
    out, lse = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale)
    ref, ref_lse = _compact_ref(inp.q, pool, inp.slots, scale)
    d = out.float().cpu().numpy().astype(np.float64) - ref
    max_rel = np.abs(d).max() / np.abs(ref).max()
    rms_rel = np.sqrt((d ** 2).mean()) / np.sqrt((ref ** 2).mean())
    assert max_rel < 1e-2 and rms_rel < 4e-3, (max_rel, rms_rel)
    # scores here reach ~15: the FP16 rounding of the scaled query (2^-11 relative) moves the LSE in proportion
    assert np.all(np.abs(lse.cpu().numpy() - ref_lse) <= 2e-3 + 2.0 ** -10 * np.abs(ref_lse))


@pytest.mark.parametrize('splits', [1, 2])
def test_mla_timeline(splits):
    """The per-wave timeline of the sparse MLA kernel (xt_mla_timeline): every wave of every (row, split) workgroup
    stamps its phases in order, and the outputs are those of the same launch without the timeline."""
    w, inp = _case(81, rows=6)
    pool = _pool(w, 17)
    scale = 1 / math.sqrt(576)
    plain, _ = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale, splits=splits)
    units = w.rows * splits
    with ops.decode_timeline(units * 8 + 8, kind='mla') as tl:
        timed, _ = ops.sparse_mla(inp.q, pool, inp.slots, None, None, scale, splits=splits)
    assert torch.equal(plain.view(torch.int16), timed.view(torch.int16))
    st = tl.stamps
    assert not st[units * 8:].any()
    st = st[:units * 8, :6]
    assert (st > 0).all() and (np.diff(st, axis=1) >= 0).all()
