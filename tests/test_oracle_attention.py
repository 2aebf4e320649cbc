"""The CPU oracle's attention, gather and merge pinned against torch float64 softmax (a separate implementation),
closed-form special cases and the invariants the reference's tests check."""
import numpy as np
import pytest
import torch

from oracle import attention, nvfp4


def _torch_ref(q, k, v, valid, scale):
    """tests/qsa_decode_check.py:14-26 form: per head softmax(k q * scale) @ v in float64, 0 without keys."""
    hq, group = q.shape[0], q.shape[0] // k.shape[1]
    out = torch.zeros(hq, v.shape[-1], dtype=torch.float64)
    sel = torch.from_numpy(np.nonzero(valid)[0])
    if sel.numel() == 0:
        return out.numpy()
    qd, kd, vd = (torch.from_numpy(np.asarray(t, np.float64)) for t in (q, k, v))
    for h in range(hq):
        s = (kd[sel, h // group] @ qd[h]) * scale
        out[h] = torch.softmax(s, 0) @ vd[sel, h // group]
    return out.numpy()


@pytest.mark.parametrize('n,hq,hkv', [(1, 8, 1), (37, 8, 2), (300, 32, 4)])
def test_softmax_matches_torch(n, hq, hkv):
    rng = np.random.default_rng(n)
    q = rng.standard_normal((hq, 64))
    k = rng.standard_normal((n, hkv, 64))
    v = rng.standard_normal((n, hkv, 64))
    valid = rng.random(n) < 0.8
    valid[0] = True
    got = attention.softmax_attention(q, k, v, valid, 0.125)
    assert np.allclose(got, _torch_ref(q, k, v, valid, 0.125), rtol=0, atol=1e-12)


def test_special_cases():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((4, 32))
    k = rng.standard_normal((5, 1, 32))
    v = rng.standard_normal((5, 1, 32))
    one = np.zeros(5, bool)
    one[3] = True
    assert np.array_equal(attention.softmax_attention(q, k, v, one, 0.3), np.repeat(v[3], 4, 0))   # P = 1
    assert not attention.softmax_attention(q, k, v, np.zeros(5, bool), 0.3).any()                   # empty row


@pytest.mark.parametrize('keys_per_split', [1, 7, 128, 1000])
def test_split_merge_equals_one_pass(keys_per_split):
    rng = np.random.default_rng(keys_per_split)
    q = rng.standard_normal((8, 128)) * 2
    k = rng.standard_normal((513, 1, 128))
    v = rng.standard_normal((513, 1, 128))
    valid = rng.random(513) < 0.7
    m, l, acc = attention.split_partials(q, k, v, valid, 0.09, keys_per_split)
    got = attention.merge_partials(m, l, acc)
    assert np.allclose(got, attention.softmax_attention(q, k, v, valid, 0.09), rtol=0, atol=1e-12)
    m0, l0, a0 = attention.split_partials(q, k, v, np.zeros(513, bool), 0.09, keys_per_split)
    assert not attention.merge_partials(m0, l0, a0).any()


def _pool(rng, slots, heads, dim):
    x = nvfp4.f32_to_bf16_f32(rng.standard_normal((slots, heads, dim)).astype(np.float32))
    pay, sc, g = nvfp4.nvfp4_encode(x)
    return pay, sc, g


def test_gather_equals_dequantize_then_gather():
    """The reference test's property (tests/qsa_fp4_check.py:52-66): the gather from the packed pool equals the
    pool dequantized to BF16 and then gathered; zero-fill writes zeros for invalid columns."""
    rng = np.random.default_rng(5)
    heads, dim, slots = 2, 64, 500
    kp, ks, gk = _pool(rng, slots, heads, dim)
    vp, vs, gv = _pool(rng, slots, heads, dim)
    raw = (kp, vp, ks, vs, gk, gv)
    kref = nvfp4.bf16_bits(nvfp4.dequant(kp, ks, gk))
    batch, topk, width = 3, 40, 300
    r2t = rng.integers(0, slots, (4, width)).astype(np.int32)
    req = np.array([2, 0, 3])
    seq = np.array([250, 30, 290], np.int32)
    idx = np.full((batch, topk), -1, np.int32)
    counts = [40, 17, 33]
    for b, n in enumerate(counts):
        idx[b, :n] = rng.permutation(int(seq[b]))[:n]
    idx[1, 5] = 299   # beyond the request's length: invalid
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    canary = np.uint16(0x7FC1)
    out_k = np.full((cu[-1], heads, dim), canary, np.uint16)
    out_v = out_k.copy()
    attention.gather_qsa(raw, r2t, req, idx, seq, cu, out_k, out_v, batch, topk)
    for b in range(batch):
        for c in range(counts[b]):
            pos = idx[b, c]
            if 0 <= pos < seq[b]:
                assert np.array_equal(out_k[cu[b] + c], kref[r2t[req[b], pos]])
            else:
                assert np.all(out_k[cu[b] + c] == canary)
    zf = 48
    cu2 = (np.arange(batch + 1) * zf).astype(np.int32)
    zk = np.full((batch * zf, heads, dim), canary, np.uint16)
    zv = zk.copy()
    attention.gather_qsa(raw, r2t, req, idx, seq, cu2, zk, zv, batch, topk, zero_fill_cols=zf)
    assert not np.any(zk == canary)
    assert np.all(zk[1 * zf + 5] == 0) and np.all(zk[0 * zf + 45] == 0)


def test_decode_page_table_equals_token_table():
    rng = np.random.default_rng(9)
    heads, dim, page, ctx, batch = 2, 128, 64, 512, 3
    slots = batch * ctx
    kp, ks, gk = _pool(rng, slots, heads, dim)
    vp, vs, gv = _pool(rng, slots, heads, dim)
    pool = (kp, vp, ks, vs, gk, gv)
    pt = rng.permutation(slots // page).reshape(batch, ctx // page).astype(np.int32)
    tt = (pt[:, :, None] * page + np.arange(page)[None, None]).reshape(batch, ctx)
    idx = np.stack([np.sort(rng.permutation(ctx)[:100]) for _ in range(batch)]).astype(np.int32)
    q = rng.standard_normal((batch, 8, dim)).astype(np.float32)
    seq = np.full(batch, ctx)
    rows = np.arange(batch)
    a = attention.sparse_decode(q, pool, pt, page, rows, idx, None, seq, 0.088)
    b = attention.sparse_decode(q, pool, tt, 1, rows, idx, None, seq, 0.088)
    assert np.array_equal(a, b)


def _mla_torch(q, keys, vals, idx, length, sink, scale):
    """tests/ds_sparse_mla_check.py:44-67 form in torch float64 (masked_fill, sink in the denominator)."""
    qd = torch.from_numpy(q)
    kd = torch.from_numpy(keys)
    vd = torch.from_numpy(vals)
    ix = torch.from_numpy(idx).long()
    pos = torch.arange(ix.shape[1])
    valid = (ix >= 0) & (pos[None] < torch.from_numpy(length)[:, None])
    k = kd[ix.clamp_min(0)]
    v = vd[ix.clamp_min(0)]
    s = torch.einsum('rhd,rnd->rhn', qd, k) * scale
    s = s.masked_fill(~valid[:, None, :], float('-inf'))
    m = s.amax(-1, keepdim=True)
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    p = torch.exp(s - m)
    total = p.sum(-1, keepdim=True) + torch.exp(torch.from_numpy(sink)[None, :, None] - m)
    o = torch.einsum('rhn,rnd->rhd', p, v) / total
    return torch.where(valid.any(1)[:, None, None], o, torch.zeros_like(o)).numpy()


def test_sparse_mla_matches_torch_with_sink():
    rng = np.random.default_rng(11)
    tokens, heads, dl, dr = 300, 16, 128, 32
    lat = nvfp4.f32_to_bf16_f32(rng.standard_normal((tokens, dl)).astype(np.float32))
    pay, sc, g = nvfp4.nvfp4_encode(lat)
    rope = nvfp4.f32_to_bf16_f32(rng.standard_normal((tokens, dr)).astype(np.float32))
    deq = nvfp4.dequant(pay, sc, g).astype(np.float64)
    keys = np.concatenate([deq, rope.astype(np.float64)], -1)
    rows, topk = 5, 64
    idx = rng.integers(0, tokens, (rows, topk)).astype(np.int32)
    idx[rng.random(idx.shape) < 0.1] = -1
    length = np.array([64, 10, 0, 1, 50], np.int32)
    sink = rng.standard_normal(heads)
    q = rng.standard_normal((rows, heads, dl + dr)) * 0.5
    out, lse = attention.sparse_mla(q, pay, sc, rope, g, idx, length, sink, 0.07)
    want = _mla_torch(q, keys, deq, idx, length, sink, 0.07)
    assert np.allclose(out, want, rtol=0, atol=1e-12)
    assert np.all(np.isneginf(lse[2])) and not out[2].any()


def test_sparse_mla_two_lists_equal_one_concatenated_cache():
    """The second key list in its own cache (sparse_mla.py:109-118) gives what one list over the two caches stacked
    gives (same keys, same order); a row whose lists are both empty writes zeros."""
    rng = np.random.default_rng(12)
    dl, dr, heads = 64, 16, 8
    caches = []
    for tokens in (200, 90):
        lat = nvfp4.f32_to_bf16_f32(rng.standard_normal((tokens, dl)).astype(np.float32))
        pay, sc, g = nvfp4.nvfp4_encode(lat)
        rope = nvfp4.f32_to_bf16_f32(rng.standard_normal((tokens, dr)).astype(np.float32))
        caches.append((pay, sc, rope, g))
    (p1, s1, r1, g1), (p2, s2, r2, g2) = caches
    rows = 4
    i1 = rng.integers(0, 200, (rows, 30)).astype(np.int32)
    i2 = rng.integers(0, 90, (rows, 12)).astype(np.int32)
    l1 = np.array([30, 5, 0, 30], np.int32)
    l2 = np.array([12, 0, 0, 3], np.int32)
    q = rng.standard_normal((rows, heads, dl + dr)) * 0.5
    sink = rng.standard_normal(heads)
    out, lse = attention.sparse_mla(q, p1, s1, r1, g1, i1, l1, sink, 0.1, extra=(p2, s2, r2, g2, i2, l2))
    # one cache: the second cache's rows re-encoded under the first cache's scale are not the same bytes, so stack
    # the dequantized keys instead and compare against a direct softmax
    d1 = nvfp4.dequant(p1, s1, g1).astype(np.float64)
    d2 = nvfp4.dequant(p2, s2, g2).astype(np.float64)
    for r in range(rows):
        k1 = np.concatenate([d1[i1[r, :l1[r]]], r1[i1[r, :l1[r]]]], -1)
        k2 = np.concatenate([d2[i2[r, :l2[r]]], r2[i2[r, :l2[r]]]], -1)
        keys = np.concatenate([k1, k2], 0)
        if keys.shape[0] == 0:
            assert not out[r].any() and np.isneginf(lse[r]).all()
            continue
        s = keys @ q[r].T * 0.1
        m = s.max(0)
        p = np.exp(s - m)
        want = (p.T @ keys[:, :dl]) / (p.sum(0) + np.exp(sink - m))[:, None]
        assert np.allclose(out[r], want, rtol=1e-12, atol=1e-12)
        assert np.allclose(lse[r], m + np.log(p.sum(0)), rtol=1e-12, atol=1e-12)


def _block_case(seed, b=3, kh=2, group=4, d=32, ctx=640, block=64, topk=5):
    rng = np.random.default_rng(seed)
    pages = b * (ctx // block)
    k_pay = rng.integers(0, 256, (pages, kh, block, d // 2), dtype=np.uint8)
    v_pay = rng.integers(0, 256, (pages, kh, block, d // 2), dtype=np.uint8)
    k_sf = rng.integers(0x20, 0x48, (pages, kh, block, d // 16), dtype=np.uint8)   # E4M3 2^-8 .. 2
    v_sf = rng.integers(0x20, 0x48, (pages, kh, block, d // 16), dtype=np.uint8)
    perm = rng.permutation(pages).reshape(b, ctx // block)
    r2t = (perm[:, :, None] * block + np.arange(block)[None, None, :]).reshape(b, ctx).astype(np.int32)
    ids = np.stack([np.stack([np.sort(rng.permutation(ctx // block)[:topk]) for _ in range(b)]) for _ in range(kh)])
    ids = ids.astype(np.int32)
    ids[1, 0, 3:] = -1                         # a shorter list (padded at the end)
    seq = np.array([ctx, ctx - 37, 5 * block + 1][:b], dtype=np.int32)
    q = rng.standard_normal((b, kh * group, d))
    return q, (k_pay, k_sf, v_pay, v_sf), r2t, np.array([2, 0, 1][:b]), ids, seq


def test_block_decode_equals_token_decode_on_the_expanded_lists():
    """kv_fp4.py's block-granular decode equals the token-granular oracle (pinned above against torch) once the
    head-major pages are laid out token-major (slot = page * block + row) and every block id is expanded to its
    positions; LSE equals the log-sum-exp of the expanded keys' scores."""
    block, scale, kv_scale = 64, 0.2, 0.75
    q, (k_pay, k_sf, v_pay, v_sf), r2t, sid, ids, seq = _block_case(3, block=block)
    out, lse = attention.block_sparse_decode(q, k_pay, k_sf, v_pay, v_sf, r2t, sid, ids, seq, block, scale, kv_scale)
    kh = k_pay.shape[1]
    group = q.shape[1] // kh
    tok = lambda a: a.transpose(0, 2, 1, 3).reshape(-1, kh, a.shape[-1])
    for h in range(kh):
        pool = (tok(k_pay)[:, h:h + 1], tok(v_pay)[:, h:h + 1], tok(k_sf)[:, h:h + 1], tok(v_sf)[:, h:h + 1],
                kv_scale, kv_scale)
        pos = (ids[h].astype(np.int64)[:, :, None] * block + np.arange(block)).reshape(len(sid), -1)
        pos = np.where(np.repeat(ids[h] >= 0, block, axis=1), pos, -1)
        ref = attention.sparse_decode(q[:, h * group:(h + 1) * group], pool, r2t, 1, sid, pos, None, seq, scale)
        np.testing.assert_allclose(out[:, h * group:(h + 1) * group], ref, rtol=1e-12, atol=1e-12)
    # a (row, head) without keys: out 0, LSE -inf
    ids2 = ids.copy()
    ids2[0, 1] = -1
    out2, lse2 = attention.block_sparse_decode(q, k_pay, k_sf, v_pay, v_sf, r2t, sid, ids2, seq, block, scale)
    assert np.all(out2[1, :group] == 0) and np.all(np.isneginf(lse2[1, :group]))
    assert np.isfinite(lse).all()


def test_block_decode_clamps_length_to_the_table_and_skips_blocks_past_it():
    block = 64
    q, pool, r2t, sid, ids, seq = _block_case(4, block=block)
    seq_big = seq.copy()
    seq_big[0] = 10 ** 6                       # clamped to req_to_token.shape[1] (kv_fp4.py:69)
    a, _ = attention.block_sparse_decode(q, *pool, r2t, sid, ids, seq_big, block, 0.1)
    b, _ = attention.block_sparse_decode(q, *pool, r2t, sid, ids, np.where(np.arange(3) == 0, r2t.shape[1], seq),
                                         block, 0.1)
    np.testing.assert_array_equal(a, b)


def _prefill_case(seed, kh=2, group=4, d=32, block=64, pages=12, q_lens=(70, 1, 33), prefix=(90, 300, 0),
                  bq=16, topk=4):
    """Head-major pages, a token-granular req_to_token whose positions sit on arbitrary slots (no block alignment),
    and per-(KV head, query block) lists of distinct block ids padded with -1."""
    rng = np.random.default_rng(seed)
    k_pay = rng.integers(0, 256, (pages, kh, block, d // 2), dtype=np.uint8)
    v_pay = rng.integers(0, 256, (pages, kh, block, d // 2), dtype=np.uint8)
    k_sf = rng.integers(0x20, 0x48, (pages, kh, block, d // 16), dtype=np.uint8)
    v_sf = rng.integers(0x20, 0x48, (pages, kh, block, d // 16), dtype=np.uint8)
    b = len(q_lens)
    seq = np.array([p + n for p, n in zip(prefix, q_lens)], dtype=np.int32)
    ctx = int(seq.max())
    r2t = np.stack([rng.permutation(pages * block)[:ctx] for _ in range(b)]).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(q_lens)])
    nqb = [-(-n // bq) for n in q_lens]
    cu_blk = np.concatenate([[0], np.cumsum(nqb)])
    ids = np.full((kh, cu_blk[-1], topk), -1, dtype=np.int32)
    for h in range(kh):
        for bb in range(b):
            nb = -(-int(seq[bb]) // block)
            for j in range(nqb[bb]):
                n = min(topk, nb) - (j + h) % 2
                ids[h, cu_blk[bb] + j, :n] = rng.permutation(nb)[:n]
    q = rng.standard_normal((cu[-1], kh * group, d))
    return q, (k_pay, k_sf, v_pay, v_sf), r2t, np.roll(np.arange(b), 1), ids, cu, cu_blk, seq, np.array(prefix[:b])


def test_block_prefill_equals_token_decode_on_the_expanded_lists():
    """kv_fp4.py's causal block-sparse prefill equals the token-granular oracle (pinned against torch) given, per query,
    its block list expanded to positions with the query's position as the causal limit; slots come from per-token
    lookups, so tokens need not sit on their block's page."""
    block, scale, kv_scale, bq = 64, 0.3, 0.5, 16
    q, (k_pay, k_sf, v_pay, v_sf), r2t, sid, ids, cu, cu_blk, seq, prefix = _prefill_case(5, bq=bq)
    out = attention.block_sparse_prefill(q, k_pay, k_sf, v_pay, v_sf, r2t, sid, ids, cu, cu_blk, seq, prefix, bq, block,
                                         scale, kv_scale)
    kh = k_pay.shape[1]
    group = q.shape[1] // kh
    tok = lambda a: a.transpose(0, 2, 1, 3).reshape(-1, kh, a.shape[-1])
    rows = np.repeat(sid, np.diff(cu))
    local = np.arange(cu[-1]) - np.repeat(cu[:-1], np.diff(cu))
    qpos = np.repeat(prefix, np.diff(cu)) + local
    blk = np.repeat(cu_blk[:-1], np.diff(cu)) + local // bq
    for h in range(kh):
        pool = (tok(k_pay)[:, h:h + 1], tok(v_pay)[:, h:h + 1], tok(k_sf)[:, h:h + 1], tok(v_sf)[:, h:h + 1],
                kv_scale, kv_scale)
        lists = ids[h][blk].astype(np.int64)
        pos = np.where(np.repeat(lists >= 0, block, axis=1),
                       (lists[:, :, None] * block + np.arange(block)).reshape(len(blk), -1), -1)
        ref = attention.sparse_decode(q[:, h * group:(h + 1) * group], pool, r2t, 1, rows, pos, None,
                                      np.repeat(seq, np.diff(cu)), scale, query_pos=qpos)
        np.testing.assert_allclose(out[:, h * group:(h + 1) * group], ref, rtol=1e-12, atol=1e-12)
    # a query whose only block lies in its future has no key: 0
    ids2 = ids.copy()
    ids2[:, 0] = -1
    ids2[:, 0, 0] = 5                           # block 5 (positions 320..383) > every position of query block 0
    out2 = attention.block_sparse_prefill(q, k_pay, k_sf, v_pay, v_sf, r2t, sid, ids2, cu, cu_blk, seq, prefix, bq,
                                          block, scale)
    assert np.all(out2[:bq] == 0)


def test_block_prefill_with_every_block_is_dense_causal_attention():
    """With every block of the context listed, each query attends to exactly positions 0 .. its own: dense causal
    attention over the dequantized context (the BF16 copy path of kv_fp4.py:601-629 gives the same)."""
    block, scale, bq = 64, 0.25, 1
    q, pool, r2t, sid, _, cu, _, seq, prefix = _prefill_case(8, q_lens=(40, 3), prefix=(100, 200), bq=bq)
    k_pay, k_sf, v_pay, v_sf = pool
    kh = k_pay.shape[1]
    nb = -(-int(seq.max()) // block)
    cu_blk = cu.copy()
    ids = np.tile(np.arange(nb, dtype=np.int32)[::-1], (kh, cu[-1], 1))          # every block, in reverse order
    out = attention.block_sparse_prefill(q, *pool, r2t, sid, ids, cu, cu_blk, seq, prefix, bq, block, scale)
    rows = 256
    kd = attention.dequantize_context(k_pay, k_sf, r2t, sid, seq, rows)
    vd = attention.dequantize_context(v_pay, v_sf, r2t, sid, seq, rows)
    group = q.shape[1] // kh
    for b in range(len(sid)):
        for i in range(cu[b + 1] - cu[b]):
            n = int(prefix[b]) + i + 1
            k, v = kd[b * rows:b * rows + n], vd[b * rows:b * rows + n]
            for h in range(kh):
                qs = q[cu[b] + i, h * group:(h + 1) * group]
                s = qs @ k[:, h].astype(np.float64).T * scale
                p = np.exp(s - s.max(1, keepdims=True))
                want = (p / p.sum(1, keepdims=True)) @ v[:, h].astype(np.float64)
                np.testing.assert_allclose(out[cu[b] + i, h * group:(h + 1) * group], want, rtol=1e-10, atol=1e-12)


def test_dequantize_context_copies_each_position_from_its_slot():
    """kv_fp4.py:496-530: row b * rows_per_req + pos holds the token at slot req_to_token[sid, pos] (page s // block,
    row s % block), decoded by the NVFP4 dequantizer; rows at or past seq_lens[b] stay unwritten; the index cache
    (no head dimension) alike; slot ids past the table wrap modulo the pool size."""
    _, (k_pay, k_sf, _, _), r2t, sid, _, _, _, seq, _ = _prefill_case(11)
    pages, kh, block, half = k_pay.shape
    rows = 448
    out = attention.dequantize_context(k_pay, k_sf, r2t, sid, seq, rows)
    assert out.shape == (len(sid) * rows, kh, 2 * half)
    for b in range(len(sid)):
        for pos in (0, int(seq[b]) - 1):
            s = int(r2t[sid[b], pos])
            np.testing.assert_array_equal(out[b * rows + pos],
                                          nvfp4.dequant(k_pay[s // block, :, s % block], k_sf[s // block, :, s % block]))
        assert np.isnan(out[b * rows + int(seq[b]):(b + 1) * rows]).all()
        assert not np.isnan(out[b * rows:b * rows + int(seq[b])]).any()
    one = attention.dequantize_context(k_pay[:, 1], k_sf[:, 1], r2t, sid + pages * block, seq, rows)
    np.testing.assert_array_equal(one[:, 0], out[:, 1])


def test_varlen_split_form_equals_one_pass_softmax():
    """qsa_decode.py's split/merge form (128-key splits) equals the one-pass softmax per row; an empty row is 0."""
    rng = np.random.default_rng(9)
    counts = [300, 0, 1, 129, 128]
    cu_k = np.concatenate([[0], np.cumsum(counts)])
    k = rng.standard_normal((cu_k[-1], 2, 16))
    v = rng.standard_normal((cu_k[-1], 2, 16))
    q = rng.standard_normal((7, 8, 16))
    cu_q = np.array([0, 2, 3, 4, 6, 7])
    got = attention.varlen_decode(q, k, v, cu_q, cu_k, 0.3)
    for r, n in enumerate(counts):
        a = cu_k[r]
        want = attention.softmax_attention(q[cu_q[r]], k[a:a + n], v[a:a + n], np.ones(n, bool), 0.3)
        np.testing.assert_allclose(got[r], want, rtol=1e-12, atol=1e-12)
    assert np.all(got[1] == 0)


def test_v4_keys_decode_the_packed_pages():
    """The oracle's V4 page decoding (sparse_mla.py:38-59) equals the exact keys the packing rule produced, through
    torch's float8_e4m3fn values: pages of 64 and 128 tokens, padded page strides."""
    from tests._v4 import pack_v4
    g = torch.Generator().manual_seed(3)
    lat = torch.randn(256, 512, generator=g) * torch.rand(256, 1, generator=g) * 4
    for ps in (64, 128):
        view, keys, stride = pack_v4(lat, ps)
        got = attention.v4_keys(view.as_strided((view.shape[0] * stride,), (1,)).numpy(), ps, stride)
        np.testing.assert_array_equal(got, keys)


def test_sparse_mla_v4_matches_torch_with_sink_and_two_lists():
    """Sparse MLA on V4 keys (value = key): torch float64 softmax with the sink in the denominator; two lists equal
    one list over the concatenated keys; a row without keys is 0 with LSE -inf."""
    rng = np.random.default_rng(4)
    k1, k2 = rng.standard_normal((50, 512)), rng.standard_normal((30, 512))
    q = rng.standard_normal((3, 4, 512)) * 0.1
    i1 = rng.integers(-1, 50, (3, 20)).astype(np.int32)
    i2 = rng.integers(-1, 30, (3, 10)).astype(np.int32)
    l1 = np.array([20, 5, 0], np.int32)
    l2 = np.array([10, 10, 0], np.int32)
    sink = rng.standard_normal(4)
    out, lse = attention.sparse_mla_v4(q, k1, i1, l1, sink, 0.05, k2, i2, l2)
    cat = np.concatenate([k1, k2])
    ic = np.concatenate([np.where((i1 >= 0) & (np.arange(20) < l1[:, None]), i1, -1),
                         np.where((i2 >= 0) & (np.arange(10) < l2[:, None]), i2 + 50, -1)], 1)
    out2, lse2 = attention.sparse_mla_v4(q, cat, ic, None, sink, 0.05)
    np.testing.assert_allclose(out, out2, rtol=1e-12, atol=1e-14)
    for r in range(2):
        sel = ic[r][ic[r] >= 0]
        kd = torch.from_numpy(cat[sel])
        s = torch.from_numpy(q[r]) @ kd.T * 0.05
        m = s.max(1, keepdim=True).values
        p = torch.exp(s - m)
        o = (p @ kd) / (p.sum(1, keepdim=True) + torch.exp(torch.from_numpy(sink)[:, None] - m))
        np.testing.assert_allclose(out[r], o.numpy(), rtol=1e-10, atol=1e-12)
    assert np.all(out[2] == 0) and np.all(np.isneginf(lse[2]))
