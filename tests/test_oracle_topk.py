"""Pins of the top-k producers' oracle (oracle/topk.py) on the CPU: each function against an implementation that does
not share its code (torch loops, a flat-key path for the paged one, brute force for the selection) and against
hand-worked cases in which a plausible mistake (ReLU after the head sum, the scale left out, the weight on the wrong
head, masks off by one, ties to the higher position) changes the answer."""
import math

import numpy as np
import torch

from oracle import nvfp4, topk


def test_topk_rows_brute_force_with_ties_masks_and_short_rows():
    rng = np.random.default_rng(3)
    x = rng.integers(-4, 5, (6, 40)).astype(np.float32)   # many ties
    x[1, :30] = -np.inf                                     # 10 finite values for topk 16
    x[2, :] = -np.inf                                       # none
    x[3, 5] = np.nan
    x[4, 7] = np.inf                                        # +inf is not finite either
    got = topk.topk_rows(x, 16)
    for r in range(6):
        cand = [(-float(x[r, c]), c) for c in range(40) if np.isfinite(x[r, c])]
        want = sorted(c for _, c in sorted(cand)[:16])
        assert list(got[r, :len(want)]) == want and (got[r, len(want):] == -1).all(), r


def test_topk_rows_ties_go_to_the_lower_position():
    x = np.array([[1, 3, 3, 3, 0]], np.float32)
    assert topk.topk_rows(x, 2).tolist() == [[1, 2]]
    assert topk.topk_rows(x, 4).tolist() == [[0, 1, 2, 3]]


def test_qsa_logits_against_torch_head_loop():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(7, 4, 32, generator=g).double()
    k = torch.randn(50, 32, generator=g).double()
    starts = np.array([0, 3, 10, 0, 49, 20, 0])
    ends = np.array([50, 4, 30, 0, 50, 10, 25])
    want = torch.zeros(7, 50, dtype=torch.float64)
    for h in range(4):
        want += torch.relu(q[:, h] @ k.T)
    want /= math.sqrt(32)
    pos = torch.arange(50)[None, :]
    want = want.masked_fill(~((pos >= torch.tensor(starts)[:, None]) & (pos < torch.tensor(ends)[:, None])), -math.inf)
    got = topk.qsa_indexer_logits(q.numpy(), k.numpy(), starts, ends)
    assert np.array_equal(np.isinf(got), torch.isinf(want).numpy())
    fin = np.isfinite(got)
    assert np.allclose(got[fin], want.numpy()[fin], rtol=1e-12, atol=0)


def test_qsa_logits_hand_worked():
    # two heads: q . k = +3 and -2 -> ReLU per head then sum = 3 (a sum before ReLU would give 1); scale 2 -> 1.5
    q = np.array([[[1.0, 1.0], [-1.0, -1.0]]])
    k = np.array([[1.0, 2.0], [0.0, 0.0]])
    got = topk.qsa_indexer_logits(q, k, np.array([0]), np.array([1]), score_scale=2.0)
    assert got[0, 0] == 1.5 and got[0, 1] == -np.inf


def test_dsa_logits_against_the_reference_formula_and_a_loop():
    g = torch.Generator().manual_seed(6)
    q = (torch.randn(9, 32, 16, generator=g) * 2).to(torch.float8_e4m3fn).float().double()
    k = (torch.randn(40, 16, generator=g) * 2).to(torch.float8_e4m3fn).float().double()
    k_scale = torch.rand(40, generator=g).double() + 0.5
    w = torch.randn(9, 32, generator=g).double()
    ks = np.array([0, 5, 0, 39, 10, 0, 0, 3, 20])
    ke = np.array([40, 6, 0, 40, 30, 1, 40, 4, 21])
    ref = (torch.einsum('qhd,kd->qhk', q, k).relu() * w[:, :, None]).sum(1) * k_scale[None, :]
    pos = torch.arange(40)
    keep = (pos[None, :] >= torch.tensor(ks)[:, None]) & (pos[None, :] < torch.tensor(ke)[:, None])
    for clean, fill in ((False, 0.0), (True, -math.inf)):
        got = topk.dsa_mqa_logits(q.numpy(), k.numpy(), k_scale.numpy(), w.numpy(), ks, ke, clean)
        want = ref.masked_fill(~keep, fill).numpy()
        assert np.array_equal(np.isinf(got), np.isinf(want))
        fin = np.isfinite(want)
        assert np.allclose(got[fin], want[fin], rtol=1e-12, atol=1e-12)
    # a loop over one element, weights on their own heads
    qq, kk = q.numpy(), k.numpy()
    s = sum(w[4, h].item() * max(0.0, float(qq[4, h] @ kk[12])) for h in range(32)) * k_scale[12].item()
    assert math.isclose(topk.dsa_mqa_logits(qq, kk, k_scale.numpy(), w.numpy(), ks, ke)[4, 12], s, rel_tol=1e-12)


def test_dsa_paged_logits_equal_the_flat_logits_of_the_gathered_keys():
    rng = np.random.default_rng(7)
    pages, block, d = 12, 8, 16
    vals = rng.integers(0, 256, (pages, block, d)).astype(np.uint8)
    vals[(vals & 0x7F) == 0x7F] = 0x38                       # no NaN bytes
    scl = (rng.random((pages, block)) + 0.5).astype(np.float32)
    cache = np.concatenate([vals.reshape(pages, -1), scl.view(np.uint8).reshape(pages, -1)], 1)
    table = np.array([[3, 7, 1], [0, 11, 5]], np.int32)
    lens = np.array([20, 9])
    q = nvfp4.e4m3_decode(rng.integers(0, 120, (2, 32, d)).astype(np.uint8)).astype(np.float64)
    w = rng.standard_normal((2, 32))
    got = topk.dsa_paged_mqa_logits(q, cache, w, lens, table, 30, clean_logits=True)
    for b in range(2):
        keys = nvfp4.e4m3_decode(vals[table[b]].reshape(-1, d)).astype(np.float64)
        flat = topk.dsa_mqa_logits(q[b:b + 1], keys, scl[table[b]].reshape(-1), w[b:b + 1], np.array([0]),
                                   np.array([lens[b]]), clean_logits=True)[0]
        want = np.full(30, -np.inf)
        want[:24] = flat
        assert np.array_equal(got[b], want), b


# ----------------------------------------------------------------------------------------------------------------
# MiniMax NVFP4 block scores (kv_fp4.py:168-222 decode, :407-446 prefill)

_E2M1 = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6], dtype=torch.float64)


def _mm_pool(pages, d, rng):
    pay = rng.integers(0, 256, (pages, 128, d // 2)).astype(np.uint8)
    sf = rng.integers(0x20, 0x50, (pages, 128, d // 16)).astype(np.uint8)     # E4M3 2^-3 .. 2^2.9, no NaN
    return pay, sf


def _lut_keys(pay, sf):
    """Every slot's key [pages * 128, d] through the 16-entry table, low nibble first, scale j // 16."""
    p = torch.from_numpy(pay.reshape(-1, pay.shape[-1]).astype(np.int64))
    vals = torch.stack([_E2M1[p & 15], _E2M1[p >> 4]], -1).reshape(p.shape[0], -1)
    s = torch.from_numpy(sf.reshape(-1, sf.shape[-1]).copy()).view(torch.float8_e4m3fn).double()
    return vals * s.repeat_interleave(16, -1)


def test_minimax_decode_scores_against_a_brute_force():
    rng = np.random.default_rng(11)
    d, bs, pages = 64, 32, 12
    pay, sf = _mm_pool(pages, d, rng)
    keys = _lut_keys(pay, sf)
    r2t = rng.permutation(pages * 128).astype(np.int32).reshape(4, -1)[:, :300]
    wrapped = r2t.copy()
    wrapped[1, 5] -= pages * 128                               # a negative slot reads the same key
    seq = np.array([300, 40, 129, 33])
    slot_ids = np.array([2, 1, 0, 3])
    q = rng.standard_normal((4, 3, d))
    for score_type in ('max', 'lse'):
        got = topk.minimax_block_scores_decode(q, pay, sf, r2t, slot_ids, seq, bs, 0.125, 1.5, init_blocks=3,
                                               local_blocks=2, score_type=score_type)
        again = topk.minimax_block_scores_decode(q, pay, sf, wrapped, slot_ids, seq, bs, 0.125, 1.5, init_blocks=3,
                                                 local_blocks=2, score_type=score_type)
        assert np.array_equal(got, again, equal_nan=True)
        c = float(np.float32(np.float32(0.125) * np.float32(1.4426950409)) * np.float32(1.5))
        for b in range(4):
            n, nb = int(seq[b]), -(-int(seq[b]) // bs)
            k = keys[torch.from_numpy(r2t[slot_ids[b], :n].astype(np.int64))]
            sc = torch.from_numpy(q[b]) @ k.T * c                # [heads, n]
            for blk in range(nb):
                seg = sc[:, blk * bs:(blk + 1) * bs]
                if blk >= nb - 2:
                    want = torch.full((3,), 1e29, dtype=torch.float64)
                elif blk < 3:
                    want = torch.full((3,), 1e30, dtype=torch.float64)
                elif score_type == 'max':
                    want = seg.max(1).values
                else:
                    want = torch.logsumexp(seg * math.log(2), 1) / math.log(2)
                assert np.allclose(got[:, b, blk], want.numpy(), rtol=1e-12, atol=0), (b, blk)
            assert np.isnan(got[:, b, nb:]).all()


def test_minimax_decode_skip_trivial_and_forced_precedence():
    rng = np.random.default_rng(12)
    pay, sf = _mm_pool(2, 32, rng)
    r2t = np.arange(256, dtype=np.int32).reshape(1, 256)
    q = rng.standard_normal((1, 2, 32))
    # 4 blocks of 32: local_blocks 2 -> blocks 2, 3 at 1e29 even though init_blocks 3 covers block 2
    got = topk.minimax_block_scores_decode(q, pay, sf, r2t, [0], [128], 32, 1.0, 1.0, 3, 2)
    assert got[0, 0].tolist()[:2] == [1e30, 1e30] and got[0, 0].tolist()[2:] == [1e29, 1e29]
    # 4 blocks <= topk 4: no scores at all; topk 3: scores
    assert np.isnan(topk.minimax_block_scores_decode(q, pay, sf, r2t, [0], [128], 32, 1.0, 1.0, 0, 0, topk=4)).all()
    assert np.isfinite(topk.minimax_block_scores_decode(q, pay, sf, r2t, [0], [128], 32, 1.0, 1.0, 0, 0,
                                                        topk=3)).all()


def test_minimax_prefill_scores_against_a_brute_force():
    rng = np.random.default_rng(13)
    d, bs, pages = 32, 32, 10
    pay, sf = _mm_pool(pages, d, rng)
    keys = _lut_keys(pay, sf)
    r2t = rng.permutation(pages * 128).astype(np.int32).reshape(2, -1)[:, :600]
    prefix, ext = [0, 150], [140, 70]
    seq = [p + e for p, e in zip(prefix, ext)]
    cu = np.array([0, 140, 210])
    q = rng.standard_normal((210, 2, d))
    got = topk.minimax_block_scores_prefill(q, pay, sf, r2t, [1, 0], cu, seq, prefix, bs, 0.5, 1.0)
    c = float(np.float32(np.float32(0.5) * np.float32(1.4426950409)))
    for b, sid in enumerate((1, 0)):
        k = keys[torch.from_numpy(r2t[sid, :seq[b]].astype(np.int64))]
        for t in range(ext[b]):
            row = cu[b] + t
            hi = min(seq[b], prefix[b] + (t // 64 + 1) * 64)    # the row's 64-row tile bounds the blocks written
            nblk = -(-hi // bs)
            sc = (torch.from_numpy(q[row]) @ k.T * c).numpy()     # [heads, n]
            for blk in range(nblk):
                cols = [p for p in range(blk * bs, min(hi, (blk + 1) * bs)) if p <= prefix[b] + t]
                want = sc[:, cols].max(1) if cols else np.full(2, -np.inf)
                assert np.allclose(got[:, row, blk], want, rtol=1e-12, atol=0), (b, t, blk)
            assert np.isnan(got[:, row, nblk:]).all()
    # rows 63 and 64 of the first request: 2 and 4 blocks written, row 64's last block all -inf
    assert np.isfinite(got[0, 63, :2]).all() and np.isnan(got[0, 63, 2:]).all()
    assert np.isfinite(got[0, 64, :3]).all() and got[0, 64, 3] == -np.inf
