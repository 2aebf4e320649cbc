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
