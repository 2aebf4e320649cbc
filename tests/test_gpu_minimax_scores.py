"""MiniMax index block scores on the GPU (xt_minimax_decode_scores / xt_minimax_prefill_scores) against the oracle
(oracle/topk.py, kv_fp4.py:168-222 and :407-446): the scores within the FP32 summation bound of exact products, the
forced, skipped and unwritten entries exactly, and the top-k block sets equal, as the reference's own check compares
them (tests/minimax_kv_fp4_check.py:103-108, :146). The shapes are that check's: index q [b, 4, 128], one index key
head, 128-token pages (:29), the decode and prefill cases of :180-182."""
import numpy as np
import pytest
import torch

from oracle import nvfp4
from oracle import topk as ref
from xtier_amd import minimax, ops

pytestmark = pytest.mark.gpu
PAGE = 128


def _pool(pages, dim, g):
    pay = torch.randint(0, 256, (pages, PAGE, dim // 2), generator=g, dtype=torch.uint8)
    sc = torch.randint(0x18, 0x58, (pages, PAGE, dim // 16), generator=g, dtype=torch.uint8)
    sc[:, ::7, 0] = torch.randint(1, 8, (pages, (PAGE + 6) // 7), generator=g, dtype=torch.uint8)   # subnormal scales
    return pay, sc


def _mapping(seq_lens, g, width=16384):
    """req_to_token with each request's pages in random physical order (tests/minimax_kv_fp4_check.py:51-63)."""
    blocks = [-(-s // PAGE) for s in seq_lens]
    pages = sum(blocks) + 1
    perm = torch.randperm(pages - 1, generator=g) + 1
    r2t = torch.zeros(len(seq_lens), width, dtype=torch.int32)
    off = 0
    for r, n in enumerate(blocks):
        for blk in range(n):
            pg = int(perm[off + blk])
            r2t[r, blk * PAGE:(blk + 1) * PAGE] = torch.arange(pg * PAGE, (pg + 1) * PAGE)
        off += n
    return r2t, pages


def _keys(pay, sc):
    return nvfp4.dequant(pay.numpy().reshape(-1, pay.shape[-1]), sc.numpy().reshape(-1, sc.shape[-1]),
                         1.0).astype(np.float64)


def _block_bound(q, keys_abs, toks, n, bs, c):
    """Per head and block: c (dim + 2) 2^-24 max over the block's keys of sum |q| |k| (the FP32 sum of exact
    products), [heads, blocks]."""
    a = np.abs(q) @ keys_abs[toks[:n]].T                           # [heads, n]
    nb = -(-n // bs)
    pad = np.zeros((a.shape[0], nb * bs))
    pad[:, :n] = a
    return c * (q.shape[-1] + 2) * 2.0 ** -24 * pad.reshape(a.shape[0], nb, bs).max(-1)


@pytest.mark.parametrize('seq_lens,dim,bs,score_type,q_dtype,s_dtype,wide', [
    ([4000, 2500, 1300], 128, 128, 'max', torch.bfloat16, torch.float32, False),
    ([8000], 128, 128, 'lse', torch.bfloat16, torch.float32, True),
    ([128, 129, 300], 128, 64, 'max', torch.float16, torch.float32, False),
    ([700, 33], 64, 32, 'lse', torch.bfloat16, torch.float32, True),
    ([1000, 257], 256, 256, 'max', torch.bfloat16, torch.bfloat16, False),
])
def test_decode_scores(seq_lens, dim, bs, score_type, q_dtype, s_dtype, wide):
    g = torch.Generator().manual_seed(sum(seq_lens) + dim + bs)
    r2t, pages = _mapping(seq_lens, g)
    pay, sc = _pool(pages, dim, g)
    b, heads = len(seq_lens), 4
    q = (torch.randn(b, heads, dim, generator=g) * 0.5).to(q_dtype)
    idx = torch.int64 if wide else torch.int32
    seq = torch.tensor(seq_lens, dtype=idx)
    sid = torch.arange(b, dtype=idx)
    max_blocks = -(-max(seq_lens) // bs) + 3
    init, local = 2, 1
    for skip in (None, 2):
        score = torch.full((heads, b, max_blocks), 7.0, dtype=s_dtype, device='cuda')
        ops.minimax_decode_scores(q.cuda(), pay.cuda(), sc.cuda(), r2t.cuda(), score, seq.cuda(), sid.cuda(), bs,
                                  dim ** -0.5, 1.25, init, local, score_type, skip_topk=skip)
        got = score.float().cpu().numpy().astype(np.float64)
        want = ref.minimax_block_scores_decode(q.float().numpy(), pay.numpy(), sc.numpy(), r2t.numpy(), sid.numpy(),
                                               seq_lens, bs, dim ** -0.5, 1.25, init, local, score_type,
                                               topk=skip)
        c = ops.minimax_score_factor(dim ** -0.5, 1.25)
        keys = _keys(pay, sc)
        for r, n in enumerate(seq_lens):
            nb = -(-n // bs)
            if skip is not None and nb <= skip:
                assert (got[:, r] == 7.0).all()                     # nothing written
                continue
            assert (got[:, r, nb:] == 7.0).all()
            bound = _block_bound(q[r].float().numpy(), np.abs(keys), r2t[r].long().numpy(), n, bs, c)
            w, o = want[:, r, :nb], got[:, r, :nb]
            forced = (w == 1e29) | (w == 1e30)
            assert np.array_equal(o[forced], torch.from_numpy(w[forced]).to(s_dtype).double().numpy())
            # score rounding: FP32 (2^-24) or BF16 (2^-9) relative; LSE adds the exp2 / log2 rounding
            rel = 2.0 ** -9 if s_dtype == torch.bfloat16 else 2.0 ** -23
            tol = bound + rel * np.abs(w) + (4e-6 * (1 + np.abs(w)) if score_type == 'lse' else 0)
            assert (np.abs(o - w)[~forced] <= tol[~forced]).all(), float(np.abs(o - w)[~forced].max())


def test_decode_topk_sets_equal():
    """The check of tests/minimax_kv_fp4_check.py:103-108: top-16 block sets per head and request, init 0, local 1."""
    g = torch.Generator().manual_seed(5)
    seq_lens = [4000, 2500, 1300]
    r2t, pages = _mapping(seq_lens, g)
    pay, sc = _pool(pages, 128, g)
    q = torch.randn(3, 4, 128, generator=g).to(torch.bfloat16)
    nb = -(-max(seq_lens) // PAGE)
    score = torch.full((4, 3, nb), float('-inf'), device='cuda')
    sid = torch.arange(3, dtype=torch.int32)
    ops.minimax_decode_scores(q.cuda(), pay.cuda(), sc.cuda(), r2t.cuda(), score,
                              torch.tensor(seq_lens, dtype=torch.int32).cuda(), sid.cuda(), PAGE, 128 ** -0.5, 1.0, 0,
                              1)
    want = ref.minimax_block_scores_decode(q.float().numpy(), pay.numpy(), sc.numpy(), r2t.numpy(), sid.numpy(),
                                           seq_lens, PAGE, 128 ** -0.5, 1.0, 0, 1)
    want = np.where(np.isnan(want), -np.inf, want)
    got = score.cpu().numpy()
    for h in range(4):
        for r in range(3):
            k = min(16, -(-seq_lens[r] // PAGE))
            assert set(np.argsort(-got[h, r], kind='stable')[:k]) == set(np.argsort(-want[h, r], kind='stable')[:k])


@pytest.mark.parametrize('prefix,ext,dim,bs,heads,q_dtype', [
    ([0], [1500], 128, 128, 4, torch.bfloat16),
    ([1000], [500], 128, 128, 4, torch.bfloat16),
    ([0, 300], [900, 600], 128, 128, 4, torch.bfloat16),
    ([5000], [3000], 128, 128, 4, torch.bfloat16),
    ([70, 0], [200, 65], 64, 32, 2, torch.float16),
    ([129], [300], 256, 256, 1, torch.bfloat16),
    ([0, 17], [130, 250], 128, 64, 3, torch.bfloat16),
])
def test_prefill_scores(prefix, ext, dim, bs, heads, q_dtype):
    g = torch.Generator().manual_seed(sum(prefix) + sum(ext) + dim)
    seq_lens = [p + e for p, e in zip(prefix, ext)]
    r2t, pages = _mapping(seq_lens, g)
    pay, sc = _pool(pages, dim, g)
    total = sum(ext)
    q = (torch.randn(total, heads, dim, generator=g) * 0.3).to(q_dtype)
    cu = torch.tensor([0] + list(np.cumsum(ext)), dtype=torch.int32)
    seq = torch.tensor(seq_lens, dtype=torch.int32)
    pre = torch.tensor(prefix, dtype=torch.int32)
    sid = torch.arange(len(ext), dtype=torch.int32)
    max_blocks = -(-max(seq_lens) // bs)
    score = torch.full((heads, total, max_blocks), 7.0, device='cuda')
    ops.minimax_prefill_scores(q.cuda(), pay.cuda(), sc.cuda(), r2t.cuda(), score, cu.cuda(), seq.cuda(), pre.cuda(),
                               sid.cuda(), bs, dim ** -0.5, 1.0, max(ext))
    got = score.cpu().numpy().astype(np.float64)
    want = ref.minimax_block_scores_prefill(q.float().numpy(), pay.numpy(), sc.numpy(), r2t.numpy(), sid.numpy(),
                                            cu.numpy(), seq_lens, prefix, bs, dim ** -0.5, 1.0)
    assert np.array_equal(np.isnan(want), got == 7.0)            # exactly the entries the reference writes
    assert np.array_equal(np.isneginf(want), np.isneginf(got))
    c = ops.minimax_score_factor(dim ** -0.5, 1.0)
    keys = np.abs(_keys(pay, sc))
    for r in range(len(ext)):
        toks = r2t[r].long().numpy()
        for t in range(ext[r]):
            row = int(cu[r]) + t
            fin = np.isfinite(want[:, row])
            bound = _block_bound(q[row].float().numpy(), keys, toks, seq_lens[r], bs, c)
            nb = bound.shape[1]
            f = fin[:, :nb]
            err = np.abs(got[:, row, :nb][f] - want[:, row, :nb][f])
            assert (err <= (bound + 2.0 ** -23 * np.abs(want[:, row, :nb]))[f]).all(), (r, t)


@pytest.mark.parametrize('bs', [96, 160, 192, 224])
def test_block_sizes_not_powers_of_two_are_refused(bs):
    """Block sizes must be 32, 64, 128 or 256 (the reference's tl.arange(0, block_size) takes powers of two): the
    prefill stages keys 128 at a time and masks them by causality and length only, so any other multiple of 32 would
    let the next block's keys into a block's maximum. Both score entry points refuse them before launching."""
    g = torch.Generator().manual_seed(bs)
    seq_lens = [600]
    r2t, pages = _mapping(seq_lens, g)
    pay, sc = _pool(pages, 128, g)
    q = (torch.randn(300, 2, 128, generator=g) * 0.3).to(torch.bfloat16).cuda()
    nb = -(-600 // bs)
    score = torch.full((2, 300, nb), 7.0, device='cuda')
    i32 = lambda v: torch.tensor(v, dtype=torch.int32).cuda()
    with pytest.raises(NotImplementedError, match='block size'):
        ops.minimax_prefill_scores(q, pay.cuda(), sc.cuda(), r2t.cuda(), score, i32([0, 300]), i32(seq_lens),
                                   i32([300]), i32([0]), bs, 128 ** -0.5, 1.0, 300)
    assert bool((score == 7.0).all())   # nothing written
    dscore = torch.full((2, 1, nb), 7.0, device='cuda')
    with pytest.raises(NotImplementedError, match='block size'):
        ops.minimax_decode_scores(q[:1], pay.cuda(), sc.cuda(), r2t.cuda(), dscore, i32(seq_lens), i32([0]), bs,
                                  128 ** -0.5, 1.0, 0, 0)
    assert bool((dscore == 7.0).all())


class _SglangDecodeStandIn:
    """What SGLang's flash_decode_with_topk_idx does around its score kernel, reduced to the launch (its argument list
    as the reference's shim receives it, kv_fp4.py:233-236) and a top-k over the score buffer."""

    def __init__(self):
        import sys
        import types
        self.mod = types.ModuleType('xt_sglang_decode_standin')
        self.mod._decode_score_kernel = None
        sys.modules[self.mod.__name__] = self.mod

    def run(self, q, k_cache, req_to_token, seq_lens, slot_ids, block_size, topk, init_blocks, local_blocks,
            score_type, **_):
        b, heads = q.shape[0], q.shape[1]
        nb = -(-int(seq_lens.max()) // block_size)
        score = torch.full((heads, b, nb), float('-inf'), device=q.device)
        self.mod._decode_score_kernel[(b * 2, 1)](
            q, k_cache, req_to_token, score, seq_lens, slot_ids, k_cache.shape[0], b, heads, q.shape[2], block_size,
            topk, 128 ** -0.5, 1.0, init_blocks, local_blocks, *q.stride(), *k_cache.stride(), req_to_token.stride(0),
            *score.stride(), NUM_KV_CHUNKS=2, SCORE_TYPE=score_type, SKIP_TRIVIAL_TOPK_SCORE=False)
        return score, score.topk(min(topk, nb), -1).indices


def test_decode_topk_hook_end_to_end():
    standin = _SglangDecodeStandIn()
    run = standin.run
    run.__func__.__module__ = standin.mod.__name__
    g = torch.Generator().manual_seed(9)
    seq_lens = [3000, 700]
    r2t, pages = _mapping(seq_lens, g)
    pay, sc = _pool(pages, 128, g)
    pay, sc = pay.cuda(), sc.cuda()
    setattr(pay, minimax.TAG, sc)
    q = torch.randn(2, 4, 128, generator=g).to(torch.bfloat16)
    kw = dict(req_to_token=r2t.cuda(), seq_lens=torch.tensor(seq_lens, dtype=torch.int32).cuda(),
              slot_ids=torch.arange(2, dtype=torch.int32).cuda(), block_size=PAGE, topk=8, init_blocks=0,
              local_blocks=1, score_type='max', disable_index_value=True, sink=None)
    score, _ = minimax.decode_topk(run, q=q.cuda(), k_cache=pay, **kw)
    want = ref.minimax_block_scores_decode(q.float().numpy(), pay.cpu().numpy(), sc.cpu().numpy(), r2t.numpy(),
                                           [0, 1], seq_lens, PAGE, 128 ** -0.5, 1.0, 0, 1)
    got = score.cpu().numpy()
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(want), np.isneginf(got))        # the blocks past the shorter request: unwritten
    assert np.allclose(got[fin], want[fin], rtol=1e-5, atol=1e-5)
    assert standin.mod._decode_score_kernel is None                 # restored
