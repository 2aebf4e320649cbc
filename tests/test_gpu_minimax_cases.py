"""The MiniMax cases of tests/minimax_kv_fp4_check.py (check_decode :81-111, check_prefill :114-148) on this build:
MiniMax-M3.1's shape (64 query heads over 4 KV heads x 128, 128-token pages in a random physical order, one spare
page), NVFP4 pages quantized with unit global scale. The reference compares its NVFP4 kernels with SGLang's BF16
kernels on the dequantized cache by relative L2 error (decode < 2e-3, prefill < 1e-3): two kernels that round alike.
Here the comparison is the exact (FP64) oracle, where the BF16 rounding of the output alone contributes about 1.1e-3:
relative L2 below 2e-3 in both cases, and no worse than 1.25x the error of the oracle at the flash kernels' precision
(BF16 output, P rounded to BF16); plus the usual tolerance check. The dequantized context copies must be bit-equal to
the dequantized cache, as in the reference."""
import numpy as np
import pytest
import torch

from oracle import attention, nvfp4
from tests._attn import check
from xtier_amd import ops, workloads

pytestmark = pytest.mark.gpu

PAGE, D, KH, QH = 128, 128, 4, 64


def _mapping(seq_lens, gen):
    """req_to_token [b, 16384]: each request's pages in a random physical order after one spare page (page 0)."""
    blocks = [-(-s // PAGE) for s in seq_lens]
    pages = sum(blocks) + 1
    perm = torch.randperm(pages - 1, generator=gen, device='cuda') + 1
    r2t = torch.zeros(len(seq_lens), 16384, dtype=torch.int32, device='cuda')
    off = 0
    for r, n in enumerate(blocks):
        for blk in range(n):
            pg = int(perm[off + blk])
            r2t[r, blk * PAGE:(blk + 1) * PAGE] = torch.arange(pg * PAGE, (pg + 1) * PAGE, device='cuda',
                                                               dtype=torch.int32)
        off += n
    return r2t, pages


def _pages(pages, heads, gen, scale=1.0):
    x = (workloads.kv_tensor(pages * PAGE, heads, D, gen, 'cuda').float() * scale).to(torch.bfloat16)
    pay = torch.empty(pages * PAGE, heads, D // 2, dtype=torch.uint8, device='cuda')
    sc = torch.empty(pages * PAGE, heads, D // 16, dtype=torch.uint8, device='cuda')
    ops.quantize_append(x, torch.arange(pages * PAGE, device='cuda'), torch.ones(1, device='cuda'), pay, sc)
    return workloads.head_major_pages(pay, sc, PAGE)


def _rel_l2(got, ref):
    g = got.float().cpu().numpy().astype(np.float64)
    return np.linalg.norm(g - ref) / np.linalg.norm(ref)


@pytest.mark.parametrize('seq_lens', [[4000, 2500, 1300], [8000], [128, 129, 300]])
def test_reference_decode_cases(seq_lens):
    print(f'minimax decode case {seq_lens}', flush=True)
    gen = workloads.generator('cuda', 81 + len(seq_lens) + seq_lens[0])
    b, topk = len(seq_lens), 16
    r2t, pages = _mapping(seq_lens, gen)
    kp, ks = _pages(pages, KH, gen)
    vp, vs = _pages(pages, KH, gen)
    seq = torch.tensor(seq_lens, dtype=torch.int32, device='cuda')
    slot_ids = torch.arange(b, dtype=torch.int32, device='cuda')
    q = torch.randn(b, QH, D, generator=gen, device='cuda').to(torch.bfloat16)
    idx = torch.full((KH, b, topk), -1, dtype=torch.int32, device='cuda')
    for r, s in enumerate(seq_lens):
        for h in range(KH):
            pick = torch.randperm(-(-s // PAGE), generator=gen, device='cuda')[:topk]
            idx[h, r, :len(pick)] = pick.to(torch.int32)
    got = ops.fp4_sparse_decode(q, kp, ks, vp, vs, r2t, slot_ids, idx, seq, PAGE)
    host = [t.cpu().numpy() for t in (kp, ks, vp, vs)]
    args = (q.float().cpu().numpy(), *host, r2t.cpu().numpy(), slot_ids.cpu().numpy(), idx.cpu().numpy(),
            seq.cpu().numpy(), PAGE, D ** -0.5)
    ref, _ = attention.block_sparse_decode(*args)
    flash, _ = attention.block_sparse_decode(*args, attend=attention.flash_precision_attention)
    err, flash_err = _rel_l2(got, ref), _rel_l2(torch.from_numpy(flash), ref)
    assert err < 2e-3 and err <= 1.25 * flash_err, (err, flash_err)
    check(got, ref, flash)


def _prefill_lists(prefix_lens, ext_lens, topk, gen):
    """Per (KV head, query) block lists, query blocks of one: the query's own block, then up to topk - 1 distinct
    earlier blocks (local_blocks 1 of the reference's call), -1 padded."""
    rows = []
    for p, e in zip(prefix_lens, ext_lens):
        for i in range(e):
            own = (p + i) // PAGE
            lst = []
            for h in range(KH):
                far = torch.randperm(own, generator=gen, device='cuda')[:topk - 1].tolist() if own else []
                ids = [own] + far
                lst.append(ids + [-1] * (topk - len(ids)))
            rows.append(lst)
    return torch.tensor(rows, dtype=torch.int32, device='cuda').permute(1, 0, 2).contiguous()


@pytest.mark.parametrize('prefix_lens,ext_lens', [([0], [1500]), ([1000], [500]), ([0, 300], [900, 600]),
                                                  ([5000], [3000])])
def test_reference_prefill_cases(prefix_lens, ext_lens):
    print(f'minimax prefill case prefix {prefix_lens} ext {ext_lens}', flush=True)
    gen = workloads.generator('cuda', 91 + sum(prefix_lens) + sum(ext_lens))
    seq_lens = [p + e for p, e in zip(prefix_lens, ext_lens)]
    b, topk = len(seq_lens), 16
    r2t, pages = _mapping(seq_lens, gen)
    kp, ks = _pages(pages, KH, gen)
    vp, vs = _pages(pages, KH, gen)
    total = sum(ext_lens)
    q = torch.randn(total, QH, D, generator=gen, device='cuda').to(torch.bfloat16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(ext_lens)]), dtype=torch.int32, device='cuda')
    seq = torch.tensor(seq_lens, dtype=torch.int32, device='cuda')
    pre = torch.tensor(prefix_lens, dtype=torch.int32, device='cuda')
    slot_ids = torch.arange(b, dtype=torch.int32, device='cuda')
    idx = _prefill_lists(prefix_lens, ext_lens, topk, gen)
    # the context copies equal the dequantized cache, bit for bit
    rows = -(-max(seq_lens) // PAGE) * PAGE
    copy = ops.dequantize_context(kp, ks, r2t, slot_ids, seq, rows).float().cpu().numpy()
    kph, ksh = kp.cpu().numpy(), ks.cpu().numpy()
    for r, s in enumerate(seq_lens):
        slots = r2t[r, :s].long().cpu().numpy()
        want = nvfp4.dequant(kph[slots // PAGE, :, slots % PAGE], ksh[slots // PAGE, :, slots % PAGE])
        np.testing.assert_array_equal(copy[r * rows:r * rows + s], want)
    # the NVFP4 prefill on sampled query rows
    out = ops.fp4_prefill_gqa_share_sparse(q, kp, vp, None, r2t, slot_ids, idx, 1, PAGE, cu, seq, pre,
                                           max(ext_lens), k_sc=ks, v_sc=vs)
    sample = np.unique(np.concatenate([np.linspace(0, total - 1, 40).astype(int), cu.cpu().numpy()[:-1]]))
    req = np.searchsorted(cu.cpu().numpy()[1:], sample, side='right')
    pos = np.array(prefix_lens)[req] + sample - cu.cpu().numpy()[req]
    n = len(sample)
    args = (q.float().cpu().numpy()[sample], kph, ksh, vp.cpu().numpy(), vs.cpu().numpy(), r2t.cpu().numpy(),
            slot_ids.cpu().numpy()[req], idx.cpu().numpy()[:, sample], np.arange(n + 1), np.arange(n + 1),
            np.array(seq_lens)[req], pos, 1, PAGE, D ** -0.5)
    ref = attention.block_sparse_prefill(*args)
    flash = attention.block_sparse_prefill(*args, attend=attention.flash_precision_attention)
    got = out[torch.from_numpy(sample).cuda()]
    err, flash_err = _rel_l2(got, ref), _rel_l2(torch.from_numpy(flash), ref)
    assert err < 2e-3 and err <= 1.25 * flash_err, (err, flash_err)
    check(got, ref, flash)
