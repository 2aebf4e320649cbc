"""The ceiling kernels the roofline fractions are read against (include/xtier_amd.h xt_ceiling_*): the MFMA loop's
sums, that the gather reads exactly the listed records (per-row XOR of every valid record's words, skipped
positions, table entries and slots included), and that the split-arrival probe merges every group's partials and
leaves its counters at zero, in both of its forms, on two calls in a row."""
import numpy as np
import pytest
import torch

from xtier_amd import ops, workloads

pytestmark = pytest.mark.gpu


def test_mfma_ceiling_sums():
    out = ops.ceiling_mfma(37, 3)
    assert out.shape == (3 * 256,) and bool((out == 64.0 * 37).all())


@pytest.mark.parametrize('topk,record', [(1, 576), (300, 576), (512, 576), (300, 160)])
def test_gather_ceiling_reads_exactly_the_listed_records(topk, record):
    """576-byte records take the unrolled kernel, other sizes the generic loop."""
    batch, ctx, page, records = 3, 4096, 64, 3 * 4096 + 64
    gen = workloads.generator('cuda', topk)
    pool = torch.randint(0, 256, (records, record), dtype=torch.uint8, device='cuda', generator=gen)
    pt = workloads.page_table(batch, ctx, page, gen, 'cuda')
    idx = workloads.index_lists(batch, ctx, topk, gen, 'cuda')
    idx[0, 0] = -1                          # an invalid position
    if topk > 1:
        idx[1, 1] = ctx + 5 * page          # a position past the table
        pt[2, int(idx[2, 0]) // page] = -1  # a missing page
    sink = ops.ceiling_gather(pool, pt, idx, page)
    chunks = (topk + 255) // 256
    got = np.bitwise_xor.reduce(sink.cpu().numpy().astype(np.uint32).reshape(batch, chunks * 512), axis=1)
    words = pool.cpu().numpy().view(np.uint32)          # [records, record / 4]
    p, t = idx.cpu().numpy(), pt.cpu().numpy()
    for r in range(batch):
        want = np.uint32(0)
        for pos in p[r]:
            if pos < 0 or pos // page >= t.shape[1] or t[r, pos // page] < 0:
                continue
            want ^= np.bitwise_xor.reduce(words[t[r, pos // page] * page + pos % page])
        assert got[r] == want, r


@pytest.mark.parametrize('topk,splits', [(512, 2), (2048, 2), (1024, 4), (256, 1)])
def test_gather_pieces_reads_each_units_head_pieces(topk, splits):
    """Workgroup g's words XOR to the XOR of its unit's head pieces (128 payload + 16 scale bytes) over the valid keys
    of its split, the unit numbered as the decode numbers them."""
    batch, ctx, page = 3, 4096, 64
    records = batch * ctx + 64
    gen = workloads.generator('cuda', topk + splits)
    pool = torch.randint(0, 256, (records, 576), dtype=torch.uint8, device='cuda', generator=gen)
    pt = workloads.page_table(batch, ctx, page, gen, 'cuda')
    idx = workloads.index_lists(batch, ctx, topk, gen, 'cuda')
    idx[0, 3] = -1
    idx[1, 7] = ctx + 9 * page
    pt[2, int(idx[2, 0]) // page] = -1
    sink = ops.ceiling_gather_pieces(pool, pt, idx, page, splits)
    n = batch * 4 * splits
    got = np.bitwise_xor.reduce(sink.cpu().numpy().astype(np.uint32).reshape(n, 512), axis=1)
    words = pool.cpu().numpy().view(np.uint32)          # [records, 144]
    p, t = idx.cpu().numpy(), pt.cpu().numpy()
    kps = topk // splits
    for g in range(n):
        x = g % 8
        u = x * (n // 8) + min(x, n % 8) + g // 8
        split, head, row = u % splits, (u // splits) % 4, u // splits // 4
        want = np.uint32(0)
        for pos in p[row, split * kps:(split + 1) * kps]:
            if pos < 0 or pos // page >= t.shape[1] or t[row, pos // page] < 0:
                continue
            w = words[t[row, pos // page] * page + pos % page]
            want ^= np.bitwise_xor.reduce(w[32 * head:32 * head + 32]) ^ np.bitwise_xor.reduce(
                w[128 + 4 * head:128 + 4 * head + 4])
        assert got[g] == want, g


@pytest.mark.parametrize('splits,nbytes,fenced', [(2, 4224, False), (2, 4224, True), (4, 8448, False),
                                                  (8, 16896, False), (8, 16896, True)])
def test_split_merge_probe_merges_every_group(splits, nbytes, fenced):
    """The last arriver of each group of `splits` workgroups sums the group's partials (words {offset, 1, 2, 3}):
    thread t gets splits * sum(offset + 1) over its 16-byte words; the counters are zero again after each call."""
    blocks = 64 * splits
    part = torch.zeros(blocks * nbytes, dtype=torch.uint8, device='cuda')
    counters = torch.zeros(blocks // splits, dtype=torch.int32, device='cuda')
    out = torch.full((blocks // splits * 512,), -1, dtype=torch.int32, device='cuda')
    want = np.array([(splits * sum(o + 1 for o in range(t * 16, nbytes, 8192))) & 0xFFFFFFFF for t in range(512)])
    for _ in range(2):
        ops.ceiling_split_merge(part, counters, out, splits, nbytes, blocks, fenced)
        torch.cuda.synchronize()
        got = out.view(-1, 512).cpu().numpy().astype(np.int64) & 0xFFFFFFFF
        assert (got == want[None, :]).all()
        assert int(counters.abs().sum()) == 0
    ops.ceiling_launch(256)
    torch.cuda.synchronize()
