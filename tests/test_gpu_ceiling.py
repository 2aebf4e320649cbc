"""The ceiling kernels the roofline fractions are read against (include/xtier_amd.h xt_ceiling_*): the MFMA loop's
sums, and that the gather reads exactly the listed records (per-row XOR of every valid record's words, skipped
positions, table entries and slots included)."""
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
