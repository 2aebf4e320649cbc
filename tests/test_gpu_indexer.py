"""The top-k producers on the GPU against the oracle (oracle/topk.py): the selection bit for bit on the same FP32
logits; the QSA indexer logits (qsa_prefill.py:77-102) and the DSA FP8 logits (indexer_torch.py:28-72) within the
rounding of FP32 sums of exact products, the masked columns exactly; the hooks that carry them."""
import math

import numpy as np
import pytest
import torch

from oracle import topk as ref
from xtier_amd import glm, ops, qsa

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('cols,k', [(1, 1), (100, 64), (5000, 2048), (4999, 1000), (100000, 2048), (70000, 4096)])
def test_topk_rows_bit_for_bit(cols, k):
    g = torch.Generator().manual_seed(cols + k)
    x = torch.randn(7, cols, generator=g)
    x[0] = torch.round(x[0] * 4) / 4                      # heavy ties
    x[1, : cols // 2] = -math.inf                        # masked half
    x[2] = -math.inf                                     # nothing finite
    if cols > 3:
        x[3, 1], x[3, 2] = math.nan, math.inf            # not finite: never taken
    x[4] = 1.0                                           # all equal: the lowest positions
    zero = torch.where(torch.rand(cols, generator=g) < 0.5, -0.0, 0.0)
    x[6] = torch.where(torch.arange(cols) % 7 == 3, x[6].abs() + 0.5, zero)   # -0 and +0 tie below the positives
    xg = x.cuda()
    got = ops.topk_rows(xg, k).cpu().numpy()
    want = ref.topk_rows(x.numpy(), k)
    assert np.array_equal(got, want)


@pytest.mark.parametrize('cols,k', [(96256, 2048), (70000, 512)])
def test_topk_rows_values_placed_by_position(cols, k):
    """Rows whose largest values sit at positions picked by the row's layout (one element of every other
    2048-position block, its complement, one lane of every 64, one position in 97): the selection must not depend
    on where in the row the large values are."""
    g = torch.Generator().manual_seed(cols)
    pos = torch.arange(cols)
    chunk, lane, elem = pos // 2048, (pos // 4) % 512, pos % 4
    picked = (chunk % 2 == 0) & (elem == (chunk // 2) % 4)
    x = torch.randn(4, cols, generator=g)
    x[0] = torch.where(picked, x[0], x[0] + 10)           # large values everywhere but the picked positions
    x[1] = torch.where(picked, x[1] + 10, x[1])           # large values only at the picked positions
    x[2] = torch.where(lane % 64 == 5, x[2] + 10, x[2])   # the large values all in one lane of every wavefront
    x[3] = torch.where(pos % 97 == 0, x[3], -math.inf)    # about cols / 97 finite values, fewer than k
    got = ops.topk_rows(x.cuda(), k).cpu().numpy()
    assert np.array_equal(got, ref.topk_rows(x.numpy(), k))


def test_topk_rows_empty_rows():
    x = torch.randn(3, 8, device='cuda')[:, :0]          # rows of no column: nothing is read, every entry is -1
    assert np.array_equal(ops.topk_rows(x, 5).cpu().numpy(), np.full((3, 5), -1, np.int32))


def test_topk_rows_strided_rows_and_out():
    x = torch.randn(5, 3000, device='cuda')
    out = torch.full((5, 100), 7, dtype=torch.int32, device='cuda')
    ops.topk_rows(x[:, :2500], 100, out=out)
    assert np.array_equal(out.cpu().numpy(), ref.topk_rows(x[:, :2500].cpu().numpy(), 100))


def _bound_qsa(q, k, scale):
    """FP32 summation bound of the head sum of ReLU(q . k) / scale: exact products summed over dim, then over heads."""
    a = np.einsum('rhd,nd->rn', np.abs(q), np.abs(k))
    dim, heads = q.shape[2], q.shape[1]
    return (dim + heads + 2) * 2.0 ** -24 * a / scale


@pytest.mark.parametrize('rows,heads,dim,keys,dtype', [
    (37, 4, 128, 1000, torch.bfloat16), (352, 4, 128, 4096, torch.bfloat16), (5, 1, 64, 333, torch.bfloat16),
    (9, 8, 256, 700, torch.float16), (3, 32, 128, 257, torch.bfloat16), (20, 16, 64, 2100, torch.float16)])
def test_qsa_indexer_logits(rows, heads, dim, keys, dtype):
    g = torch.Generator().manual_seed(rows * keys)
    q = torch.randn(rows, heads, dim, generator=g).to(dtype)
    k = torch.randn(keys, 1, dim, generator=g).to(dtype)
    # causal ranges as the reference's check builds them (tests/qsa_prefill_check.py:25-33), plus empty and clipped
    pos = torch.arange(rows) * (keys // max(1, rows)) + keys // 3
    starts = torch.zeros(rows, dtype=torch.int32)
    ends = torch.clamp((pos + 1), max=keys + 50).to(torch.int32)
    starts[0], ends[0] = 5, 5
    if rows > 2:
        starts[2] = keys // 2
    got = ops.qsa_indexer_logits(q.cuda(), k.cuda(), starts.cuda(), ends.cuda()).cpu().numpy()
    qn, kn = q.float().numpy().astype(np.float64), k[:, 0].float().numpy().astype(np.float64)
    want = ref.qsa_indexer_logits(qn, kn, starts.numpy(), ends.numpy())
    assert np.array_equal(np.isinf(got), np.isinf(want)) and not np.isnan(got).any()
    fin = np.isfinite(want)
    err = np.abs(got.astype(np.float64)[fin] - want[fin])
    # the kernel multiplies by 1 / score_scale: one rounding of the reciprocal and one of the product
    bound = (_bound_qsa(qn, kn, math.sqrt(dim)) + np.abs(want) * 2.0 ** -23)[fin]
    assert (err <= bound).all(), float((err / bound).max())


@pytest.mark.parametrize('rows,prefix', [(352, 380000), (1000, 100000), (64, 8192), (4096, 30000), (37, 500000)])
def test_qsa_indexer_logits_reference_cases(rows, prefix):
    """The cases of tests/qsa_prefill_check.py:25-53: 4 heads x 128, compressed keys (ratio 4) up to the last row, each
    row's range [0, (pos + 1) / 4)."""
    g = torch.Generator().manual_seed(20261023 + rows)
    keys = (prefix + rows) // 4
    q = torch.randn(rows, 4, 128, generator=g).bfloat16()
    k = torch.randn(keys, 1, 128, generator=g).bfloat16()
    starts = torch.zeros(rows, dtype=torch.int32)
    ends = ((torch.arange(prefix, prefix + rows) + 1) // 4).to(torch.int32)
    got = ops.qsa_indexer_logits(q.cuda(), k.cuda(), starts.cuda(), ends.cuda()).cpu().numpy()
    qn, kn = q.float().numpy().astype(np.float64), k[:, 0].float().numpy().astype(np.float64)
    want = ref.qsa_indexer_logits(qn, kn, starts.numpy(), ends.numpy())
    fin = np.isfinite(want)
    assert np.array_equal(np.isinf(got), ~fin) and not np.isnan(got).any()
    a = np.zeros(want.shape)
    for h in range(4):
        a += np.abs(qn[:, h]) @ np.abs(kn).T
    bound = (130 + 4 + 2) * 2.0 ** -24 * a / math.sqrt(128) + np.abs(want) * 2.0 ** -23
    assert (np.abs(got.astype(np.float64)[fin] - want[fin]) <= bound[fin]).all()


def test_qsa_prefill_hook():
    calls = []
    original = lambda *a: calls.append(a) or 'original'
    q = torch.randn(4, 4, 128).bfloat16()
    k = torch.randn(9, 1, 128).bfloat16()
    s, e = torch.zeros(4, dtype=torch.int32), torch.full((4,), 9, dtype=torch.int32)
    assert qsa.qsa_mqa_prefill(original, q, k, s, e) == 'original'            # CPU tensors
    assert qsa.qsa_mqa_prefill(original, q.cuda()[:, :3], k.cuda(), s, e) == 'original'   # 3 heads
    got = qsa.qsa_mqa_prefill(original, q.cuda(), k.cuda(), s.cuda(), e.cuda(), 2.0)
    assert len(calls) == 2 and got.shape == (4, 9)
    want = ref.qsa_indexer_logits(q.float().numpy(), k[:, 0].float().numpy(), s.numpy(), e.numpy(), 2.0)
    assert np.allclose(got.cpu().numpy(), want, rtol=1e-5, atol=1e-5)


def _fp8(shape, g, scale=2.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.float8_e4m3fn)


@pytest.mark.parametrize('num_q,heads,num_kv,clean', [(300, 32, 1000, False), (64, 64, 5000, True),
                                                      (7, 96, 33, False)])
def test_dsa_mqa_logits(num_q, heads, num_kv, clean):
    """The shapes of tests/glm_indexer_torch_check.py:27-43 (300 queries x 1000 keys, 32 heads x 128) and wider."""
    g = torch.Generator().manual_seed(num_q + heads)
    q, k = _fp8((num_q, heads, 128), g), _fp8((num_kv, 128), g)
    k_scale = torch.rand(num_kv, generator=g) + 0.5
    w = torch.randn(num_q, heads, generator=g)
    ks = torch.randint(0, max(1, num_kv // 2), (num_q,), generator=g, dtype=torch.int32)
    ke = ks + torch.randint(1, num_kv, (num_q,), generator=g, dtype=torch.int32)
    got = glm.fp8_mqa_logits(None, q.cuda(), (k.cuda(), k_scale.cuda()), w.cuda(), ks.cuda(), ke.cuda(), clean)
    assert got.shape == (num_q, num_kv) and got.stride(0) == (num_kv + 3) // 4 * 4
    got = got.cpu().numpy().astype(np.float64)
    want = ref.dsa_mqa_logits(q.float().numpy(), k.float().numpy(), k_scale.numpy(), w.numpy(), ks.numpy(),
                              ke.numpy(), clean)
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    rel = np.linalg.norm(got[fin] - want[fin]) / np.linalg.norm(want[fin])
    assert rel < 1e-5, rel                                 # the reference's own bound (glm_indexer_torch_check.py:42)
    a = (np.einsum('qhd,nd->qhn', np.abs(q.float().numpy()), np.abs(k.float().numpy())) *
         np.abs(w.numpy())[:, :, None]).sum(1) * k_scale.numpy()[None, :]
    assert (np.abs(got[fin] - want[fin]) <= ((128 + heads + 4) * 2.0 ** -24 * a)[fin] + 1e-30).all()


@pytest.mark.parametrize('scale', [0.05, 2.0, 20.0])
def test_dsa_logits_one_head_within_the_fp32_sum_bound(scale):
    """With one-hot head weights and unit key scales each logit is ReLU of one 128-term FP8 dot product: held to the
    bound of an FP32 sum of exact products (an FP8 matrix instruction that rounds inside its 16-product sums misses it
    by hundreds of units in the last place)."""
    g = torch.Generator().manual_seed(7)
    num_q, heads, num_kv, dim = 256, 32, 1024, 128
    q, k = _fp8((num_q, heads, dim), g, scale), _fp8((num_kv, dim), g, scale)
    w = torch.zeros(num_q, heads)
    w[torch.arange(num_q), torch.arange(num_q) % heads] = 1.0
    ks = torch.zeros(num_q, dtype=torch.int32)
    ke = torch.full((num_q,), num_kv, dtype=torch.int32)
    got = ops.dsa_mqa_logits(q.cuda(), (k.cuda(), torch.ones(num_kv, device='cuda')), w.cuda(), ks.cuda(),
                             ke.cuda()).cpu().numpy().astype(np.float64)
    qs = q.float().numpy().astype(np.float64)[np.arange(num_q), np.arange(num_q) % heads]
    kd = k.float().numpy().astype(np.float64)
    exact = np.maximum(qs @ kd.T, 0.0)
    assert (np.abs(got - exact) <= (dim + 2) * 2.0 ** -24 * (np.abs(qs) @ np.abs(kd).T)).all()


def test_dsa_paged_mqa_logits():
    """The decode case of tests/glm_indexer_torch_check.py:44-65: 3 rows over 8 pages of 64 in a pool of 40."""
    g = torch.Generator().manual_seed(20261029)
    H, D, BLOCK, pages = 32, 128, 64, 40
    kv = torch.empty(pages, BLOCK * (D + 4), dtype=torch.uint8)
    vals = _fp8((pages, BLOCK, D), g)
    scl = torch.rand(pages, BLOCK, generator=g) + 0.5
    kv[:, :BLOCK * D] = vals.view(torch.uint8).reshape(pages, -1)
    kv[:, BLOCK * D:] = scl.view(torch.uint8).reshape(pages, -1)
    kv4 = kv.view(pages, BLOCK, 1, D + 4)
    table = torch.randperm(pages, generator=g)[:24].view(3, 8).to(torch.int32)
    lens = torch.tensor([512, 300, 77], dtype=torch.int32)
    q = _fp8((3, 1, H, D), g)
    w = torch.randn(3, H, generator=g)
    for clean in (False, True):
        for msl in (8 * BLOCK, 8 * BLOCK + 100):
            got = glm.fp8_paged_mqa_logits(None, q.cuda(), kv4.cuda(), w.cuda(), lens.view(3, 1).cuda(),
                                           table.cuda(), None, msl, clean).cpu().numpy().astype(np.float64)
            want = ref.dsa_paged_mqa_logits(q[:, 0].float().numpy(), kv.numpy(), w.numpy(), lens.numpy(),
                                            table.numpy(), msl, clean)
            assert np.array_equal(np.isinf(got), np.isinf(want)) and got.shape == want.shape
            fin = np.isfinite(want) & (want != 0)
            assert np.linalg.norm(got[fin] - want[fin]) / np.linalg.norm(want[fin]) < 1e-5
            assert np.array_equal(got[~fin & ~np.isinf(want)], want[~fin & ~np.isinf(want)])


def test_glm_schedule_and_sm_count():
    assert glm.get_paged_mqa_logits_metadata(None, 1, 2, x=3) is None
    assert glm.get_num_sms(None) == torch.cuda.get_device_properties(0).multi_processor_count
    assert {t for t, _ in glm.HOOKS} == {'deep_gemm.fp8_mqa_logits', 'deep_gemm.fp8_paged_mqa_logits',
                                         'deep_gemm.get_paged_mqa_logits_metadata', 'deep_gemm.get_num_sms'}
