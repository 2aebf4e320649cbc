"""Sparse MLA on DeepSeek V4 FP8 pages (sparse_mla.py:167-231) on the GPU against the FP64 oracle, measured as the
reference test measures it (max |err| / max |ref| < 1e-2, rms err / rms ref < 4e-3, tests/ds_sparse_mla_check.py:70-75,
:160): a window cache in pages of 256 and a compressed cache in pages of 128, holes, shorter lists, the sink, rows
without keys, decode-sized (split keys, FP32 merge) and prefill-sized calls, 64 and 128 heads, graph replay equal to
eager, and the flash_mla_with_kvcache hook."""
import numpy as np
import pytest
import torch

from oracle import attention
from tests._v4 import pack_v4
from xtier_amd import deepseek, ops

pytestmark = pytest.mark.gpu
SCALE = 512 ** -0.5


def _caches():
    g = torch.Generator().manual_seed(20261029)
    lat1 = torch.randn(4096, 512, generator=g) * torch.rand(4096, 1, generator=g) * 4
    lat2 = torch.randn(2048, 512, generator=g) * torch.rand(2048, 1, generator=g) * 4
    c1, k1, _ = pack_v4(lat1, 256)
    c2, k2, _ = pack_v4(lat2, 128)
    return c1, k1, c2, k2


CACHES = None


def _get():
    global CACHES
    if CACHES is None:
        c1, k1, c2, k2 = _caches()
        CACHES = (c1.cuda(), k1, c2.cuda(), k2)
    return CACHES


def _inputs(rows, heads, n1, n2, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(rows, 1, heads, 512, generator=g) * 2).to(torch.bfloat16)
    i1 = torch.randint(0, 4096, (rows, 1, n1), generator=g, dtype=torch.int32)
    i2 = torch.randint(0, 2048, (rows, 1, n2), generator=g, dtype=torch.int32)
    i1[:, :, ::7] = -1
    l1 = torch.full((rows,), n1, dtype=torch.int32)
    l2 = torch.full((rows,), n2, dtype=torch.int32)
    l1[1 % rows] = n1 // 3
    sink = torch.randn(heads, generator=g)
    return q, i1, i2, l1, l2, sink


def _errors(out, ref, nonempty):
    o = out.reshape(ref.shape).float().cpu().numpy().astype(np.float64)[nonempty]
    r = ref[nonempty]
    assert np.isfinite(o).all()
    d = o - r
    return np.abs(d).max() / np.abs(r).max(), np.sqrt((d ** 2).mean()) / np.sqrt((r ** 2).mean())


@pytest.mark.parametrize('rows,heads,n1,n2,splits', [(6, 64, 128, 512, None), (6, 128, 128, 512, 3),
                                                     (300, 64, 128, 512, None), (4, 128, 2048, 0, 8)])
def test_v4_against_oracle(rows, heads, n1, n2, splits):
    c1, k1, c2, k2 = _get()
    q, i1, i2, l1, l2, sink = _inputs(rows, heads, n1, max(n2, 1), rows + heads)
    two = n2 > 0
    out, lse = ops.sparse_mla(q.cuda(), c1, i1.cuda(), l1.cuda(), sink.cuda(), SCALE,
                              c2 if two else None, i2.cuda() if two else None, l2.cuda() if two else None,
                              splits=splits)
    assert out.shape == (rows, 1, heads, 512) and lse.shape == (rows, heads, 1)
    ref, ref_lse = attention.sparse_mla_v4(q[:, 0].float().numpy(), k1, i1[:, 0].numpy(), l1.numpy(),
                                           sink.numpy(), SCALE, k2 if two else None,
                                           i2[:, 0].numpy() if two else None, l2.numpy() if two else None)
    nonempty = np.isfinite(ref_lse).any(1)
    max_rel, rms_rel = _errors(out[:, 0], ref, nonempty)
    assert max_rel < 1e-2 and rms_rel < 4e-3, (max_rel, rms_rel)
    l_ = lse[:, :, 0].cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert (np.isfinite(l_) == fin).all() and np.abs(l_[fin] - ref_lse[fin]).max() < 2e-3


def test_v4_rows_without_keys():
    c1, k1, c2, k2 = _get()
    q, i1, i2, l1, l2, sink = _inputs(5, 64, 64, 64, 9)
    l1[0] = 0
    l2[0] = 0
    i1[2] = -1
    i2[2] = -1
    out, lse = ops.sparse_mla(q.cuda(), c1, i1.cuda(), l1.cuda(), sink.cuda(), SCALE, c2, i2.cuda(), l2.cuda(),
                              splits=2)
    o = out[:, 0].float().cpu()
    for r in (0, 2):
        assert torch.equal(o[r], torch.zeros_like(o[r])) and torch.isneginf(lse[r]).all()
    assert torch.isfinite(o).all()


def test_v4_graph_replay_equals_eager():
    c1, k1, c2, k2 = _get()
    q, i1, i2, l1, l2, sink = _inputs(8, 128, 256, 256, 11)
    qd, i1d, i2d, l1d, l2d, sd = (t.cuda() for t in (q, i1, i2, l1, l2, sink))
    splits = 2
    ws = torch.zeros(ops.mla_workspace_bytes(8, 128, splits, v4=True), dtype=torch.uint8, device='cuda')
    out = torch.empty(8, 128, 512, dtype=torch.bfloat16, device='cuda')
    lse = torch.empty(8, 128, dtype=torch.float32, device='cuda')
    args = (c1, i1d, l1d, sd, SCALE, c2, i2d, l2d)
    ops.sparse_mla(qd[:, 0], *args, out=out, lse=lse, splits=splits, ws=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.sparse_mla(qd[:, 0], *args, out=out, lse=lse, splits=splits, ws=ws)
    gen = torch.Generator(device='cuda').manual_seed(3)
    for _ in range(3):
        qd.copy_((torch.randn(qd.shape, generator=gen, device='cuda') * 2).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager, _ = ops.sparse_mla(qd[:, 0], *args, splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16))


def test_flash_mla_hook():
    """sparse_mla.py:220-231: keyword calls with indices on an FP8 V4 cache run the sparse MLA; others fall through."""
    c1, k1, c2, k2 = _get()
    q, i1, i2, l1, l2, sink = _inputs(4, 64, 64, 64, 13)
    kw = dict(q=q.cuda(), k_cache=c1, indices=i1.cuda(), topk_length=l1.cuda(), attn_sink=sink.cuda(),
              softmax_scale=SCALE, is_fp8_kvcache=True, head_dim_v=512, extra_k_cache=c2,
              extra_indices_in_kvcache=i2.cuda(), extra_topk_length=l2.cuda())
    got = deepseek.flash_mla_with_kvcache(None, **kw)
    want = ops.sparse_mla(q.cuda(), c1, i1.cuda(), l1.cuda(), sink.cuda(), SCALE, c2, i2.cuda(), l2.cuda())
    assert torch.equal(got[0].view(torch.int16), want[0].view(torch.int16))
    assert deepseek.flash_mla_with_kvcache(lambda *a, **k: 'original', **dict(kw, is_fp8_kvcache=False)) == 'original'
    assert deepseek.flash_mla_with_kvcache(lambda *a, **k: 'original', **dict(kw, head_dim_v=448)) == 'original'


REF_CACHES = None


def _reference_caches():
    """The caches of tests/ds_sparse_mla_check.py:108-120: a 16384-token window cache in pages of 256 and an 8192-slot
    compressed cache in pages of 128, latents N(0, 1) times U(0, 4) per token."""
    global REF_CACHES
    if REF_CACHES is None:
        g = torch.Generator().manual_seed(20261029)
        lat1 = torch.randn(16384, 512, generator=g) * torch.rand(16384, 1, generator=g) * 4
        lat2 = torch.randn(8192, 512, generator=g) * torch.rand(8192, 1, generator=g) * 4
        c1, k1, _ = pack_v4(lat1, 256)
        c2, k2, _ = pack_v4(lat2, 128)
        REF_CACHES = (c1.cuda(), k1, c2.cuda(), k2)
    return REF_CACHES


@pytest.mark.parametrize('rows', [1, 2, 12, 300, 4096])
@pytest.mark.parametrize('extra', [False, True])
def test_v4_reference_case_matrix(rows, extra):
    """The case matrix of tests/ds_sparse_mla_check.py:127-160: 128 heads, window lists of 128 with 10 % holes, a
    valid first entry and lengths 1..128; compressed lists of 512 with 10 % holes and lengths 0..512 (the first
    rows / 8 rows empty); the sink. All rows against the oracle (every 64th of the 4096)."""
    print(f'v4 case rows={rows} extra={extra}', flush=True)
    c1, k1, c2, k2 = _reference_caches()
    g = torch.Generator().manual_seed(1000 * rows + extra)
    heads = 128
    q = (torch.randn(rows, 1, heads, 512, generator=g) * 2).to(torch.bfloat16)
    idx1 = torch.randint(0, 16384, (rows, 1, 128), generator=g, dtype=torch.int32)
    idx1[torch.rand(idx1.shape, generator=g) < 0.1] = -1
    idx1[:, 0, 0] = torch.randint(0, 16384, (rows,), generator=g, dtype=torch.int32)
    len1 = torch.randint(1, 129, (rows,), generator=g, dtype=torch.int32)
    idx2 = len2 = None
    if extra:
        idx2 = torch.randint(0, 8192, (rows, 1, 512), generator=g, dtype=torch.int32)
        idx2[torch.rand(idx2.shape, generator=g) < 0.1] = -1
        len2 = torch.randint(0, 513, (rows,), generator=g, dtype=torch.int32)
        len2[:max(1, rows // 8)] = 0
    sink = torch.randn(heads, generator=g)
    cuda = lambda t: None if t is None else t.cuda()
    out, lse = ops.sparse_mla(q.cuda(), c1, idx1.cuda(), len1.cuda(), sink.cuda(), SCALE, c2 if extra else None,
                              cuda(idx2), cuda(len2))
    rows_checked = np.arange(0, rows, 64) if rows > 300 else np.arange(rows)
    sel = torch.from_numpy(rows_checked)
    ref, ref_lse = attention.sparse_mla_v4(q[sel, 0].float().numpy(), k1, idx1[sel, 0].numpy(), len1[sel].numpy(),
                                           sink.numpy(), SCALE, k2 if extra else None,
                                           idx2[sel, 0].numpy() if extra else None,
                                           len2[sel].numpy() if extra else None)
    nonempty = np.isfinite(ref_lse).any(1)
    max_rel, rms_rel = _errors(out[sel.cuda(), 0], ref, nonempty)
    assert max_rel < 1e-2 and rms_rel < 4e-3, (max_rel, rms_rel)
    l_ = lse[sel.cuda(), :, 0].cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert (np.isfinite(l_) == fin).all() and np.abs(l_[fin] - ref_lse[fin]).max() < 2e-3
