"""The QSA hooks on the GPU with a stand-in SGLang backend: paged_attention (fused over the NVFP4 pool) against the FP64
oracle, extraction / pack_qsa_prefill_kv inside forward_extend equal to the direct gather / pack, and a captured
paged_attention replayed equal to eager (tests/qsa_decode_check.py:94-108)."""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from tests._attn import check, oracle
from tests._pools import bf16_numpy, random_pool
from xtier_amd import ops, qsa, workloads

pytestmark = pytest.mark.gpu


class _Method:
    name = 'nvfp4'

    def __init__(self, gk, gv):
        self.k_scales_gpu = torch.stack([gk[0] * 0 + 9, gk[0]])     # layer 1 is the pool's
        self.v_scales_gpu = torch.stack([gv[0] * 0 + 9, gv[0]])


class _KVPool:
    def __init__(self, raw):
        self.raw = raw
        self.method = _Method(raw[4], raw[5])

    def get_kv_cache_quant_method(self):
        return self.method

    def get_raw_kv_buffer(self, layer_id):
        assert layer_id == 1
        return self.raw[:4]


class _Backend:
    def __init__(self, raw, req_to_token, seq_lens, rows=None):
        self.token_to_kv_pool = _KVPool(raw)
        self.req_to_token_pool = SimpleNamespace(req_to_token=req_to_token)
        self.meta = SimpleNamespace(row_req_pool_indices=rows, sequence_lengths=seq_lens)

    def _resolve_metadata(self, forward_batch):
        return self.meta

    def _expand_block_indices(self, topk_indices, metadata):
        return topk_indices


def _setup(seed=3, reqs=6, ctx=2048, topk=300, heads=4, qh=32, dim=128):
    pool = random_pool(seed, reqs * ctx, heads, dim)
    gen = workloads.generator('cpu', seed + 1)
    pt = workloads.page_table(reqs, ctx, 64, gen, 'cpu')
    r2t = workloads.token_table(pt, 64)
    idx = workloads.index_lists(reqs, ctx, topk, gen, 'cpu')
    idx[1, ::5] = -1
    seq = torch.full((reqs,), ctx, dtype=torch.int32)
    seq[2] = ctx // 2
    q = (torch.randn(reqs, qh * dim, generator=gen) * 2).to(torch.bfloat16)
    return pool, r2t, idx, seq, q


@pytest.mark.parametrize('heads,qh,dim', [
    (4, 32, 128),
    (2, 24, 256),   # the reference's Qwen3.8 QSA shape (tests/qsa_fp4_check.py:21, tests/qsa_decode_check.py:54)
    (2, 16, 64),
])
def test_paged_attention_fused_matches_oracle(heads, qh, dim):
    pool, r2t, idx, seq, q = _setup(heads=heads, qh=qh, dim=dim)
    reqs = q.shape[0]
    rows = torch.tensor([5, 4, 3, 2, 1, 0])        # row r reads request 5 - r
    backend = _Backend(pool.raw, r2t.cuda(), seq[rows].cuda(), rows=rows.cuda())
    layer = SimpleNamespace(layer_id=1, scaling=1 / math.sqrt(dim))
    out = qsa.paged_attention(None, backend, q.cuda(), layer, SimpleNamespace(req_pool_indices=None),
                              idx[rows].cuda())
    assert out.shape == (reqs, qh * dim) and out.dtype == torch.bfloat16
    ref, flash, _ = oracle(pool.raw, bf16_numpy(q).reshape(reqs, qh, dim), r2t.numpy(), 1, rows.numpy(),
                           idx[rows].numpy(), None, seq[rows].numpy(), 1 / math.sqrt(dim))
    check(out.view(reqs, qh, dim), ref, flash)


def test_extraction_and_pack_inside_forward_extend():
    pool, r2t, idx, seq, q = _setup(seed=8)
    reqs, topk = idx.shape
    backend = _Backend(pool.raw, r2t.cuda(), seq.cuda())
    layer = SimpleNamespace(layer_id=1)
    req = torch.arange(reqs, dtype=torch.int64).cuda()
    valid = ((idx >= 0) & (idx < seq[:, None])).sum(1)
    cu_k = torch.cat([torch.zeros(1, dtype=torch.int32), torch.cumsum(valid, 0).to(torch.int32)]).cuda()
    total = int(cu_k[-1])
    seen = {}

    def original(self, q_, k_, v_, layer_, fb):
        a = torch.full((total, 4, 128), float('nan'), dtype=torch.bfloat16, device='cuda')
        b = a.clone()
        qsa.extraction(None, None, None, r2t.cuda(), req, idx.cuda(), seq.cuda(), cu_k, a, b, reqs, topk)
        seen['gather'] = (a, b)
        seen['pack'] = qsa.pack_qsa_prefill_kv(None, k=None, v=None, req_to_token=r2t.cuda(), req_indices=req,
                                               cu_k=cu_k, total_k=total, max_k=topk)
        return 'done'
    assert qsa.forward_extend(original, backend, None, None, None, layer, None) == 'done'
    a2 = torch.full_like(seen['gather'][0], float('nan'))
    b2 = a2.clone()
    ops.gather(pool.raw, r2t.cuda(), req, idx.cuda(), seq.cuda(), cu_k, a2, b2, reqs, topk)
    assert torch.equal(seen['gather'][0].view(torch.int16), a2.view(torch.int16))
    assert torch.equal(seen['gather'][1].view(torch.int16), b2.view(torch.int16))
    pk, pv = ops.pack(pool.raw, r2t.cuda(), req, cu_k, total, topk, torch.bfloat16)
    assert torch.equal(seen['pack'][0].view(torch.int16), pk.view(torch.int16))
    assert torch.equal(seen['pack'][1].view(torch.int16), pv.view(torch.int16))


@pytest.mark.parametrize('heads,qh,dim', [(4, 32, 128), (2, 24, 256)])
def test_paged_attention_graph_replay_equals_eager(heads, qh, dim):
    pool, r2t, idx, seq, q = _setup(seed=12, heads=heads, qh=qh, dim=dim)
    backend = _Backend(pool.raw, r2t.cuda(), seq.cuda())
    layer = SimpleNamespace(layer_id=1, scaling=0.09)
    fb = SimpleNamespace(req_pool_indices=torch.arange(q.shape[0]).cuda())
    qs = q.cuda().clone()
    idx_d = idx.cuda()
    qsa.paged_attention(None, backend, qs, layer, fb, idx_d)      # eager first: the workspace exists before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = qsa.paged_attention(None, backend, qs, layer, fb, idx_d)
    gen = torch.Generator().manual_seed(4)
    for _ in range(3):
        qs.copy_((torch.randn(q.shape, generator=gen) * 2).to(torch.bfloat16).cuda())
        graph.replay()
        torch.cuda.synchronize()
        eager = qsa.paged_attention(None, backend, qs, layer, fb, idx_d)
        torch.cuda.synchronize()
        assert torch.equal(captured.view(torch.int16), eager.view(torch.int16))
