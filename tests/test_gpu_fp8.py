"""The QSA path on an FP8 (E4M3) pool on the GPU (the FP8 branch of xtier/packs/qwen4_exp/qsa_fp4.py:104-116, checked by
tests/qsa_fp8_check.py at Qwen3.8's QSA shape, 2 KV heads x 256, with per-token magnitudes over four decades): the
decode gather in both layouts and the prefix pack bit for bit against the oracle (NaN compared as NaN, as the
reference compares), the packed-row layout of the top-k lists, and paged_attention through the hook (gather + split-K
decode) against the FP64 oracle."""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import attention, nvfp4
from tests._attn import check
from xtier_amd import ops, qsa

pytestmark = pytest.mark.gpu

HEADS, DIM, ROWS = 2, 256, 70000


def _pool(seed, lo=-3.0, hi=1.0):
    gen = torch.Generator().manual_seed(seed)
    mag = 10 ** torch.empty(ROWS, 1, 1).uniform_(lo, hi, generator=gen)
    k8, v8 = ((torch.randn(ROWS, HEADS, DIM, generator=gen) * mag).to(torch.float8_e4m3fn) for _ in range(2))
    return k8.view(torch.uint8), v8.view(torch.uint8)


def _same_bits(got, want):
    g = got.view(torch.int16).cpu().numpy().view(np.uint16).copy()
    nan = (g & 0x7FFF) > 0x7F80
    g[nan] = 0x7FC0
    w = want.copy()
    w[(w & 0x7FFF) > 0x7F80] = 0x7FC0
    return np.array_equal(g, w)


def _lists(gen, batch, topk, seq_lens):
    idx = torch.full((batch, topk), -1, dtype=torch.int32)
    counts = []
    for b, n in enumerate((2048, 1500, 2000)[:batch]):
        idx[b, :n] = torch.randperm(int(seq_lens[b]), generator=gen)[:n].to(torch.int32)
        counts.append(n)
    return idx, counts


def test_fp8_gather_both_layouts_and_pack_bit_exact():
    k8, v8 = _pool(20261029)
    host = (k8.numpy(), v8.numpy(), None, None, None, None)
    raw = (k8.cuda(), v8.cuda(), None, None, None, None)
    gen = torch.Generator().manual_seed(1)
    batch, topk, width = 3, 2048, 120000
    r2t = torch.randint(0, ROWS, (4, width), dtype=torch.int32, generator=gen)
    req = torch.tensor([2, 0, 3], dtype=torch.int64)
    seq = torch.tensor([50000, 3000, 69000], dtype=torch.int32)
    idx, counts = _lists(gen, batch, topk, seq)
    cu = torch.tensor([0] + counts).cumsum(0).to(torch.int32)
    for cu_k, zf in ((cu, 0), (torch.arange(batch + 1, dtype=torch.int32) * 2112, 2112)):
        cap = int(cu_k[-1])
        out_k = torch.full((cap, HEADS, DIM), float('nan'), dtype=torch.bfloat16, device='cuda')
        out_v = out_k.clone()
        ops.gather(raw, r2t.cuda(), req.cuda(), idx.cuda(), seq.cuda(), cu_k.cuda(), out_k, out_v, batch, topk,
                   zero_fill_cols=zf)
        want_k = np.full((cap, HEADS, DIM), 0x7FC0, np.uint16)
        want_v = want_k.copy()
        attention.gather_qsa(host, r2t.numpy(), req.numpy(), idx.numpy(), seq.numpy(), cu_k.numpy(), want_k, want_v,
                             batch, topk, zero_fill_cols=zf)
        assert _same_bits(out_k, want_k) and _same_bits(out_v, want_v), zf
    p_req = torch.tensor([1, 3], dtype=torch.int64)
    p_lens = [37000, 64000]
    p_cu = torch.tensor([0] + p_lens).cumsum(0).to(torch.int32)
    pk, pv = ops.pack(raw, r2t.cuda(), p_req.cuda(), p_cu.cuda(), sum(p_lens), max(p_lens), torch.bfloat16)
    wk, wv = attention.pack_qsa(host, r2t.numpy(), p_req.numpy(), p_cu.numpy(), sum(p_lens))
    assert _same_bits(pk, wk) and _same_bits(pv, wv)


def test_valid_counts_and_cumulative_rows():
    gen = torch.Generator().manual_seed(3)
    for batch, topk in ((1, 1), (3, 2048), (1500, 64), (5000, 7)):
        seq = torch.randint(0, 3000, (batch,), dtype=torch.int32, generator=gen)
        idx = torch.randint(-1, 3000, (batch, topk), dtype=torch.int32, generator=gen)
        counts, cu = ops.valid_counts(seq.cuda(), idx.cuda())
        want = ((idx >= 0) & (idx < seq[:, None])).sum(1).to(torch.int32)
        assert torch.equal(counts.cpu(), want)
        assert torch.equal(cu.cpu(), torch.cat([torch.zeros(1, dtype=torch.int32), want.cumsum(0).to(torch.int32)]))


class _Fp8Pool:
    dtype = torch.float8_e4m3fn

    def __init__(self, k8, v8):
        self.k8, self.v8 = k8.view(torch.float8_e4m3fn), v8.view(torch.float8_e4m3fn)

    def get_key_buffer(self, layer_id):
        return self.k8

    def get_value_buffer(self, layer_id):
        return self.v8


def test_paged_attention_on_fp8_pool_through_the_hook():
    """Qwen3.8's shape (24 q / 2 KV heads x 256): the hook gathers the valid top-k rows (sorted, -1 padded) into BF16
    and runs the split-K decode; against the FP64 oracle on the E4M3 values."""
    k8, v8 = _pool(20261030, -2.0, 0.0)     # unit-scale values, where the absolute bounds are meaningful
    k8, v8 = k8[:40000].contiguous(), v8[:40000].contiguous()
    gen = torch.Generator().manual_seed(5)
    reqs, ctx, topk, qh = 5, 8000, 700, 24
    r2t = torch.randperm(40000, generator=gen)[:reqs * ctx].view(reqs, ctx).to(torch.int32)
    seq = torch.full((reqs,), ctx, dtype=torch.int32)
    seq[2] = 300
    idx = torch.full((reqs, topk), -1, dtype=torch.int32)
    for b in range(reqs):
        n = min(topk, int(seq[b])) - (b == 4) * 200
        idx[b, :n] = torch.sort(torch.randperm(int(seq[b]), generator=gen)[:n]).values.to(torch.int32)
    q = (torch.randn(reqs, qh * DIM, generator=gen)).to(torch.bfloat16)
    backend = SimpleNamespace(token_to_kv_pool=_Fp8Pool(k8.cuda(), v8.cuda()),
                              req_to_token_pool=SimpleNamespace(req_to_token=r2t.cuda()),
                              _resolve_metadata=lambda fb: SimpleNamespace(row_req_pool_indices=None,
                                                                          sequence_lengths=seq.cuda()),
                              _expand_block_indices=lambda ti, md: ti)
    layer = SimpleNamespace(layer_id=0, scaling=1 / math.sqrt(DIM))
    fb = SimpleNamespace(req_pool_indices=torch.arange(reqs).cuda())
    out = qsa.paged_attention(None, backend, q.cuda(), layer, fb, idx.cuda())
    assert out.shape == (reqs, qh * DIM)
    kf = nvfp4.e4m3_decode(k8.numpy())
    vf = nvfp4.e4m3_decode(v8.numpy())
    qf = q.float().numpy().reshape(reqs, qh, DIM)
    ref, flash = np.zeros((reqs, qh, DIM)), np.zeros((reqs, qh, DIM))
    for b in range(reqs):
        valid = attention.key_validity(idx[b].numpy(), topk, int(seq[b]))
        sl = r2t[b].numpy()[idx[b].numpy()[valid]]
        ones = np.ones(len(sl), bool)
        ref[b] = attention.softmax_attention(qf[b], kf[sl], vf[sl], ones, layer.scaling)
        flash[b] = attention.flash_precision_attention(qf[b], kf[sl], vf[sl], ones, layer.scaling)
    check(out.view(reqs, qh, DIM), ref, flash)


class _Fa2Scratch:
    """SGLang's _get_fa2_scratch: one BF16 K and V buffer per backend, reallocated only when a request outgrows it."""

    def __init__(self):
        self.k = self.v = None

    def __call__(self, capacity, heads, dim, dtype, device):
        if self.k is None or self.k.shape[0] < capacity:
            self.k = torch.empty(capacity, heads, dim, dtype=dtype, device=device)
            self.v = torch.empty_like(self.k)
        return self.k[:capacity], self.v[:capacity]


def test_paged_attention_on_fp8_pool_graph_replay_equals_eager():
    """Under a CUDA graph the FP8 path takes the metadata's fa2 buffers and asks the scratch for the graph's capacity
    (_cuda_graph_max_tokens * topk), as qsa_fp4.py:250-258 does: a capture of fewer rows than that capacity, replayed
    with new queries and with eager calls of other sizes in between, matches the eager result bit for bit each time."""
    k8, v8 = _pool(20261031, -2.0, 0.0)
    k8, v8 = k8[:40000].contiguous().cuda(), v8[:40000].contiguous().cuda()
    gen = torch.Generator().manual_seed(7)
    reqs, ctx, topk, qh, max_tokens = 4, 6000, 512, 24, 8
    r2t = torch.randperm(40000, generator=gen)[:reqs * ctx].view(reqs, ctx).to(torch.int32).cuda()
    seq = torch.tensor([6000, 5000, 300, 4000], dtype=torch.int32).cuda()
    idx = torch.full((reqs, topk), -1, dtype=torch.int32)
    for b in range(reqs):
        n = min(topk, int(seq[b])) - (b == 3) * 100
        idx[b, :n] = torch.sort(torch.randperm(int(seq[b]), generator=gen)[:n]).values.to(torch.int32)
    idx = idx.cuda()
    graph_md = SimpleNamespace(row_req_pool_indices=None, sequence_lengths=seq, is_cuda_graph=True,
                               fa2_valid_counts=torch.zeros(max_tokens, dtype=torch.int32, device='cuda'),
                               fa2_cu_seqlens_k=torch.zeros(max_tokens + 1, dtype=torch.int32, device='cuda'),
                               fa2_cu_seqlens_q=torch.arange(max_tokens + 1, dtype=torch.int32, device='cuda'))
    eager_md = SimpleNamespace(row_req_pool_indices=None, sequence_lengths=seq, is_cuda_graph=False)
    state = {'md': eager_md}
    scratch = _Fa2Scratch()
    backend = SimpleNamespace(token_to_kv_pool=_Fp8Pool(k8, v8), req_to_token_pool=SimpleNamespace(req_to_token=r2t),
                              _resolve_metadata=lambda fb: state['md'], _expand_block_indices=lambda ti, md: ti,
                              _get_fa2_scratch=scratch, _cuda_graph_max_tokens=max_tokens)
    layer = SimpleNamespace(layer_id=0, scaling=1 / math.sqrt(DIM))
    fb = SimpleNamespace(req_pool_indices=torch.arange(reqs).cuda())
    qs = torch.randn(reqs, qh * DIM, generator=gen).to(torch.bfloat16).cuda()
    qsa.paged_attention(None, backend, qs, layer, fb, idx)      # eager first: workspaces exist before the capture
    state['md'] = graph_md
    qsa.paged_attention(None, backend, qs, layer, fb, idx)      # the graph capacity's scratch, before the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = qsa.paged_attention(None, backend, qs, layer, fb, idx)
    assert scratch.k.shape[0] == max_tokens * topk
    for i in range(3):
        qs.copy_((torch.randn(qs.shape, generator=gen) * (1 + i)).to(torch.bfloat16).cuda())
        graph.replay()
        torch.cuda.synchronize()
        state['md'] = eager_md
        qsa.paged_attention(None, backend, qs[:2], layer, fb, idx[:2])   # an eager call of another size in between
        eager = qsa.paged_attention(None, backend, qs, layer, fb, idx)
        torch.cuda.synchronize()
        state['md'] = graph_md
        assert torch.equal(captured.view(torch.int16), eager.view(torch.int16)), i
