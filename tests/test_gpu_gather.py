"""QSA decode gather and prefill packing on the GPU against the oracle, bit for bit, at Qwen3.8's QSA shape (2 KV
heads x 256) and at the decode workload's shape (4 x 128); outputs pre-filled with a NaN canary so stray or missing
writes show (the method of tests/qsa_fp4_check.py:52-66)."""
import numpy as np
import pytest
import torch

from oracle import attention
from tests._pools import random_pool
from xtier_amd import ops

pytestmark = pytest.mark.gpu
CANARY = 0x7FC1


def _requests(rng, slots, batch, topk, width, counts, lens):
    r2t = rng.integers(0, slots, (batch + 1, width)).astype(np.int32)
    req = rng.permutation(batch + 1)[:batch].astype(np.int64)
    seq = np.array(lens, np.int32)
    idx = np.full((batch, topk), -1, np.int32)
    for b, n in enumerate(counts):
        idx[b, :n] = rng.permutation(int(seq[b]))[:n]
    return r2t, req, seq, idx


@pytest.mark.parametrize('heads,dim,slots', [(2, 256, 7000), (4, 128, 9000)])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
def test_gather_compact_and_zero_fill(heads, dim, slots, dtype):
    pool = random_pool(heads * dim + slots, slots, heads, dim)
    rng = np.random.default_rng(20261023)
    batch, topk, width = 3, 2048, 12000
    counts = [2048, 1500, 2000]
    r2t, req, seq, idx = _requests(rng, slots, batch, topk, width, counts, [5000, 3000, 6900])
    idx[1, 10] = 4000          # beyond request 1's length: skipped (compact) / zero (page-aligned)
    idx[2, 3] = -1
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    dev = lambda a: torch.from_numpy(a).cuda()
    for label, cu_, zf in (('compact', cu, 0), ('page-aligned', (np.arange(batch + 1) * 2112).astype(np.int32), 2112)):
        cap = int(cu_[-1]) if not zf else batch * zf
        out_k = torch.full((cap, heads, dim), CANARY, dtype=torch.int16).view(dtype).cuda()
        out_v = out_k.clone()
        ops.gather(pool.raw, dev(r2t), dev(req), dev(idx), dev(seq), dev(cu_), out_k, out_v, batch, topk, zf)
        wk = np.full((cap, heads, dim), CANARY, np.uint16)
        wv = wk.copy()
        if dtype == torch.bfloat16:
            attention.gather_qsa(pool.host, r2t, req, idx, seq, cu_, wk, wv, batch, topk, zf)
        else:   # the same FP32 values rounded to FP16
            _gather_f32(pool.host, r2t, req, idx, seq, cu_, batch, topk, zf, wk, wv)
        assert np.array_equal(out_k.view(torch.int16).cpu().numpy().view(np.uint16), wk), label
        assert np.array_equal(out_v.view(torch.int16).cpu().numpy().view(np.uint16), wv), label


def test_gather_lengths_past_the_table_width():
    """Positions at or past a req_to_token row's pitch are invalid even when seq_lens reaches beyond: the table is a
    contiguous [rows, width] view into a longer buffer of valid slots, so a read past a row would gather real rows."""
    heads, dim, slots = 4, 128, 9000
    pool = random_pool(7, slots, heads, dim)
    rng = np.random.default_rng(5)
    batch, topk, width = 2, 512, 3000
    r2t, req, seq, idx = _requests(rng, slots, batch, topk, width, [512, 512], [5000, 5000])   # positions < 5000
    buf = torch.from_numpy(rng.integers(0, slots, (batch + 1) * width + 4096).astype(np.int32))
    buf[:(batch + 1) * width] = torch.from_numpy(r2t.reshape(-1))
    table = buf.cuda()[:(batch + 1) * width].view(batch + 1, width)
    counts = np.array([512, 512], np.int32)
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    dev = lambda a: torch.from_numpy(a).cuda()
    out_k = torch.full((int(cu[-1]), heads, dim), CANARY, dtype=torch.int16).view(torch.bfloat16).cuda()
    out_v = out_k.clone()
    ops.gather(pool.raw, table, dev(req), dev(idx), dev(seq), dev(cu), out_k, out_v, batch, topk, 0)
    wk = np.full((int(cu[-1]), heads, dim), CANARY, np.uint16)
    wv = wk.copy()
    attention.gather_qsa(pool.host, r2t, req, idx, np.minimum(seq, width), cu, wk, wv, batch, topk, 0)
    assert np.array_equal(out_k.view(torch.int16).cpu().numpy().view(np.uint16), wk)
    assert np.array_equal(out_v.view(torch.int16).cpu().numpy().view(np.uint16), wv)


def _gather_f32(raw, r2t, req, idx, seq, cu, batch, topk, zf, wk, wv):
    """FP16 variant of the oracle gather: the reference rounds the same FP32 values to the output dtype."""
    from oracle import nvfp4
    k_pay, v_pay, k_sf, v_sf, gk, gv = raw
    num = zf if zf else topk
    for b in range(batch):
        for c in range(num):
            pos = idx[b, c] if c < topk else -1
            valid = c < cu[b + 1] - cu[b] and 0 <= pos < seq[b]
            if not valid and not zf:
                continue
            for pay, sf, g, out in ((k_pay, k_sf, gk, wk), (v_pay, v_sf, gv, wv)):
                if valid:
                    s = r2t[req[b], pos]
                    vals = nvfp4.dequant(pay[s], sf[s], g)
                else:
                    vals = np.zeros(out.shape[1:], np.float32)
                out[cu[b] + c] = vals.astype(np.float16).view(np.uint16)


@pytest.mark.parametrize('heads,dim', [(2, 256), (4, 128)])
def test_pack_prefixes(heads, dim):
    slots = 9000
    pool = random_pool(7 + dim, slots, heads, dim)
    rng = np.random.default_rng(1)
    r2t = rng.integers(0, slots, (4, 8000)).astype(np.int32)
    req = np.array([1, 3], np.int64)
    lens = [3700, 6400]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    dev = lambda a: torch.from_numpy(a).cuda()
    pk, pv = ops.pack(pool.raw, dev(r2t), dev(req), dev(cu), sum(lens), max(lens), torch.bfloat16)
    wk, wv = attention.pack_qsa(pool.host, r2t, req, cu, sum(lens))
    assert np.array_equal(pk.view(torch.int16).cpu().numpy().view(np.uint16), wk)
    assert np.array_equal(pv.view(torch.int16).cpu().numpy().view(np.uint16), wv)


def test_gather_rejects_non_power_of_two_head():
    raw = tuple(torch.zeros(16, 2, 48, dtype=torch.uint8, device='cuda') for _ in range(2)) + tuple(
        torch.zeros(16, 2, 6, dtype=torch.uint8, device='cuda') for _ in range(2)) + (
        torch.ones(1, device='cuda'), torch.ones(1, device='cuda'))
    z = torch.zeros(4, dtype=torch.int32, device='cuda')
    with pytest.raises(ValueError, match='power-of-2'):
        ops.gather(raw, z.view(1, 4), z[:1].long(), z.view(1, 4), z[:1], z[:2], torch.empty(4, 2, 96,
                   dtype=torch.bfloat16, device='cuda'), torch.empty(4, 2, 96, dtype=torch.bfloat16, device='cuda'),
                   1, 4)


def test_reference_qwen_case():
    """tests/qsa_fp4_check.py as the reference runs it: a 70000-token pool of 2 KV heads x 256 whose per-token
    magnitudes spread over three decades, quantized with a unit global scale; requests [2, 0, 3] of a random
    req_to_token [4, 120000] with lengths 50000 / 3000 / 69000 and 2048 / 1500 / 2000 valid top-k positions, gathered
    compact and page-aligned (2112 columns, zero-filled); then the prefixes of requests [1, 3] (37000 and 64000
    tokens) packed. Every output bit against the oracle reading the same pool bytes."""
    heads, dim, rows = 2, 256, 70000
    gen = torch.Generator(device='cuda').manual_seed(20261023)
    one = torch.ones(1, dtype=torch.float32, device='cuda')
    raw = []
    for _ in range(2):
        x = torch.randn(rows, heads, dim, generator=gen, device='cuda') * 10 ** (
            torch.rand(rows, 1, 1, generator=gen, device='cuda') * 3 - 2)
        pay = torch.empty(rows, heads, dim // 2, dtype=torch.uint8, device='cuda')
        sf = torch.empty(rows, heads, dim // 16, dtype=torch.uint8, device='cuda')
        ops.quantize_append(x.to(torch.bfloat16), torch.arange(rows, device='cuda'), one, pay, sf)
        raw += [pay, sf]
    raw = (raw[0], raw[2], raw[1], raw[3], one, one)
    host = tuple(t.cpu().numpy() for t in raw[:4]) + (1.0, 1.0)
    batch, topk, width = 3, 2048, 120000
    r2t = torch.randint(0, rows, (4, width), generator=gen, device='cuda', dtype=torch.int32)
    req = torch.tensor([2, 0, 3], dtype=torch.int64, device='cuda')
    seq = torch.tensor([50000, 3000, 69000], dtype=torch.int32, device='cuda')
    idx = torch.full((batch, topk), -1, dtype=torch.int32, device='cuda')
    counts = (2048, 1500, 2000)
    for b, n in enumerate(counts):
        idx[b, :n] = torch.randperm(int(seq[b]), generator=gen, device='cuda')[:n].to(torch.int32)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32, device='cuda')
    h = lambda t: t.cpu().numpy()
    for label, cu, zf in (('compact', cu_k, 0),
                          ('page-aligned', torch.arange(batch + 1, dtype=torch.int32, device='cuda') * 2112, 2112)):
        cap = int(cu[-1]) if not zf else batch * zf
        out_k = torch.full((cap, heads, dim), CANARY, dtype=torch.int16, device='cuda').view(torch.bfloat16)
        out_v = out_k.clone()
        ops.gather(raw, r2t, req, idx, seq, cu, out_k, out_v, batch, topk, zf)
        wk = np.full((cap, heads, dim), CANARY, np.uint16)
        wv = wk.copy()
        attention.gather_qsa(host, h(r2t), h(req), h(idx), h(seq), h(cu), wk, wv, batch, topk, zf)
        assert np.array_equal(out_k.view(torch.int16).cpu().numpy().view(np.uint16), wk), label
        assert np.array_equal(out_v.view(torch.int16).cpu().numpy().view(np.uint16), wv), label
    p_req = torch.tensor([1, 3], dtype=torch.int64, device='cuda')
    p_lens = [37000, 64000]
    p_cu = torch.tensor(np.concatenate([[0], np.cumsum(p_lens)]), dtype=torch.int32, device='cuda')
    pk, pv = ops.pack(raw, r2t, p_req, p_cu, sum(p_lens), max(p_lens), torch.bfloat16)
    wk, wv = attention.pack_qsa(host, h(r2t), h(p_req), h(p_cu), sum(p_lens))
    assert np.array_equal(pk.view(torch.int16).cpu().numpy().view(np.uint16), wk)
    assert np.array_equal(pv.view(torch.int16).cpu().numpy().view(np.uint16), wv)
