"""Independent pins for three oracle functions that the GPU parity tests lean on: the QSA prefix pack, the flash-kernel
precision reference, and the log-sum-exp of the block-sparse decode. Each is checked against a separate torch
implementation and against a closed form that a plausible slip (swapped nibbles, P kept in FP32, LSE in log2, a
dropped kv_scale) would fail."""
import numpy as np
import torch

from oracle import attention, nvfp4

E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def torch_dequant(pay, sf, g):
    """(e2m1 * e4m3) * g in FP32 with torch's own float8_e4m3fn: element 2i is the low nibble of byte i
    (qsa_fp4.py:94-101), scale j // 16 for element j."""
    p = torch.from_numpy(np.ascontiguousarray(pay)).long()
    vals = torch.stack([E2M1[p & 15], E2M1[p >> 4]], -1).flatten(-2)
    s = torch.from_numpy(np.ascontiguousarray(sf)).view(torch.float8_e4m3fn).float()
    return (vals * s.repeat_interleave(16, -1)) * torch.tensor(g, dtype=torch.float32)


def _pool(rng, slots, heads, dim):
    x = nvfp4.f32_to_bf16_f32((rng.standard_normal((slots, heads, dim)) *
                               np.exp(rng.uniform(-4, 3, (slots, 1, 1)))).astype(np.float32))
    return nvfp4.nvfp4_encode(x)


# --- pack_qsa ------------------------------------------------------------------------------------------------------

def test_pack_equals_whole_pool_dequant_then_index():
    """qsa_fp4.py:146-162: every row of a request's prefix is the pool row dequantized in BF16 (the property of
    tests/qsa_fp4_check.py: reading the packed pool equals SGLang's dequantized pool, gathered)."""
    rng = np.random.default_rng(11)
    slots, heads, dim = 700, 2, 64
    kp, ks, gk = _pool(rng, slots, heads, dim)
    vp, vs, gv = _pool(rng, slots, heads, dim)
    raw = (kp, vp, ks, vs, gk, gv)
    kfull = torch_dequant(kp, ks, gk).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    vfull = torch_dequant(vp, vs, gv).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    r2t = np.stack([rng.permutation(slots)[:400] for _ in range(3)]).astype(np.int32)
    req = np.array([2, 0, 1])
    lens = [400, 1, 257]
    cu = np.concatenate([[0], np.cumsum(lens)])
    out_k, out_v = attention.pack_qsa(raw, r2t, req, cu, int(cu[-1]))
    for b, n in enumerate(lens):
        sl = r2t[req[b], :n]
        assert np.array_equal(out_k[cu[b]:cu[b + 1]], kfull[sl])
        assert np.array_equal(out_v[cu[b]:cu[b + 1]], vfull[sl])


def test_pack_equals_gather_with_every_position_listed():
    """A pack of request b's first n positions is the decode gather of indices 0..n-1 with count n."""
    rng = np.random.default_rng(12)
    slots, heads, dim = 300, 4, 32
    kp, ks, gk = _pool(rng, slots, heads, dim)
    vp, vs, gv = _pool(rng, slots, heads, dim)
    raw = (kp, vp, ks, vs, gk, gv)
    r2t = np.stack([rng.permutation(slots)[:120] for _ in range(2)]).astype(np.int32)
    req = np.array([1, 0])
    lens = np.array([120, 45])
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pk, pv = attention.pack_qsa(raw, r2t, req, cu, int(cu[-1]))
    topk = 120
    idx = np.full((2, topk), -1, np.int32)
    for b, n in enumerate(lens):
        idx[b, :n] = np.arange(n)
    gk_, gv_ = np.zeros_like(pk), np.zeros_like(pv)
    attention.gather_qsa(raw, r2t, req, idx, lens.astype(np.int32), cu, gk_, gv_, 2, topk)
    assert np.array_equal(pk, gk_) and np.array_equal(pv, gv_)


def test_pack_nibble_order_is_pinned():
    """Byte 0x21 of a head row holds element 0 = code 1 (0.5) and element 1 = code 2 (1.0): swapping nibbles fails."""
    pay = np.zeros((1, 1, 16), np.uint8)
    pay[0, 0, 0] = 0x21
    sf = np.full((1, 1, 2), 0x38, np.uint8)   # E4M3 1.0
    raw = (pay, pay, sf, sf, np.float32(1.0), np.float32(1.0))
    out_k, _ = attention.pack_qsa(raw, np.zeros((1, 1), np.int32), np.array([0]), np.array([0, 1]), 1)
    vals = nvfp4.bf16_to_f32(out_k[0, 0])
    assert vals[0] == 0.5 and vals[1] == 1.0 and not vals[2:].any()


# --- flash_precision_attention -------------------------------------------------------------------------------------

def torch_flash(q, k, v, scale):
    """tests/qsa_decode_check.py:29-45 in torch: FP32 scores, P = exp(s - max) rounded to BF16 for the PV product,
    FP32 sum of the unrounded P, output rounded to BF16."""
    hq, group = q.shape[0], q.shape[0] // k.shape[1]
    qf, kf, vf = (torch.from_numpy(np.asarray(t, np.float32)) for t in (q, k, v))
    out = torch.zeros(hq, v.shape[-1], dtype=torch.float64)
    for h in range(hq):
        s = (kf[:, h // group] @ qf[h]) * scale
        p = torch.exp(s - s.max())
        o = (p.to(torch.bfloat16).float() @ vf[:, h // group]) / p.sum()
        out[h] = o.to(torch.bfloat16).double()
    return out.numpy()


def test_flash_precision_matches_torch():
    rng = np.random.default_rng(13)
    for n, hq, hkv, dim in ((1, 4, 1, 32), (33, 8, 2, 64), (700, 24, 2, 256)):
        q = (rng.standard_normal((hq, dim)) * 2).astype(np.float32)
        k = (rng.standard_normal((n, hkv, dim)) * 2).astype(np.float32)
        v = rng.standard_normal((n, hkv, dim)).astype(np.float32)
        got = attention.flash_precision_attention(q, k, v, np.ones(n, bool), dim ** -0.5)
        want = torch_flash(q, k, v, dim ** -0.5)
        # FP32 summation order may move a value across one BF16 rounding boundary, or, where the PV sum cancels to a
        # small value, by the FP32 rounding of its terms (n * 2^-24 of the largest); no further
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
        assert np.all(np.abs(got - want) <= ulp + n * 2.0 ** -24 * np.abs(v).max())
        assert np.mean(got == want) > 0.99


def _bf16(x):
    return np.float32(nvfp4.f32_to_bf16_f32(np.array([x], np.float32))[0])


def test_flash_precision_rounds_p_to_bf16_known_answer():
    """Two keys with scores 0 and ln(y), y = 0.5 + 0.75 * 2^-8: P = (1, p1) with p1 = exp(ln y) in FP32, which BF16
    rounds up by 0.75 of its step. With V rows (0, 1) the output is bf16(p1) / (1 + p1), rounded to BF16: 0.3359375.
    Keeping P in FP32 gives p1 / (1 + p1) -> 0.33398438, and skipping the output rounding gives neither."""
    y = 0.5 + 0.75 * 2.0 ** -8
    q = np.array([[1.0]], np.float32)
    k = np.array([[[0.0]], [[np.log(y)]]], np.float32)
    v = np.array([[[0.0]], [[1.0]]], np.float32)
    got = attention.flash_precision_attention(q, k, v, np.ones(2, bool), 1.0)[0, 0]
    p1 = np.exp(np.float32(k[1, 0, 0]))     # FP32 exp of the FP32 score, as the reference computes it
    denom = np.float32(1.0) + p1
    want, wrong = _bf16(_bf16(p1) / denom), _bf16(p1 / denom)
    assert (want, wrong) == (np.float32(0.3359375), np.float32(0.33398438))
    assert got == want and np.float32(_bf16(p1) / denom) != want


# --- block_sparse_decode LSE ---------------------------------------------------------------------------------------

def test_block_decode_lse_is_torch_logsumexp_of_the_expanded_keys():
    """kv_fp4.py:101-116: the LSE of each (row, head) is the natural log-sum-exp of scale * kv_scale * q.k over the
    positions its blocks expand to (clipped at the row's length). Checked with torch.logsumexp on keys dequantized by
    torch; log2-domain or unscaled LSEs fail."""
    rng = np.random.default_rng(14)
    pages, kh, block, d, b, group = 12, 2, 16, 64, 3, 4
    x = nvfp4.f32_to_bf16_f32(rng.standard_normal((pages * kh * block, d)).astype(np.float32))
    pay, sf, g = nvfp4.nvfp4_encode(x)     # the pages carry no global scale: fold g into the softmax scale
    k_pay = pay.reshape(pages, kh, block, d // 2)
    k_sf = sf.reshape(pages, kh, block, d // 16)
    v_pay, v_sf = k_pay[::-1].copy(), k_sf[::-1].copy()
    ctx = 5 * block
    r2t = np.stack([rng.permutation(pages)[:5].repeat(block) * block + np.tile(np.arange(block), 5)
                    for _ in range(b)]).astype(np.int32)
    ids = np.full((kh, b, 4), -1, np.int32)
    for h in range(kh):
        for r in range(b):
            n = rng.integers(1, 5)
            ids[h, r, :n] = rng.permutation(5)[:n]
    seq = np.array([ctx, ctx - 7, 2 * block + 3], np.int32)
    q = rng.standard_normal((b, kh * group, d))
    scale, kv_scale = 0.3 * float(g), 0.7
    _, lse = attention.block_sparse_decode(q, k_pay, k_sf, v_pay, v_sf, r2t, np.arange(b), ids, seq, block, scale,
                                           kv_scale)
    for r in range(b):
        for h in range(kh):
            pos = np.concatenate([np.arange(e * block, (e + 1) * block) for e in ids[h, r] if e >= 0])
            pos = pos[pos < seq[r]]
            if pos.size == 0:
                assert np.all(np.isneginf(lse[r, h * group:(h + 1) * group]))
                continue
            slot = r2t[r, pos // block * block].astype(np.int64) + pos % block
            kk = torch_dequant(k_pay[slot // block, h, slot % block], k_sf[slot // block, h, slot % block], 1.0)
            s = kk.double() @ torch.from_numpy(q[r, h * group:(h + 1) * group]).T * (scale * kv_scale)
            want = torch.logsumexp(s, 0).numpy()
            np.testing.assert_allclose(lse[r, h * group:(h + 1) * group], want, rtol=0, atol=1e-10)
    fin = lse[np.isfinite(lse)]
    assert fin.size and np.all(np.abs(fin) < 50)   # the scores are not saturated: the log of the sum matters


# --- FP8 pools ------------------------------------------------------------------------------------------------------

def test_fp8_gather_and_pack_equal_torch_decode_then_index():
    """qsa_fp4.py:104-116: on an FP8 pool every value is its E4M3 value; checked against torch's float8_e4m3fn ->
    bfloat16 of the whole pool, then indexed (NaN bytes compared as NaN, as tests/qsa_fp8_check.py compares them)."""
    rng = np.random.default_rng(15)
    slots, heads, dim = 400, 2, 64
    k8 = rng.integers(0, 256, (slots, heads, dim), dtype=np.uint8)
    v8 = rng.integers(0, 256, (slots, heads, dim), dtype=np.uint8)
    raw = (k8, v8, None, None, None, None)
    full = lambda a: torch.from_numpy(a).view(torch.float8_e4m3fn).to(torch.bfloat16).float().numpy()
    kf, vf = full(k8), full(v8)
    r2t = np.stack([rng.permutation(slots)[:300] for _ in range(2)]).astype(np.int32)
    req, lens = np.array([1, 0]), [300, 77]
    cu = np.concatenate([[0], np.cumsum(lens)])
    pk, pv = attention.pack_qsa(raw, r2t, req, cu, int(cu[-1]))
    for b, n in enumerate(lens):
        sl = r2t[req[b], :n]
        np.testing.assert_array_equal(nvfp4.bf16_to_f32(pk[cu[b]:cu[b + 1]]), kf[sl])
        np.testing.assert_array_equal(nvfp4.bf16_to_f32(pv[cu[b]:cu[b + 1]]), vf[sl])
    idx = np.full((2, 80), -1, np.int32)
    idx[0, :60] = rng.permutation(300)[:60]
    idx[1, :50] = rng.permutation(77)[:50]
    seq = np.array([300, 40], np.int32)
    cnt = [60, int((idx[1, :50] < 40).sum())]
    idx[1, :50] = np.concatenate([np.sort(idx[1, :50][idx[1, :50] < 40]), np.sort(idx[1, :50][idx[1, :50] >= 40])])
    cu2 = np.array([0, 60, 60 + cnt[1]])
    gk_ = np.zeros((cu2[-1], heads, dim), np.uint16)
    gv_ = gk_.copy()
    attention.gather_qsa(raw, r2t, req, idx, seq, cu2, gk_, gv_, 2, 80)
    for b in range(2):
        sl = r2t[req[b], idx[b, :cnt[b]]]
        np.testing.assert_array_equal(nvfp4.bf16_to_f32(gk_[cu2[b]:cu2[b + 1]]), kf[sl])
        np.testing.assert_array_equal(nvfp4.bf16_to_f32(gv_[cu2[b]:cu2[b + 1]]), vf[sl])
