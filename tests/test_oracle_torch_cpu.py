"""The torch CPU restatement (the CPU baseline bench.py times) pinned against the numpy oracle: the dequantization bit
for bit over every byte, the slot lookup and validity rules exactly, and the attention within FP32 rounding, with -1
holes, short rows, a count limit, a causal limit and a row without keys."""
import numpy as np
import torch

from oracle import attention, nvfp4, torch_cpu


def test_dequant_every_byte_bit_exact():
    pay = np.arange(256, dtype=np.uint8).reshape(2, 1, 128)
    sf = (np.arange(32).reshape(2, 1, 16) * 7 % 126).astype(np.uint8)   # scale bytes, no NaN among them
    for g in (1.0, np.float32(0.013671875), np.float32(3.1e-3)):
        got = torch_cpu.dequant(torch.from_numpy(pay), torch.from_numpy(sf.astype(np.uint8)), g).numpy()
        want = nvfp4.dequant(pay, sf.astype(np.uint8), g)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _case(seed=3, b=5, ctx=704, hkv=2, hq=8, d=64, topk=90, page=16):
    rng = np.random.default_rng(seed)
    slots = b * ctx
    x = nvfp4.f32_to_bf16_f32(rng.standard_normal((2, slots, hkv, d)).astype(np.float32))
    kp, ks, gk = nvfp4.nvfp4_encode(x[0])
    vp, vs, gv = nvfp4.nvfp4_encode(x[1])
    pt = rng.permutation(slots // page).reshape(b, ctx // page).astype(np.int32)
    idx = np.stack([np.sort(rng.permutation(ctx)[:topk]) for _ in range(b)]).astype(np.int32)
    idx[1, ::6] = -1
    seq = np.full(b, ctx, np.int32)
    seq[2] = 300
    counts = np.full(b, topk, np.int32)
    counts[3] = 40
    counts[4] = 0
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    return (kp, vp, ks, vs, gk, gv), pt, idx, seq, counts, q


def test_slots_match_the_oracle_rules():
    pool, pt, idx, seq, counts, _ = _case()
    qpos = np.full(len(seq), 650, np.int32)
    got = torch_cpu.slots_of(torch.from_numpy(pt), 16, torch.from_numpy(idx), torch.from_numpy(seq),
                             torch.from_numpy(counts), torch.from_numpy(qpos)).numpy()
    for r in range(len(seq)):
        valid = attention.key_validity(idx[r], counts[r], seq[r], qpos[r])
        want = np.full(idx.shape[1], -1)
        want[valid] = attention.slots_of(pt, r, idx[r][valid], 16)
        assert np.array_equal(got[r], want)


def test_decode_matches_the_oracle():
    pool, pt, idx, seq, counts, q = _case()
    slots = torch_cpu.slots_of(torch.from_numpy(pt), 16, torch.from_numpy(idx), torch.from_numpy(seq),
                               torch.from_numpy(counts))
    tpool = tuple(torch.from_numpy(a) for a in pool[:4]) + pool[4:]
    got = torch_cpu.sparse_decode(torch.from_numpy(q), tpool, slots, 0.125).numpy()
    want = attention.sparse_decode(q, pool, pt, 16, np.arange(len(seq)), idx, counts, seq, 0.125)
    assert not got[4].any()                                   # no valid key
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())
