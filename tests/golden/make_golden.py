"""Writes the golden fixtures of this directory from the CPU oracle (seeded, deterministic):

- nvfp4_encode.npz: BF16 input [64, 2, 128] with per-token magnitudes over five decades (x_bf16 as uint16 bits), and
  its NVFP4 encoding (pay, sc, g) by the rules of xtier/backend/formats.py:114-128;
- decode_small.npz: a 2-request NVFP4 pool (1 KV head, d 128, context 256, page 64, shuffled pages), q for 8 query
  heads, index lists with holes, and the FP64 sparse-attention output and the natural LSE per row and head.

The oracle itself is pinned by the tests of tests/test_oracle_*.py; tests/test_golden.py checks that the oracle
still reproduces these files and the GPU tests compare the kernels with them.

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import attention, nvfp4  # noqa: E402


def encode_case():
    rng = np.random.default_rng(20261023)
    x = rng.standard_normal((64, 2, 128)) * 10.0 ** rng.uniform(-4, 1, (64, 1, 1))
    x[3, 1, 16:32] = 0.0                         # a zero block
    bits = nvfp4.bf16_bits(x.astype(np.float32))
    pay, sc, g = nvfp4.nvfp4_encode(nvfp4.bf16_to_f32(bits))
    return dict(x_bf16=bits, pay=pay, sc=sc, g=np.array([g], np.float32))


def decode_case():
    rng = np.random.default_rng(20261029)
    batch, ctx, page, dim, hq = 2, 256, 64, 128, 8
    slots = batch * ctx
    k = nvfp4.f32_to_bf16_f32(rng.standard_normal((slots, 1, dim)).astype(np.float32))
    v = nvfp4.f32_to_bf16_f32(rng.standard_normal((slots, 1, dim)).astype(np.float32))
    k[:, :, 5] *= 8
    kp, ks, gk = nvfp4.nvfp4_encode(k)
    vp, vs, gv = nvfp4.nvfp4_encode(v)
    pt = rng.permutation(slots // page).reshape(batch, ctx // page).astype(np.int32)
    topk = 96
    idx = np.stack([np.sort(rng.permutation(ctx)[:topk]) for _ in range(batch)]).astype(np.int32)
    idx[1, 10:20] = -1
    seq = np.array([ctx, 200], np.int32)
    q = nvfp4.f32_to_bf16_f32(rng.standard_normal((batch, hq, dim)).astype(np.float32))
    scale = np.float32(1 / np.sqrt(dim))
    pool = (kp, vp, ks, vs, gk, gv)
    out = attention.sparse_decode(q, pool, pt, page, np.arange(batch), idx, None, seq, float(scale))
    lse = np.zeros((batch, hq))
    for r in range(batch):
        valid = attention.key_validity(idx[r], topk, seq[r])
        sl = attention.slots_of(pt, r, idx[r][valid], page)
        kk = nvfp4.dequant(kp[sl], ks[sl], gk)[:, 0].astype(np.float64)
        s = q[r].astype(np.float64) @ kk.T * float(scale)
        lse[r] = s.max(1) + np.log(np.exp(s - s.max(1, keepdims=True)).sum(1))
    return dict(k_pay=kp, v_pay=vp, k_sf=ks, v_sf=vs, gk=np.array([gk], np.float32), gv=np.array([gv], np.float32),
                page_table=pt, indices=idx, seq_lens=seq, q_bf16=nvfp4.bf16_bits(q), scale=np.array([scale]),
                out=out, lse=lse)


def main():
    np.savez_compressed(HERE / 'nvfp4_encode.npz', **encode_case())
    np.savez_compressed(HERE / 'decode_small.npz', **decode_case())
    print('wrote', HERE / 'nvfp4_encode.npz', HERE / 'decode_small.npz')


if __name__ == '__main__':
    main()
