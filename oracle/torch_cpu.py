"""A torch CPU restatement of the NVFP4 sparse decode, batched over requests and heads so that torch's CPU kernels run it
on all the host cores: the CPU baseline that bench.py times beside the GPU. Test infrastructure, not product code; it
follows the same reference lines as ``attention.sparse_decode`` and is pinned against it in
tests/test_oracle_torch_cpu.py.

Steps (reference: qsa_fp4.py:94-101 for the dequantization, :131-140 for the validity rules, qsa_decode.py's FP64
reference form tests/qsa_decode_check.py:14-26 for the attention, here in FP32):
1. slots of the listed positions through the page table (slot = table[pos // P] * P + pos % P);
2. K / V rows of those slots dequantized to (e2m1 * e4m3) * g in FP32;
3. softmax(q . k * scale) v over the valid keys, per query head, in FP32; a row without a valid key gives 0.
"""
import torch

E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def dequant(pay, sf, g):
    """uint8 payload [..., D/2] and E4M3 scale bytes [..., D/16] -> FP32 [..., D]: element 2i from the low nibble of
    byte i, scale j // 16 for element j, (e2m1 * e4m3) * g in this order."""
    p = pay.long()
    vals = torch.stack([E2M1[p & 15], E2M1[p >> 4]], -1).flatten(-2)
    s = sf.view(torch.float8_e4m3fn).float().repeat_interleave(16, -1)
    return (vals * s) * torch.tensor(g, dtype=torch.float32)


def slots_of(table, page_size, indices, seq_lens, counts=None, query_pos=None):
    """int64 slots [B, K] of each row's listed positions (-1: invalid): column < count, 0 <= pos < seq_len and, for a
    causal query, pos <= its position; ``table`` [B, ...] holds page ids (page_size > 1) or slots (page_size 1)."""
    idx = indices.long()
    cols = torch.arange(idx.shape[1])[None, :]
    valid = (idx >= 0) & (idx < seq_lens.long()[:, None])
    if counts is not None:
        valid &= cols < counts.long()[:, None]
    if query_pos is not None:
        valid &= idx <= query_pos.long()[:, None]
    pos = torch.where(valid, idx, torch.zeros_like(idx))
    ent = torch.gather(table.long(), 1, pos // page_size)
    slots = ent * page_size + pos % page_size
    return torch.where(valid, slots, torch.full_like(slots, -1))


def sparse_decode(q, pool, slots, scale):
    """q FP32 [B, Hq, D]; pool = (k_pay, v_pay, k_sf, v_sf, gk, gv) CPU uint8 views [slots, Hkv, D/2 | D/16] and float
    global scales; slots int64 [B, K] (-1: invalid). Returns FP32 [B, Hq, D]."""
    k_pay, v_pay, k_sf, v_sf, gk, gv = pool
    b, hq, d = q.shape
    hkv = k_pay.shape[1]
    valid = slots >= 0
    s = slots.clamp(min=0)
    k = dequant(k_pay[s], k_sf[s], gk)                              # [B, K, Hkv, D]
    v = dequant(v_pay[s], v_sf[s], gv)
    qg = q.reshape(b, hkv, hq // hkv, d)
    scores = torch.matmul(qg, k.permute(0, 2, 3, 1)) * scale        # [B, Hkv, G, K]
    scores = scores.masked_fill(~valid[:, None, None, :], float('-inf'))
    p = torch.softmax(scores, -1).nan_to_num(0.0)                   # a row without valid keys: all -inf -> 0
    out = torch.matmul(p, v.permute(0, 2, 1, 3))                    # [B, Hkv, G, D]
    return out.reshape(b, hq, d)
