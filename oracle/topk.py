"""CPU oracle of the top-k producers (test infrastructure, not product code): the indexer logits that pick each
query's keys and the selection of the top-k, restated in numpy from the reference.

- ``qsa_indexer_logits``: xtier/packs/qwen4_exp/qsa_prefill.py:59-69 (per key and query row, the head sum of
  ReLU(q . k) over one tile GEMM in FP32), :100 (division by score_scale, default sqrt(head_dim)) and the mask
  described at :8-9 (every column outside [start, end) is -inf).
- ``dsa_mqa_logits``: xtier/packs/glm5_next/indexer_torch.py:28-45 (sum over heads of w[q, h] ReLU(q_h . k) times the
  key's scale; outside [ks, ke) 0, or -inf when clean_logits; the row stride padded to a multiple of 4).
- ``dsa_paged_mqa_logits``: indexer_torch.py:48-72 (the cache page layout: block x head_dim FP8 values, then block
  FP32 scales; positions at or past the context length 0 / -inf; padded to max_seq_len).
- ``minimax_block_scores_decode`` / ``minimax_block_scores_prefill``: xtier/packs/minimax_m3/kv_fp4.py:168-222 and
  :407-446 (the NVFP4 index key dequantized to BF16, per block of block_size positions the maximum, or log-sum-exp,
  of the scaled scores; decode forces the first init_blocks to 1e30 and the last local_blocks to 1e29).
- ``topk_rows``: the selection the attention kernels consume: per row the positions of the topk largest finite
  values, ascending, ties toward the lower position, -1 padded (the int32 [batch, topk] format of the index lists).

The products are formed and summed in float64 here; the GPU forms exact products (BF16 x BF16, FP8 x FP8 in FP32)
and sums them in FP32, so the tests compare with a bound on FP32 summation error.
"""
import math

import numpy as np

from . import nvfp4


def qsa_indexer_logits(q, k, starts, ends, score_scale=None):
    """q [rows, heads, dim] and k [keys, dim] as float arrays (the BF16 values), starts / ends [rows] -> float64
    logits [rows, keys]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    rows, heads, dim = q.shape
    scale = score_scale or math.sqrt(dim)
    logits = np.zeros((rows, k.shape[0]))
    for h in range(heads):                      # one head's [rows, keys] products at a time
        logits += np.maximum(q[:, h] @ k.T, 0.0)
    logits /= scale
    cols = np.arange(k.shape[0])[None, :]
    keep = (cols >= np.asarray(starts)[:, None]) & (cols < np.asarray(ends)[:, None])
    return np.where(keep, logits, -np.inf)


def dsa_mqa_logits(q, k, k_scale, weights, ks, ke, clean_logits=False):
    """q [num_q, heads, dim], k [num_kv, dim] (the FP8 values as floats), k_scale [num_kv], weights [num_q, heads],
    ks / ke [num_q] -> float64 logits [num_q, num_kv]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    s = np.maximum(np.einsum('qhd,nd->qhn', q, k), 0.0)
    logits = (s * np.asarray(weights, np.float64)[:, :, None]).sum(1) * np.asarray(k_scale, np.float64)[None, :]
    pos = np.arange(k.shape[0])[None, :]
    keep = (pos >= np.asarray(ks)[:, None]) & (pos < np.asarray(ke)[:, None])
    return np.where(keep, logits, -np.inf if clean_logits else 0.0)


def dsa_paged_keys(kvcache, block_table, head_dim):
    """The paged FP8 cache (uint8 [pages, block * (head_dim + 4)]: block x head_dim E4M3 values, then block FP32
    scales) read through block_table [batch, n] -> (values [batch, n * block, head_dim], scales [batch, n * block])."""
    cache = np.asarray(kvcache, np.uint8)
    pages = cache.shape[0]
    block = cache.shape[1] // (head_dim + 4)
    flat = cache.reshape(pages, block * (head_dim + 4))
    rows = flat[np.maximum(np.asarray(block_table), 0)]
    vals = nvfp4.e4m3_decode(rows[..., :block * head_dim]).reshape(rows.shape[0], -1, head_dim)
    scales = rows[..., block * head_dim:].copy().view(np.float32).reshape(rows.shape[0], -1)
    return vals.astype(np.float64), scales.astype(np.float64)


def dsa_paged_mqa_logits(q, kvcache, weights, context_lens, block_table, max_seq_len, clean_logits=False):
    """q [batch, heads, dim] (next_n = 1, FP8 values as floats) over the paged cache -> float64 [batch, max_seq_len]."""
    q = np.asarray(q, np.float64)
    batch, heads, dim = q.shape
    vals, scales = dsa_paged_keys(kvcache, block_table, dim)
    s = np.maximum(np.einsum('bhd,btd->bht', q, vals), 0.0)
    logits = (s * np.asarray(weights, np.float64)[:, :, None]).sum(1) * scales
    fill = -np.inf if clean_logits else 0.0
    pos = np.arange(logits.shape[1])[None, :]
    logits = np.where(pos >= np.asarray(context_lens)[:, None], fill, logits)
    out = np.full((batch, max_seq_len), fill)
    n = min(max_seq_len, logits.shape[1])
    out[:, :n] = logits[:, :n]
    return out


def _index_keys(pay, sf, slots):
    """NVFP4 index-key rows of the given slots (pay [pages, 128, d/2], sf [pages, 128, d/16]) as float64 [n, d]; slots
    wrap modulo the pool's slot count, as (slot + max_slots) % max_slots does (kv_fp4.py:190, :209, :437)."""
    pay = np.asarray(pay, np.uint8).reshape(-1, pay.shape[-1])
    sf = np.asarray(sf, np.uint8).reshape(-1, sf.shape[-1])
    slots = (np.asarray(slots, np.int64) + len(pay)) % len(pay)
    return nvfp4.dequant(pay[slots], sf[slots], 1.0).astype(np.float64)


def _score_scale(sm_scale, k_scale):
    """The FP32 factor of the scores: (sm_scale * 1.4426950409) * k_scale, as the kernels form it (kv_fp4.py:181,
    :208; :417, :441)."""
    return float(np.float32(np.float32(sm_scale) * np.float32(1.4426950409)) * np.float32(k_scale))


def minimax_block_scores_decode(q, pay, sf, req_to_token, slot_ids, seq_lens, block_size, sm_scale, k_scale,
                                init_blocks, local_blocks, score_type='max', topk=None):
    """q [batch, heads, d] -> float64 scores [heads, batch, max_blocks] (log2 domain; unused entries nan). With
    ``topk`` (SKIP_TRIVIAL_TOPK_SCORE, kv_fp4.py:186-188) a request with at most topk blocks gets no scores."""
    q = np.asarray(q, np.float64)
    batch, heads, d = q.shape
    max_blocks = int(max(-(-int(s) // block_size) for s in seq_lens)) if batch else 0
    out = np.full((heads, batch, max_blocks), np.nan)
    c = _score_scale(sm_scale, k_scale)
    r2t = np.asarray(req_to_token)
    slots = len(np.asarray(pay).reshape(-1, pay.shape[-1]))
    for b in range(batch):
        n = int(seq_lens[b])
        nb = -(-n // block_size)
        if topk is not None and nb <= topk:
            continue
        toks = r2t[(int(slot_ids[b]) + slots) % slots, :n]
        keys = _index_keys(pay, sf, toks)
        sc = q[b] @ keys.T * c                                   # [heads, n]
        local_start = max(0, nb - local_blocks)
        for blk in range(nb):
            seg = sc[:, blk * block_size:min(n, (blk + 1) * block_size)]
            m = seg.max(1)
            val = m if score_type == 'max' else m + np.log2(np.exp2(seg - m[:, None]).sum(1))
            val = np.where(np.isnan(val), -np.inf, val)
            if local_start <= blk < nb:
                val = np.full(heads, 1e29)
            elif blk < init_blocks:
                val = np.full(heads, 1e30)
            out[:, b, blk] = val
    return out


def minimax_block_scores_prefill(q, pay, sf, req_to_token, slot_ids, cu_seqlens, seq_lens, prefix_lens, block_size,
                                 sm_scale, k_scale, block_q=64):
    """q [total_q, heads, d] -> float64 scores [heads, total_q, max_blocks] (causal; -inf for blocks past a query's
    position within its block_q tile's range, nan outside the tile's range)."""
    q = np.asarray(q, np.float64)
    total, heads, d = q.shape
    c = _score_scale(sm_scale, k_scale)
    max_blocks = int(max(-(-int(s) // block_size) for s in seq_lens))
    out = np.full((heads, total, max_blocks), np.nan)
    slots = len(np.asarray(pay).reshape(-1, pay.shape[-1]))
    for b in range(len(seq_lens)):
        s0, s1 = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        n, pre = int(seq_lens[b]), int(prefix_lens[b])
        toks = np.asarray(req_to_token)[(int(slot_ids[b]) + slots) % slots, :n]
        keys = _index_keys(pay, sf, toks)
        for t in range(s1 - s0):
            tile = t // block_q
            hi = min(n, pre + (tile + 1) * block_q)
            sc = q[s0 + t] @ keys[:hi].T * c                   # [heads, hi]
            pos = np.arange(hi)
            sc = np.where(pos[None, :] <= pre + t, sc, -np.inf)
            for blk in range(-(-hi // block_size)):
                out[:, s0 + t, blk] = sc[:, blk * block_size:(blk + 1) * block_size].max(1)
    return out


def topk_rows(x, topk):
    """float32 [rows, cols] -> int32 [rows, topk]: the positions of the topk largest finite values per row, ascending,
    ties toward the lower position, -1 padded."""
    x = np.asarray(x, np.float32)
    rows, cols = x.shape
    out = np.full((rows, topk), -1, np.int32)
    for r in range(rows):
        fin = np.flatnonzero(np.isfinite(x[r]))
        if not len(fin):
            continue
        order = fin[np.lexsort((fin, -x[r, fin].astype(np.float64)))]   # value descending, then position ascending
        pick = np.sort(order[:topk])
        out[r, :len(pick)] = pick
    return out
