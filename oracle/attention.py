"""Sparse attention over an NVFP4 paged KV pool, on the CPU (numpy): the oracle for the gather, the fused decode,
the split-K merge, the chunked prefill, the block-sparse decode and prefill over head-major pages, the BF16 context
copy of such pages and sparse MLA.

Test infrastructure only. Conventions (reference: qsa_fp4.py:131-140; sparse_mla.py:42-46; qsa_decode.py:75, :83):
an index is valid when it is >= 0 and below the row's length (and, for a causal query, not after the query's own
position); invalid entries are masked before any load; a row without a valid key writes 0 (LSE -inf).
"""
import numpy as np

from . import nvfp4

LOG2E = 1.4426950408889634


# --- slot lookup ---------------------------------------------------------------------------------------------------

def slots_of(table, table_row, positions, page_size):
    """Pool slots of token positions of one request. page_size 1: ``table`` is token-granular (req_to_token,
    qsa_fp4.py:135); page_size P > 1: ``table`` holds page ids and slot = table[pos // P] * P + pos % P."""
    positions = np.asarray(positions, dtype=np.int64)
    row = np.asarray(table)[table_row]
    if page_size == 1:
        return row[positions].astype(np.int64)
    return row[positions // page_size].astype(np.int64) * page_size + positions % page_size


# --- QSA gather / pack (bit-exact BF16 rows) --------------------------------------------------------------------------

def gather_qsa(raw, req_to_token, req_indices, indices, seq_lens, cu_k, out_k, out_v, batch, topk, zero_fill_cols=0):
    """qsa_fp4.py:119-143 and :174-180 in numpy. raw = (k_pay u8 [m, H, D/2], v_pay, k_sf u8 [m, H, D/16], v_sf,
    gk, gv), or an FP8 pool's (k u8 [m, H, D], v, None, None, None, None); out_k/out_v are uint16 arrays of BF16 bits
    [rows, H, D], written in place where the reference stores.
    Rows are (e2m1 * e4m3) * g in FP32 rounded to BF16; zero-fill mode writes zeros for the invalid columns below
    zero_fill_cols."""
    k_pay, v_pay, k_sf, v_sf, gk, gv = raw
    heads = k_pay.shape[1]
    rows_of = _row_reader(raw)
    num_cols = zero_fill_cols if zero_fill_cols > 0 else topk
    span = -(-num_cols // 16) * 16
    indices = np.asarray(indices)
    for b in range(batch):
        length = int(seq_lens[b])
        req = int(req_indices[b])
        start = int(cu_k[b])
        valid_count = int(cu_k[b + 1]) - start
        cols = np.arange(span)
        pos = np.where(cols < topk, indices[b, np.minimum(cols, topk - 1)], -1).astype(np.int64)
        valid = (cols < valid_count) & (pos >= 0) & (pos < length)
        store = (cols < zero_fill_cols) if zero_fill_cols > 0 else valid
        slots = np.where(valid, np.asarray(req_to_token)[req, np.where(valid, pos, 0)], 0).astype(np.int64)
        for side, out in ((0, out_k), (1, out_v)):
            rows = rows_of(side, slots)
            rows[~valid] = 0
            dst = start + cols[store]
            out[dst] = rows[store]
    return out_k, out_v


def _row_reader(raw):
    """rows(side, slots) -> BF16 bits [n, H, D] of K (side 0) or V (side 1) at pool slots: NVFP4 (e2m1 * e4m3) * g
    (qsa_fp4.py:94-101), or, for an FP8 pool (raw = (k, v, None, None, None, None)), the E4M3 value of each byte
    (qsa_fp4.py:104-116), NaN bytes giving the quiet NaN 0x7FC0."""
    k_pay, v_pay, k_sf, v_sf, gk, gv = raw
    if k_sf is None:
        def rows(side, slots):
            vals = nvfp4.e4m3_decode((k_pay, v_pay)[side][slots])
            bits = nvfp4.bf16_bits(vals)
            bits[np.isnan(vals)] = 0x7FC0
            return bits
        return rows
    return lambda side, slots: nvfp4.bf16_bits(nvfp4.dequant(((k_pay, v_pay)[side])[slots],
                                                             ((k_sf, v_sf)[side])[slots], (gk, gv)[side]))


def pack_qsa(raw, req_to_token, req_indices, cu_k, total_k, heads_dim=None):
    """qsa_fp4.py:146-162 and :183-192: request b's first cu_k[b+1]-cu_k[b] positions, in order, as BF16 bits rows
    [total_k, H, D] (rows not covered stay 0 here; the reference leaves them unwritten); NVFP4 or FP8 pools."""
    k_pay = raw[0]
    heads = k_pay.shape[1]
    dim = k_pay.shape[2] if raw[2] is None else k_pay.shape[2] * 2
    rows_of = _row_reader(raw)
    out_k = np.zeros((total_k, heads, dim), dtype=np.uint16)
    out_v = np.zeros_like(out_k)
    for b in range(len(req_indices)):
        start, end = int(cu_k[b]), int(cu_k[b + 1])
        slots = np.asarray(req_to_token)[int(req_indices[b]), :end - start].astype(np.int64)
        out_k[start:end] = rows_of(0, slots)
        out_v[start:end] = rows_of(1, slots)
    return out_k, out_v


# --- attention references -----------------------------------------------------------------------------------------

def softmax_attention(q, k, v, valid, scale, dtype=np.float64):
    """One query row: q [Hq, D]; k, v [N, Hkv, Dk|Dv]; valid [N] bool. Softmax over the valid keys in ``dtype``
    (the FP64 reference of tests/qsa_decode_check.py:14-26 in closed form); a row without valid keys gives 0."""
    hq = q.shape[0]
    hkv = k.shape[1]
    group = hq // hkv
    out = np.zeros((hq, v.shape[-1]), dtype=dtype)
    idx = np.nonzero(np.asarray(valid))[0]
    if idx.size == 0:
        return out
    kd = np.asarray(k, dtype=dtype)[idx]
    vd = np.asarray(v, dtype=dtype)[idx]
    qd = np.asarray(q, dtype=dtype)
    for h in range(hq):
        s = kd[:, h // group] @ qd[h] * dtype(scale)
        p = np.exp(s - s.max())
        out[h] = (p @ vd[:, h // group]) / p.sum()
    return out


def flash_precision_attention(q, k, v, valid, scale):
    """The flash kernels' precision (tests/qsa_decode_check.py:29-45): FP32 scores, P rounded to BF16 for the PV
    product, FP32 sums, the output rounded to BF16; returned as float64."""
    hq = q.shape[0]
    group = hq // k.shape[1]
    out = np.zeros((hq, v.shape[-1]), dtype=np.float64)
    idx = np.nonzero(np.asarray(valid))[0]
    if idx.size == 0:
        return out
    kf = np.asarray(k, np.float32)[idx]
    vf = np.asarray(v, np.float32)[idx]
    qf = np.asarray(q, np.float32)
    for h in range(hq):
        s = (kf[:, h // group] @ qf[h]) * np.float32(scale)
        p = np.exp(s - s.max()).astype(np.float32)
        o = (nvfp4.f32_to_bf16_f32(p) @ vf[:, h // group]) / p.sum(dtype=np.float32)
        out[h] = nvfp4.f32_to_bf16_f32(o.astype(np.float32))
    return out


def key_validity(indices, count, length, query_pos=None):
    """valid[c] for one row's index list: c < count, 0 <= idx < length, and idx <= query_pos when causal."""
    indices = np.asarray(indices, dtype=np.int64)
    cols = np.arange(indices.shape[0])
    valid = (cols < count) & (indices >= 0) & (indices < length)
    if query_pos is not None:
        valid &= indices <= query_pos
    return valid


def gather_dequant(pay, sf, g, slots, valid):
    """FP32 (e2m1 * e4m3) * g rows of ``slots`` (invalid ones 0)."""
    slots = np.where(valid, slots, 0)
    rows = nvfp4.dequant(pay[slots], sf[slots], g)
    rows[~valid] = 0.0
    return rows


def sparse_decode(q, pool, table, page_size, rows, indices, counts, seq_lens, scale, query_pos=None,
                  dtype=np.float64):
    """Fused NVFP4 sparse GQA decode/prefill, reference values: for query row r (q [R, Hq, D]) of request rows[r],
    keys = the valid entries of indices[r] (token positions) resolved through the page table, K and V dequantized
    to FP32 (e2m1 * e4m3) * g, softmax(q.k * scale) v computed in ``dtype``. pool = (k_pay, v_pay, k_sf, v_sf, gk,
    gv) in the [slots, Hkv, D/2] / [slots, Hkv, D/16] layout. Returns float [R, Hq, D]."""
    k_pay, v_pay, k_sf, v_sf, gk, gv = pool
    q = np.asarray(q)
    out = np.zeros(q.shape, dtype=dtype)
    for r in range(q.shape[0]):
        idx = np.asarray(indices[r], dtype=np.int64)
        qp = None if query_pos is None else int(query_pos[r])
        valid = key_validity(idx, int(counts[r]) if counts is not None else idx.shape[0], int(seq_lens[r]), qp)
        slots = np.zeros(idx.shape[0], dtype=np.int64)
        if valid.any():
            slots[valid] = slots_of(table, int(rows[r]), idx[valid], page_size)
        k = gather_dequant(k_pay, k_sf, gk, slots, valid)
        v = gather_dequant(v_pay, v_sf, gv, slots, valid)
        out[r] = softmax_attention(q[r], k, v, valid, scale, dtype)
    return out


def split_partials(q, k, v, valid, scale, keys_per_split):
    """Split-K partials of one row in the form of qsa_decode.py:25-60: per split the running max m (log2 domain),
    the sum l and the unnormalized accumulator acc (FP64 here). Returns m [S, Hq], l [S, Hq], acc [S, Hq, Dv]."""
    n = k.shape[0]
    splits = max(1, -(-n // keys_per_split))
    hq = q.shape[0]
    group = hq // k.shape[1]
    m = np.full((splits, hq), -np.inf)
    l = np.zeros((splits, hq))
    acc = np.zeros((splits, hq, v.shape[-1]))
    for s in range(splits):
        sel = np.arange(s * keys_per_split, min(n, (s + 1) * keys_per_split))
        sel = sel[np.asarray(valid)[sel]]
        if sel.size == 0:
            continue
        for h in range(hq):
            sc = (np.asarray(k[sel, h // group], np.float64) @ np.asarray(q[h], np.float64)) * scale * LOG2E
            m[s, h] = sc.max()
            p = np.exp2(sc - m[s, h])
            l[s, h] = p.sum()
            acc[s, h] = p @ np.asarray(v[sel, h // group], np.float64)
    return m, l, acc


def merge_partials(m, l, acc):
    """qsa_decode.py:63-86: weights 2^(m - max m) (a row without keys: every weight 0), out = sum(w acc) / sum(w l),
    0 where the total is 0."""
    top = m.max(0)
    top = np.where(np.isneginf(top), 0.0, top)
    w = np.exp2(m - top[None])
    total = (w * l).sum(0)
    out = (w[..., None] * acc).sum(0)
    with np.errstate(invalid='ignore', divide='ignore'):
        return np.where(total[:, None] > 0, out / total[:, None], 0.0)


def varlen_decode(q, k, v, cu_q, cu_k, scale, keys_per_split=128):
    """qsa_decode.py:25-113: row r's query q[cu_q[r]] ([T, Hq, D]) attends to the packed keys k / v [cu_k[r],
    cu_k[r+1]) ([N, Hkv, D]), as the reference computes it: split partials of keys_per_split keys (running max in
    the log2 domain, sum, unnormalized accumulator) merged with weights 2^(m - max m); FP64 here. Returns
    [rows, Hq, D] (rows = len(cu_q) - 1); a row without keys gives 0."""
    rows = len(cu_q) - 1
    out = np.zeros((rows, q.shape[1], v.shape[-1]))
    for r in range(rows):
        a, b = int(cu_k[r]), int(cu_k[r + 1])
        if b <= a:
            continue
        m, l, acc = split_partials(np.asarray(q[int(cu_q[r])], np.float64), k[a:b], v[a:b], np.ones(b - a, bool),
                                   scale, keys_per_split)
        out[r] = merge_partials(m, l, acc)
    return out


# --- block-sparse decode over head-major pages (MiniMax) ----------------------------------------------------------

def block_sparse_decode(q, k_pay, k_sf, v_pay, v_sf, req_to_token, slot_ids, topk_idx, seq_lens, block_size, scale,
                        kv_scale=1.0, attend=None):
    """kv_fp4.py:52-116 with the chunk merge of :149-152, reference values. q [B, Hq, D]; pool pages k_pay / v_pay
    [pages, Hkv, block, D/2] u8 and k_sf / v_sf [pages, Hkv, block, D/16] E4M3 bytes (no global scale: kv_scale
    multiplies the scores and the output, :100, :112-113); topk_idx [Hkv, B, T] block ids, -1 padded. For row b and KV
    head h: length L = min(seq_lens[b], req_to_token.shape[1]) (:69); the first (number of ids >= 0) entries are read
    (:73-76), an id e >= 0 with c = e * block < L naming positions c .. c + block - 1 below L (:86-93) at page
    req_to_token[slot_ids[b], c] // block, rows req_to_token[...] % block + n (:89-91). A negative id inside the
    counted prefix is skipped here (the reference would read position -block). ``attend`` (default the FP64 softmax)
    gets (q [group, D], k [N, 1, D], v [N, 1, D], valid, scale * kv_scale). Returns (out [B, Hq, D] float64, lse
    [B, Hq] natural log-sum-exp of the scaled scores; 0 and -inf for a (row, head) without keys)."""
    attend = attend or softmax_attention
    q = np.asarray(q)
    b_n, hq, d = q.shape
    hkv = k_pay.shape[1]
    group = hq // hkv
    max_len = req_to_token.shape[1]
    out = np.zeros((b_n, hq, d))
    lse = np.full((b_n, hq), -np.inf)
    for b in range(b_n):
        length = min(int(seq_lens[b]), max_len)
        sid = int(slot_ids[b])
        for h in range(hkv):
            ids = np.asarray(topk_idx[h, b], dtype=np.int64)
            real = int((ids >= 0).sum())
            pages, rows = [], []
            for e in ids[:real]:
                c = int(e) * block_size
                if e < 0 or c >= length:
                    continue
                base = int(req_to_token[sid, c])
                n = min(block_size, length - c)
                pages.append(np.full(n, base // block_size))
                rows.append(base % block_size + np.arange(n))
            if not pages:
                continue
            pg, rw = np.concatenate(pages), np.concatenate(rows)
            k = nvfp4.dequant(k_pay[pg, h, rw], k_sf[pg, h, rw])[:, None]
            v = nvfp4.dequant(v_pay[pg, h, rw], v_sf[pg, h, rw])[:, None]
            qs = q[b, h * group:(h + 1) * group]
            ones = np.ones(k.shape[0], bool)
            out[b, h * group:(h + 1) * group] = attend(qs, k, v, ones, scale * kv_scale) * kv_scale
            s = k[:, 0].astype(np.float64) @ qs.astype(np.float64).T * scale * kv_scale
            top = s.max(0)
            lse[b, h * group:(h + 1) * group] = top + np.log(np.exp(s - top).sum(0))
    return out, lse


# --- sparse MLA ---------------------------------------------------------------------------------------------------

def block_sparse_prefill(q, k_pay, k_sf, v_pay, v_sf, req_to_token, slot_ids, topk_idx, cu_seqlens, cu_seqblocks,
                         seq_lens, prefix_lens, block_size_q, block_size, scale, kv_scale=1.0, attend=None):
    """kv_fp4.py:293-366 (the causal block-sparse prefill), reference values. q [total_q, Hq, D]; request b's queries
    are rows cu_seqlens[b] .. cu_seqlens[b+1]-1, query i at position prefix_lens[b] + i (:330-331) with the block list
    topk_idx[h, cu_seqblocks[b] + i // block_size_q] (:321); the first (number of ids >= 0) entries are read
    (:323-324, :336). Block id e names positions c = e * block .. c + block - 1 that are below seq_lens[b] (:340) and
    at most the query's position (:345); each position's slot s = req_to_token[sid, pos] (sid = slot_ids[b]; both
    wrapped into [0, pages * block), :313, :341-342) is page s // block, row s % block (:272-273). Pages and kv_scale
    as block_sparse_decode. Returns float64 [total_q, Hq, D] (0 for a (query, head) without keys)."""
    attend = attend or softmax_attention
    q = np.asarray(q)
    total, hq, d = q.shape
    hkv = k_pay.shape[1]
    group = hq // hkv
    max_slots = k_pay.shape[0] * block_size
    out = np.zeros((total, hq, d))
    for b in range(len(cu_seqlens) - 1):
        sid = int(slot_ids[b]) % max_slots
        for i in range(int(cu_seqlens[b + 1]) - int(cu_seqlens[b])):
            r = int(cu_seqlens[b]) + i
            qpos = int(prefix_lens[b]) + i
            limit = min(int(seq_lens[b]), qpos + 1)
            for h in range(hkv):
                ids = np.asarray(topk_idx[h, int(cu_seqblocks[b]) + i // block_size_q], dtype=np.int64)
                ids = ids[:int((ids >= 0).sum())]
                pos = (ids[ids >= 0, None] * block_size + np.arange(block_size)).ravel()
                pos = pos[pos < limit]
                if pos.size == 0:
                    continue
                slot = np.asarray(req_to_token[sid, pos], dtype=np.int64) % max_slots
                pg, rw = slot // block_size, slot % block_size
                k = nvfp4.dequant(k_pay[pg, h, rw], k_sf[pg, h, rw])[:, None]
                v = nvfp4.dequant(v_pay[pg, h, rw], v_sf[pg, h, rw])[:, None]
                qs = q[r, h * group:(h + 1) * group]
                out[r, h * group:(h + 1) * group] = attend(qs, k, v, np.ones(pos.size, bool), scale * kv_scale) \
                    * kv_scale
    return out


def dequantize_context(pay, sf, req_to_token, slot_ids, seq_lens, rows_per_req):
    """kv_fp4.py:496-530: request b's positions pos < min(seq_lens[b], rows_per_req) as FP32 rows b * rows_per_req +
    pos of [batch * rows_per_req, heads, D] (other rows NaN: the reference leaves them unwritten); token slot
    s = req_to_token[sid, pos] (sid, s wrapped into [0, pages * block)) at page s // block, row s % block of pay / sf
    [pages, heads, block, D/2 | D/16] ([pages, block, ...]: one head)."""
    if pay.ndim == 3:
        pay, sf = pay[:, None], sf[:, None]
    pages, heads, block, half = pay.shape
    max_slots = pages * block
    out = np.full((len(slot_ids) * rows_per_req, heads, 2 * half), np.nan, dtype=np.float32)
    for b, sid in enumerate(slot_ids):
        n = min(int(seq_lens[b]), rows_per_req)
        slot = np.asarray(req_to_token[int(sid) % max_slots, :n], dtype=np.int64) % max_slots
        pg, rw = slot // block, slot % block
        for h in range(heads):
            out[b * rows_per_req:b * rows_per_req + n, h] = nvfp4.dequant(pay[pg, h, rw], sf[pg, h, rw])
    return out


def sparse_mla(q, latent_pay, latent_sf, rope, g, indices, topk_length, sink, scale, dtype=np.float64, extra=None):
    """Sparse MLA over an NVFP4 latent + BF16 rope cache, reference values (the FP64 reference of
    tests/ds_sparse_mla_check.py:44-67 on this layout; sparse_mla.py:88-125 for the two key lists): q [R, H, Dl + Dr];
    per token the key is [(e2m1 * e4m3) * g latent (Dl), rope (Dr)] and the value is the latent; indices [R, K] are
    pool slots (-1 none), topk_length [R] or None; extra = (latent_pay, latent_sf, rope, g, indices, topk_length) of a
    second cache whose valid keys follow the first list's; sink [H] or None enters the denominator as exp(sink - m).
    Returns (out [R, H, Dl], lse [R, H] natural log of the keys' sum, -inf for a row without keys)."""
    q = np.asarray(q, dtype=dtype)
    rows_n, heads, _ = q.shape
    dl = latent_pay.shape[-1] * 2
    out = np.zeros((rows_n, heads, dl), dtype=dtype)
    lse = np.full((rows_n, heads), -np.inf, dtype=dtype)
    lists = [(latent_pay, latent_sf, rope, g, indices, topk_length)]
    if extra is not None:
        lists.append(extra)
    for r in range(rows_n):
        keys, lats = [], []
        for pay, sf, rp, gg, idx_all, lengths in lists:
            idx = np.asarray(idx_all[r], dtype=np.int64)
            cols = np.arange(idx.shape[0])
            valid = (idx >= 0) & (idx < pay.shape[0])
            if lengths is not None:
                valid &= cols < int(lengths[r])
            sel = idx[valid]
            if sel.size == 0:
                continue
            lat = nvfp4.dequant(pay[sel], sf[sel], gg).astype(dtype)
            keys.append(np.concatenate([lat, np.asarray(rp[sel], dtype=dtype)], -1))
            lats.append(lat)
        if not keys:
            continue
        key = np.concatenate(keys, 0)
        lat = np.concatenate(lats, 0)
        s = (key @ q[r].T) * dtype(scale)        # [n, H]
        m = s.max(0)
        p = np.exp(s - m[None])
        total = p.sum(0)
        lse[r] = m + np.log(total)
        if sink is not None:
            total = total + np.exp(np.asarray(sink, dtype=dtype) - m)
        out[r] = (p.T @ lat) / total[:, None]
    return out, lse


# --- sparse MLA on DeepSeek V4 FP8 pages ----------------------------------------------------------------------------

V4_NOPE, V4_ROW = 448, 576


def v4_keys(pages, page_size, page_stride, tokens=None):
    """Keys of DeepSeek V4 FP8 pages (sparse_mla.py:38-59): token t = row t % page_size of page t // page_size;
    key[:448] = e4m3(byte) * 2^(e - 127) with e the UE8M0 byte of its 64-value group (e = 0 as 2^-127, the bit pattern
    0x00400000 of :52), key[448:] = the 64 BF16 rope values. pages: uint8, page p at byte p * page_stride. Returns
    float64 [tokens, 512]."""
    flat = np.asarray(pages, dtype=np.uint8).reshape(-1)
    n_pages = flat.size // page_stride if tokens is None else -(-tokens // page_size)
    tokens = n_pages * page_size if tokens is None else tokens
    t = np.arange(tokens)
    base = (t // page_size) * page_stride
    row = t % page_size
    data = flat[(base + row * V4_ROW)[:, None] + np.arange(V4_ROW)[None, :]]
    exps = flat[(base + page_size * V4_ROW + row * 8)[:, None] + np.arange(7)[None, :]].astype(np.int64)
    scale = np.where(exps == 0, 2.0 ** -127, np.exp2(exps.astype(np.float64) - 127))
    nope = nvfp4.e4m3_decode(data[:, :V4_NOPE]).astype(np.float64) * np.repeat(scale, 64, axis=1)
    rope = nvfp4.bf16_to_f32(data[:, V4_NOPE:].copy().view(np.uint16)).astype(np.float64)
    return np.concatenate([nope, rope], 1)


def sparse_mla_v4(q, keys1, indices1, length1, sink, scale, keys2=None, indices2=None, length2=None):
    """Sparse MLA on V4 keys (value = key, 512 wide) in FP64, the reference of tests/ds_sparse_mla_check.py:44-67:
    row r attends to the valid entries of indices1[r] (>= 0 and column < length1[r]) in keys1 followed by those of
    indices2[r] in keys2; sink [H] or None enters the denominator as exp(sink - m). Returns (out [R, H, 512], lse
    [R, H] natural log of the keys' sum, -inf for a row without keys)."""
    q = np.asarray(q, dtype=np.float64)
    rows_n, heads, dim = q.shape
    out = np.zeros((rows_n, heads, dim))
    lse = np.full((rows_n, heads), -np.inf)
    for r in range(rows_n):
        ks = []
        for keys, idx_all, lengths in ((keys1, indices1, length1), (keys2, indices2, length2)):
            if keys is None:
                continue
            idx = np.asarray(idx_all[r], dtype=np.int64)
            valid = (idx >= 0) & (idx < keys.shape[0])
            if lengths is not None:
                valid &= np.arange(idx.shape[0]) < int(lengths[r])
            if valid.any():
                ks.append(keys[idx[valid]])
        if not ks:
            continue
        k = np.concatenate(ks, 0)
        s = (k @ q[r].T) * scale
        m = s.max(0)
        p = np.exp(s - m[None])
        total = p.sum(0)
        lse[r] = m + np.log(total)
        if sink is not None:
            total = total + np.exp(np.asarray(sink, dtype=np.float64) - m)
        out[r] = (p.T @ k) / total[:, None]
    return out, lse
