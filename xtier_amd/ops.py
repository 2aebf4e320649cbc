"""Python entry points over the C ABI, with the argument order, keywords and error types of the reference pack
functions they replace (xtier/packs/qwen4_exp/qsa_fp4.py, qsa_decode.py; xtier/packs/minimax_m3/kv_fp4.py;
xtier/backend/formats.py). Tensors are torch tensors on the GPU; every call runs on the current HIP stream.

``raw`` is the reference's tuple of a layer's pool buffers (qsa_fp4.py:43-58):
(k_pay u8 [slots, kv_heads, dim/2], v_pay, k_scales u8 [slots, kv_heads, dim/16], v_scales, gk f32 [1], gv f32 [1]).
"""
import ctypes
import math
import warnings

import torch

from . import _lib

LOG2E = 1.4426950408889634
_DTYPES = {torch.bfloat16: _lib.XT_DTYPE_BF16, torch.float16: _lib.XT_DTYPE_F16}
_workspaces = {}   # device index -> uint8 tensor, grown on demand (never during a graph capture)
_retired = []      # workspaces a larger one replaced: kept alive, since graphs captured earlier hold their addresses


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError('xtier_amd: GPU tensors expected')


def _check_fp8_raw(raw):
    """An FP8 pool's raw tuple (k, v, None, None, None, None) (qsa_fp4.py:43-58, :165-171): E4M3 bytes [m, heads,
    dim] with a power-of-2 head size, contiguous."""
    k, v = raw[0], raw[1]
    dim = k.shape[2]
    if not (k.is_contiguous() and v.is_contiguous() and k.shape == v.shape and dim % 32 == 0
            and dim & (dim - 1) == 0):
        raise ValueError(f'xtier qsa_fp4: packed [m, heads, dim] FP8 rows with a power-of-2 head size expected, got '
                         f'{tuple(k.shape)}')
    k, v = (t if t.dtype == torch.uint8 else t.view(torch.uint8) for t in (k, v))
    _need_cuda(k, v)
    return (k, v, None, None, None, None), k.shape[1], dim


def is_fp8_raw(raw):
    """True for an FP8 pool's raw tuple (no block scales)."""
    return raw[2] is None


def _check_raw(raw, contiguous=True):
    """The reference's _check (qsa_fp4.py:165-171): packed [m, heads, dim/2] rows with a power-of-2 head size.
    contiguous=False also admits pools whose slots and heads are strided (the interleaved layout of KVPool): each head
    row contiguous, the slot and head strides the same for K and V."""
    k, v, k_sf, v_sf, gk, gv = raw
    if k_sf is None:
        raise NotImplementedError('xtier_amd: the fused attention reads NVFP4 pools; an FP8 pool takes the gather')
    dim = k.shape[2] * 2
    if contiguous:
        packed = k.is_contiguous() and v.is_contiguous() and k_sf.is_contiguous() and v_sf.is_contiguous()
    else:
        packed = (all(t.dim() == 3 and t.stride(2) == 1 and (t.shape[1] == 1 or t.stride(1) >= t.shape[2])
                      for t in (k, v, k_sf, v_sf))
                  and k.stride()[:2] == v.stride()[:2] and k_sf.stride()[:2] == v_sf.stride()[:2]
                  and k.shape == v.shape and k_sf.shape == v_sf.shape and k_sf.shape[2] * 8 == k.shape[2])
    if not (packed and dim % 32 == 0 and dim & (dim - 1) == 0):
        raise ValueError(f'xtier qsa_fp4: packed [m, heads, dim / 2] rows with a power-of-2 head size expected, got '
                         f'{tuple(k.shape)}')
    if k.dtype != torch.uint8:
        k, v, k_sf, v_sf = (t.view(torch.uint8) for t in (k, v, k_sf, v_sf))
    _need_cuda(k, v, k_sf, v_sf, gk, gv)
    return (k, v, k_sf, v_sf, gk.float() if gk.dtype != torch.float32 else gk,
            gv.float() if gv.dtype != torch.float32 else gv), k.shape[1], dim


def _head_stride(t):
    """Bytes between the head rows of a pool view [slots, heads, width] (0, the packed default, for one head)."""
    return t.stride(1) if t.shape[1] > 1 else 0


def workspace(device, nbytes):
    """A zero-filled device byte buffer of at least nbytes, kept per device. The decode kernels need their workspace
    zero before first use and leave it so. It cannot grow inside a graph capture (the zero fill would be recorded):
    call this once with the largest size before capturing."""
    device = torch.device(device)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    buf = _workspaces.get(idx)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f'xtier_amd: the decode workspace must hold {nbytes} bytes before a graph capture; '
                               'call xtier_amd.ops.workspace(device, nbytes) first')
        if buf is not None:
            # never freed: a graph captured with it replays into these bytes (its arrival counters must stay zero)
            _retired.append(buf)
        buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        _workspaces[idx] = buf
    return buf


def _cached_workspace_bytes(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    buf = _workspaces.get(idx)
    return 0 if buf is None else buf.numel()


def new_workspace(device, rows, q_heads, dim, splits):
    """A dedicated zero-filled workspace for sparse_decode calls of this shape (one per stream / graph)."""
    return torch.zeros(decode_workspace_bytes(rows, q_heads, dim, splits), dtype=torch.uint8, device=device)


# --- NVFP4 quantization --------------------------------------------------------------------------------------------

def global_scale(x, out=None):
    """FP32 [1] device tensor g = max(amax|x| / (6 * 448), 1e-12) of a BF16 tensor [..., heads, dim] or [..., dim]
    (formats.py:122)."""
    _need_cuda(x)
    x3 = x.reshape(-1, 1, x.shape[-1]) if x.dim() < 3 else x.reshape(-1, *x.shape[-2:])
    if out is None:
        out = torch.empty(1, dtype=torch.float32, device=x.device)
    ws = torch.empty(4, dtype=torch.uint8, device=x.device)
    _lib.check(_lib.lib().xt_nvfp4_global_scale(_ptr(x3), x3.shape[0], x3.shape[1], x3.shape[2], x3.stride(0),
                                                 x3.stride(1), _ptr(out), _ptr(ws), _stream(x)), 'global_scale')
    return out


def quantize_append(x, slots, g, pay, scales, saturate=True):
    """NVFP4 quantize-on-append: rows x [n, heads, dim] BF16 (strided rows allowed, last dim contiguous) into the pool
    at slots [n] (int64; a negative slot skips its row) with the device global scale g [1]. saturate=True stores 448
    for a block scale that rounds above the E4M3 range (never NaN); False reproduces the reference's torch cast."""
    _need_cuda(x, slots, g, pay, scales)
    if x.dtype != torch.bfloat16 or x.dim() != 3 or x.stride(-1) != 1:
        raise ValueError(f'xtier_amd.quantize_append: BF16 [n, heads, dim] rows expected, got {x.dtype} '
                         f'{tuple(x.shape)}')
    if slots.dtype != torch.int64:
        slots = slots.to(torch.int64)
    slots = slots.contiguous()
    if pay.stride(-1) != 1 or scales.stride(-1) != 1 or pay.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise ValueError('xtier_amd.quantize_append: uint8 payload / scale views with packed head rows expected')
    _lib.check(_lib.lib().xt_nvfp4_quantize_append(
        _ptr(x), x.shape[0], x.shape[1], x.shape[2], x.stride(0), x.stride(1), _ptr(slots), _ptr(g),
        _ptr(pay), _ptr(scales), pay.shape[0], pay.stride(0), scales.stride(0), _head_stride(pay),
        _head_stride(scales), 1 if saturate else 0, _stream(x)),
        'quantize_append')


def _pool_strides(view, heads, page_size):
    """(page, row, head) byte strides and rows per page of one tensor's pool view: token-major [slots, heads, width]
    or [slots, width] (page_size 1); head-major pages [pages, heads, page, width]; one-head pages [pages, page, width]
    (page_size > 1)."""
    es = view.element_size()
    if view.dim() == 4:
        return view.stride(0) * es, view.stride(2) * es, view.stride(1) * es, view.shape[2]
    if page_size > 1 and view.dim() == 3:
        return view.stride(0) * es, view.stride(1) * es, 0, view.shape[1]
    return view.stride(0) * es, 0, (view.stride(1) * es if view.dim() == 3 and heads > 1 else 0), 1


def store_kv(stores, slots, page_size=1, saturate=True):
    """The fused KV-write epilogue: every store of ``stores`` written at ``slots`` [n] (int64; negative: skipped) in
    one launch. A store is (x, g, pay, scales): x BF16 [n, heads, dim] (or [n, dim]); g the device global scale
    [1] and pay / scales the pool's uint8 payload / scale views (token-major [slots, heads, width] with page_size 1,
    head-major pages [pages, heads, page, width], or one-head pages [pages, page, width]); or g None for a plain BF16
    copy into pay (the rope rows of a latent cache), scales None. Bytes equal one quantize_append per store."""
    if not 1 <= len(stores) <= 4:
        raise ValueError('xtier_amd.store_kv: 1 to 4 stores')
    descs, keep = [], []
    n = None
    pool_slots = None
    for x, g, pay, sc in stores:
        x3 = x if x.dim() == 3 else x.unsqueeze(1)
        if x3.dtype != torch.bfloat16 or x3.stride(-1) != 1:
            raise ValueError(f'xtier_amd.store_kv: BF16 rows with a contiguous last dim expected, got {x.dtype}')
        _need_cuda(x3, g, pay, sc, slots)
        n = x3.shape[0] if n is None else n
        if x3.shape[0] != n:
            raise ValueError('xtier_amd.store_kv: every store takes the same rows')
        heads, dim = x3.shape[1], x3.shape[2]
        pp, pr, ph, page = _pool_strides(pay, heads, page_size)
        sp = sr = sh = 0
        if g is not None:
            if pay.dtype != torch.uint8 or sc.dtype != torch.uint8:
                pay, sc = pay.view(torch.uint8), sc.view(torch.uint8)
            sp, sr, sh, _ = _pool_strides(sc, heads, page_size)
            g = g if g.dtype == torch.float32 else g.float()
        if page != page_size:
            raise ValueError(f'xtier_amd.store_kv: pages of {page} rows, page_size {page_size}')
        slots_here = pay.shape[0] * page
        pool_slots = slots_here if pool_slots is None else min(pool_slots, slots_here)
        descs.append(_lib.KvStore(_ptr(x3), x3.stride(0), x3.stride(1), heads, dim, _ptr(g), _ptr(pay), _ptr(sc),
                                  pp, pr, ph, sp, sr, sh))
        keep.append((x3, g, pay, sc))
    if slots.dtype != torch.int64:
        slots = slots.to(torch.int64)
    slots = slots.contiguous()
    arr = (_lib.KvStore * len(descs))(*descs)
    _lib.check(_lib.lib().xt_nvfp4_store_kv(arr, len(descs), n, _ptr(slots), pool_slots, int(page_size),
                                            1 if saturate else 0, _stream(slots)), 'store_kv')


def nvfp4_store_kv_index(k, v, ik, kpay, ksc, vpay, vsc, ipay, isc, loc, global_scale, page_size=128):
    """SGLang's fused MiniMax NVFP4 store as tests/minimax_kv_fp4_check.py:152-175 calls it (enabled by the pack at
    xtier/packs/minimax_m3/kv_fp4.py:546-559): main K and V [n, heads, dim] and index K [n, dim] quantized with the
    pool's global scale into head-major pages (kpay / vpay [pages, heads, page_size, dim/2], ksc / vsc [.., dim/16];
    ipay / isc [pages, page_size, dim/2 | dim/16]) at token slots loc [n], in one launch. The E4M3 conversion
    saturates (a scale byte is never NaN), as a store into a serving cache must."""
    g = global_scale if torch.is_tensor(global_scale) else torch.tensor([float(global_scale)], device=k.device)
    g = g.reshape(1)
    store_kv([(k, g, kpay, ksc), (v, g, vpay, vsc), (ik, g, ipay, isc)], loc, page_size=page_size)


def nvfp4_encode(x, saturate=False):
    """formats.py:114-128 on the GPU for a BF16 tensor [slots, heads, dim] (or [rows, dim]): (payload u8
    [..., dim/2], scale bytes u8 [..., dim/16], g f32 [1])."""
    shape = x.shape
    x3 = x.reshape(-1, 1, shape[-1]) if x.dim() == 2 else x
    if x3.stride(-1) != 1:
        x3 = x3.contiguous()
    n, heads, dim = x3.shape
    pay = torch.empty(n, heads, dim // 2, dtype=torch.uint8, device=x.device)
    sc = torch.empty(n, heads, dim // 16, dtype=torch.uint8, device=x.device)
    g = global_scale(x3)
    quantize_append(x3, torch.arange(n, device=x.device, dtype=torch.int64), g, pay, sc, saturate=saturate)
    return pay.reshape(*shape[:-1], dim // 2), sc.reshape(*shape[:-1], dim // 16), g


# --- QSA gather / pack --------------------------------------------------------------------------------------------

def gather(raw, req_to_token, req_indices, indices, seq_lens, cu_k, out_k, out_v, batch, topk, zero_fill_cols=0):
    """qsa_fp4.gather (qsa_fp4.py:174-180): the decode/verify rows of ``indices`` dequantized into out_k / out_v
    (compact, or page-aligned and zero-filled up to zero_fill_cols), from an NVFP4 pool or an FP8 one
    (raw = (k, v, None, None, None, None))."""
    fp8 = is_fp8_raw(raw)
    raw, heads, dim = _check_fp8_raw(raw) if fp8 else _check_raw(raw)
    if out_k.dtype not in _DTYPES or not out_k.is_contiguous() or not out_v.is_contiguous():
        raise ValueError('xtier_amd.gather: contiguous BF16/FP16 outputs expected')
    _need_cuda(req_to_token, req_indices, indices, seq_lens, cu_k, out_k, out_v)
    req_indices = req_indices.to(torch.int64) if req_indices.dtype != torch.int64 else req_indices
    tail = (_ptr(req_to_token), req_to_token.stride(0), _ptr(req_indices.contiguous()), _ptr(indices),
            indices.stride(0), _ptr(seq_lens), _ptr(cu_k), _ptr(out_k), _ptr(out_v), _DTYPES[out_k.dtype], int(batch),
            int(topk), int(zero_fill_cols), _stream(out_k))
    if fp8:
        st = _lib.lib().xt_qsa_gather_fp8(_ptr(raw[0]), _ptr(raw[1]), raw[0].shape[0], heads, dim, *tail)
    else:
        st = _lib.lib().xt_qsa_gather_nvfp4(*map(_ptr, raw), raw[0].shape[0], heads, dim, *tail)
    _lib.check(st, 'gather')


def pack(raw, req_to_token, req_indices, cu_k, total_k, max_k, output_dtype):
    """qsa_fp4.pack (qsa_fp4.py:183-192): whole prefixes as (packed_k, packed_v) [total_k, heads, dim], from an NVFP4
    or an FP8 pool."""
    fp8 = is_fp8_raw(raw)
    raw, heads, dim = _check_fp8_raw(raw) if fp8 else _check_raw(raw)
    device = raw[0].device
    packed_k = torch.empty((total_k, heads, dim), dtype=output_dtype, device=device)
    packed_v = torch.empty((total_k, heads, dim), dtype=output_dtype, device=device)
    batch = req_indices.numel()
    req_indices = req_indices.to(torch.int64).contiguous()
    tail = (_ptr(req_to_token), req_to_token.stride(0), req_to_token.stride(1), _ptr(req_indices), batch, _ptr(cu_k),
            int(max_k), _ptr(packed_k), _ptr(packed_v), _DTYPES[output_dtype], _stream(packed_k))
    if fp8:
        st = _lib.lib().xt_qsa_pack_fp8(_ptr(raw[0]), _ptr(raw[1]), raw[0].shape[0], heads, dim, *tail)
    else:
        st = _lib.lib().xt_qsa_pack_nvfp4(*map(_ptr, raw), raw[0].shape[0], heads, dim, *tail)
    _lib.check(st, 'pack')
    return packed_k, packed_v


def valid_counts(seq_lens, indices, valid=None, cu_seqlens_k=None):
    """(valid_counts [batch] int32, cu_seqlens_k [batch + 1] int32) of top-k lists indices [batch, topk]: the number of
    entries with 0 <= index < seq_lens[b] and their running sum (SGLang's qwen_sparse_fa2_cu_seqlens_triton as
    qsa_fp4.py:255-256 uses it; valid entries first, -1 padding after)."""
    batch, topk = indices.shape
    _need_cuda(seq_lens, indices)
    indices = indices if indices.dtype == torch.int32 and indices.stride(1) == 1 else \
        indices.to(torch.int32).contiguous()
    seq_lens = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
    if valid is None:
        valid = torch.empty(batch, dtype=torch.int32, device=indices.device)
    if cu_seqlens_k is None:
        cu_seqlens_k = torch.empty(batch + 1, dtype=torch.int32, device=indices.device)
    _lib.check(_lib.lib().xt_qsa_valid_counts(_ptr(seq_lens), _ptr(indices), indices.stride(0), batch, topk,
                                              _ptr(valid), _ptr(cu_seqlens_k), _stream(indices)), 'valid_counts')
    return valid, cu_seqlens_k


# --- fused sparse attention ---------------------------------------------------------------------------------------

_cu_counts = {}


def device_cus(device=None):
    """Compute units of the current (or given) GPU, 256 on an MI355X; 256 when no GPU is visible."""
    if not torch.cuda.is_available():
        return 256
    idx = torch.cuda.current_device() if device is None else torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    n = _cu_counts.get(idx)
    if n is None:
        n = _cu_counts[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return n


def default_splits(rows, kv_heads, topk, pair_heads=True):
    """Key splits per row: about one workgroup per CU, at least 512 keys per split (two steps of two loads in flight
    for each of a workgroup's 8 wavefronts), and at most 8192 keys per split (the slot list lives in LDS). With an
    even number of KV heads shared by every head's index list (`pair_heads`), workgroups of 2 KV heads are preferred
    when 2 or more such splits fill the CUs; else workgroups of 1 KV head. Small launches are latency-bound and every
    split adds to the merge, so the floor of 512 keys wins over filling the CUs. Measured on MI355X (256 CUs), per
    layer-step: batch 32 x 4 KV heads, top-2048: 2 KV heads x 4 splits 18.7 us, 1 KV head x 2 splits 19.1 us;
    batch 4 x 4 KV heads, top-2048: 1 / 2 / 4 / 8 / 16 splits 16.3 / 14.0 / 12.1 / 12.6 / 15.0 us; 1 row x 1 KV
    head, top-512: 1 / 2 splits 8.4 / 10.4 us; 4096 prefill rows -> 1."""
    if topk <= 0:
        return 1
    cap, floor = min(topk // 512, 64), min(64, math.ceil(topk / 8192))
    if pair_heads and kv_heads % 2 == 0 and rows > 0:
        s = math.ceil(device_cus() / (rows * (kv_heads // 2)))
        if 2 <= s <= cap:
            return max(s, floor)
    units = max(1, rows * kv_heads)
    return max(max(1, min(math.ceil(device_cus() / units), cap)), floor)


def varlen_splits(rows, kv_heads, group, max_k):
    """Key splits for varlen_decode: the fewest that fill every CU with workgroups of 4 (else 2) KV heads, which then
    stream whole packed key rows, as long as every split keeps at least 128 keys; else default_splits (one KV head per
    workgroup). Measured on MI355X (256 CUs): batch 32 x 4 KV heads, 2048 keys -> 8 splits of 4 KV heads."""
    tiles = -(-group // 16)
    cap = min(64, max(1, max_k // 128))
    for h in (4, 2):
        if kv_heads % h == 0 and h * tiles <= 8:
            s = math.ceil(device_cus() / max(1, rows * (kv_heads // h)))
            if s <= cap:
                return max(s, min(64, math.ceil(max_k / 8192)))
    return default_splits(rows, kv_heads, max_k, False)


def decode_workspace_bytes(rows, q_heads, dim, splits):
    return int(_lib.lib().xt_sparse_decode_workspace_bytes(rows, q_heads, dim, splits))


def sparse_decode(q, raw, table, indices, seq_lens, scale, page_size=1, row_req=None, counts=None, query_pos=None,
                  out=None, lse=None, splits=None, ws=None):
    """Fused NVFP4 sparse attention, one query per row: q [rows, q_heads, dim] BF16 attends to the valid positions of
    indices [rows, topk] (int32; valid: column < counts[r], 0 <= pos < seq_lens[r], pos <= query_pos[r] when given),
    resolved through ``table`` (token-granular req_to_token for page_size 1, else a page table) row row_req[r].
    Returns out [rows, q_heads, dim] (BF16 unless ``out`` is given); lse [rows, q_heads] FP32 is filled if given.
    ws: a workspace tensor, None (the per-device cached one), or 'static': the library's fixed per-GPU array
    (xt_sparse_decode_nvfp4_static; with ``out`` given the call allocates nothing)."""
    raw, kv_heads, dim = _check_raw(raw, contiguous=False)
    rows, q_heads, qdim = q.shape
    if qdim != dim:
        raise ValueError(f'xtier_amd.sparse_decode: q head size {qdim} != pool head size {dim}')
    _need_cuda(q, table, indices, seq_lens, row_req, counts, query_pos, out, lse)
    if q.dtype != torch.bfloat16 or q.stride(-1) != 1:
        q = q.to(torch.bfloat16).contiguous()
    if out is None:
        out = torch.empty((rows, q_heads, dim), dtype=torch.bfloat16, device=q.device)
    if out.dtype not in _DTYPES or out.stride(-1) != 1:
        raise ValueError('xtier_amd.sparse_decode: BF16/FP16 output with a contiguous last dim expected')
    if indices.dtype != torch.int32 or indices.stride(-1) != 1:
        indices = indices.to(torch.int32).contiguous()
    topk = indices.shape[1] if indices.dim() == 2 else 0
    if row_req is not None and row_req.dtype != torch.int64:
        row_req = row_req.to(torch.int64)
    seq_lens, counts, query_pos = (None if t is None else (t if t.dtype == torch.int32 else t.to(torch.int32))
                                   for t in (seq_lens, counts, query_pos))
    args = (_ptr(q), q.stride(0), q.stride(1), *map(_ptr, raw), raw[0].shape[0], raw[0].stride(0), raw[2].stride(0),
            _head_stride(raw[0]), _head_stride(raw[2]), kv_heads, q_heads, dim, _ptr(table), table.stride(0),
            int(page_size), _ptr(row_req), _ptr(indices), indices.stride(0), topk, _ptr(counts), _ptr(seq_lens),
            _ptr(query_pos), float(scale), _ptr(out), out.stride(0), out.stride(1), _DTYPES[out.dtype], _ptr(lse),
            rows)
    if isinstance(ws, str) and ws == 'static':
        # the library's own per-GPU scratch array: nothing is allocated for this call
        splits = default_splits(rows, kv_heads, topk) if splits is None else splits
        _lib.check(_lib.lib().xt_sparse_decode_nvfp4_static(*args, int(splits), _stream(q)), 'sparse_decode')
        return out
    if splits is None:
        splits = _capture_splits(q.device, rows, q_heads, dim, default_splits(rows, kv_heads, topk), ws)
    ws = _decode_ws(q.device, rows, q_heads, dim, splits, ws)
    _lib.check(_lib.lib().xt_sparse_decode_nvfp4(*args, int(splits), _ptr(ws), ws.numel(), _stream(q)),
               'sparse_decode')
    return out


def _narrowed(what, splits, fewer, need):
    """A capture that must run with fewer key splits than the shape wants says so once per shape: it is slower."""
    key = (what, splits, fewer, need)
    if key not in _warned:
        _warned.add(key)
        warnings.warn(f'xtier_amd.{what}: inside a graph capture the cached workspace holds less than the {need} bytes '
                      f'{splits} key splits need, so the call runs {fewer}, which is slower; call '
                      f'xtier_amd.ops.workspace(device, {need}) before capturing, or pass ws=', RuntimeWarning,
                      stacklevel=3)
    return fewer


_warned = set()


def _capture_splits(device, rows, q_heads, dim, splits, ws):
    """``splits``, or 1 inside a graph capture whose cached workspace is too small (one key split needs no partials,
    so no workspace has to grow inside the capture), with a warning."""
    need = decode_workspace_bytes(rows, q_heads, dim, splits)
    if splits > 1 and ws is None and torch.cuda.is_current_stream_capturing() and _cached_workspace_bytes(device) < need:
        return _narrowed('sparse_decode', splits, 1, need)
    return splits


def _decode_ws(device, rows, q_heads, dim, splits, ws):
    """The caller's workspace, else the per-device one (a throwaway buffer for one split inside a capture that the
    cached one cannot serve: the kernel never reads it then)."""
    need = decode_workspace_bytes(rows, q_heads, dim, splits)
    if ws is not None:
        return ws
    if _cached_workspace_bytes(device) >= need or not torch.cuda.is_current_stream_capturing():
        return workspace(device, need)
    return torch.empty(need, dtype=torch.uint8, device=device)


def fp4_sparse_decode(q, k_pay, k_sc, v_pay, v_sc, req_to_token, slot_ids, topk_idx, seq_lens, block_size,
                      sm_scale=None, kv_scale=1.0, num_warps=4, num_stages=2, out=None, lse=None, splits=None,
                      ws=None):
    """Block-sparse decode over an NVFP4 cache of head-major pages (kv_fp4.py:119-153): q [b, qh, d] BF16; k_pay /
    v_pay [pages, kh, block, d/2] uint8; k_sc / v_sc [pages, kh, block, d/16] E4M3 bytes (uint8 or float8_e4m3fn);
    topk_idx [kh, b, topk] block ids (-1 padded at the end); row b reads request slot_ids[b] of req_to_token, its
    length clamped to req_to_token.shape[1]. kv_scale multiplies the scores and the output. Returns [b, qh, d] (BF16
    unless ``out`` is given); lse [b, qh] FP32 is filled if given. num_warps / num_stages are accepted for the
    reference's signature and ignored."""
    assert block_size == k_pay.shape[2] and k_pay.stride(3) == 1 and k_sc.stride(3) == 1
    assert k_pay.stride() == v_pay.stride() and k_sc.stride() == v_sc.stride()
    b, qh, d = q.shape
    kh = k_pay.shape[1]
    if k_pay.shape[3] * 2 != d or k_sc.shape[3] * 16 != d or k_pay.shape != v_pay.shape or k_sc.shape != v_sc.shape:
        raise ValueError(f'xtier_amd.fp4_sparse_decode: pages {tuple(k_pay.shape)} / {tuple(k_sc.shape)} do not hold '
                         f'head size {d}')
    if qh % kh:
        raise ValueError(f'xtier_amd.fp4_sparse_decode: {qh} query heads over {kh} KV heads')
    _need_cuda(q, k_pay, k_sc, v_pay, v_sc, req_to_token, slot_ids, topk_idx, seq_lens, out, lse)
    if sm_scale is None:
        sm_scale = d ** -0.5
    k_pay, v_pay, k_sc, v_sc = (t if t.dtype == torch.uint8 else t.view(torch.uint8) for t in (k_pay, v_pay, k_sc, v_sc))
    if q.dtype != torch.bfloat16 or q.stride(-1) != 1:
        q = q.to(torch.bfloat16).contiguous()
    if out is None:
        out = torch.empty((b, qh, d), dtype=torch.bfloat16, device=q.device)
    if req_to_token.dtype != torch.int32 or req_to_token.stride(1) != 1:
        req_to_token = req_to_token.to(torch.int32).contiguous()
    if topk_idx.dtype != torch.int32 or topk_idx.stride(2) != 1:
        topk_idx = topk_idx.to(torch.int32).contiguous()
    slot_ids = slot_ids if slot_ids.dtype == torch.int64 else slot_ids.to(torch.int64)
    seq_lens = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
    topk = topk_idx.shape[2]
    if splits is None:
        splits = _capture_splits(q.device, b, qh, d, default_splits(b, kh, topk * block_size, False), ws)
    ws = _decode_ws(q.device, b, qh, d, splits, ws)
    _lib.check(_lib.lib().xt_block_sparse_decode_nvfp4(
        _ptr(q), q.stride(0), q.stride(1), _ptr(k_pay), _ptr(v_pay), _ptr(k_sc), _ptr(v_sc), float(kv_scale),
        k_pay.shape[0], kh, qh, d, int(block_size), k_pay.stride(0), k_pay.stride(1), k_pay.stride(2),
        k_sc.stride(0), k_sc.stride(1), k_sc.stride(2), _ptr(req_to_token), req_to_token.stride(0),
        req_to_token.shape[1], _ptr(slot_ids), _ptr(topk_idx), topk_idx.stride(0), topk_idx.stride(1), topk,
        _ptr(seq_lens), float(sm_scale), _ptr(out), out.stride(0), out.stride(1), _DTYPES[out.dtype], _ptr(lse), b,
        int(splits), _ptr(ws), ws.numel(), _stream(q)), 'fp4_sparse_decode')
    return out


def _pages(pay, sc, what):
    """Head-major page views (payload [pages, kh, block, d/2], scales [pages, kh, block, d/16]) -> uint8 views."""
    if pay.dtype != torch.uint8:
        pay = pay.view(torch.uint8)
    if sc.dtype != torch.uint8:
        sc = sc.view(torch.uint8)
    if pay.dim() != 4 or sc.dim() != 4 or pay.stride(3) != 1 or sc.stride(3) != 1 or pay.shape[:3] != sc.shape[:3] \
            or sc.shape[3] * 8 != pay.shape[3]:
        raise ValueError(f'xtier_amd.{what}: pages [pages, kv_heads, block, d/2] / [.., d/16] expected, got '
                         f'{tuple(pay.shape)} / {tuple(sc.shape)}')
    return pay, sc


def fp4_prefill_gqa_share_sparse(q, k_cache, v_cache, sink, req_to_token, slot_ids, topk_idx, block_size_q,
                                 block_size_k, cu_seqlens, seq_lens, prefix_lens, max_seqlen_q, sm_scale=None,
                                 use_tma=True, cu_seqblocks_q=None, max_seqblock_q=None, q_scale=None, k_scale=None,
                                 v_scale=None, loc_mapping=None, *, k_sc=None, v_sc=None, kv_scale=1.0, num_warps=4,
                                 num_stages=2, out=None, splits=None, ws=None):
    """Causal block-sparse prefill over an NVFP4 cache of head-major pages (kv_fp4.py:369-404): q [total_q, qh, d]
    BF16, request b's queries are rows cu_seqlens[b] .. cu_seqlens[b+1]-1 at positions prefix_lens[b] + i; the
    queries of one block of block_size_q share the block list topk_idx[kh, cu_seqblocks_q[b] + i // block_size_q, :]
    (block ids of block_size_k tokens, -1 padded); k_cache / v_cache payload pages, k_sc / v_sc their scale bytes.
    Returns o [total_q, qh, d] in q's dtype. Lengths are clamped to req_to_token.shape[1]; a key block wholly after a
    query's position adds nothing to its softmax (the reference's running max starts at -inf, so such a block listed
    first gives it NaN). use_tma / num_warps / num_stages / max_seqblock_q are accepted for the reference's signature
    and ignored."""
    assert sink is None and loc_mapping is None and block_size_k == k_cache.shape[2]
    k_pay, k_sc8 = _pages(k_cache, k_sc, 'fp4_prefill_gqa_share_sparse')
    v_pay, v_sc8 = _pages(v_cache, v_sc, 'fp4_prefill_gqa_share_sparse')
    assert k_pay.stride() == v_pay.stride() and k_sc8.stride() == v_sc8.stride()
    total_q, qh, d = q.shape
    kh = k_pay.shape[1]
    if k_pay.shape[3] * 2 != d or qh % kh:
        raise ValueError(f'xtier_amd.fp4_prefill_gqa_share_sparse: q {tuple(q.shape)} does not fit pages '
                         f'{tuple(k_pay.shape)}')
    _need_cuda(q, k_pay, v_pay, req_to_token, slot_ids, topk_idx, cu_seqlens, seq_lens, prefix_lens, out)
    sm_scale = (d ** -0.5 if sm_scale is None else sm_scale) * (1.0 if q_scale is None else q_scale)
    dev = q.device
    cu = cu_seqlens.to(torch.int64)
    if cu_seqblocks_q is None:
        nblk = (cu[1:] - cu[:-1] + block_size_q - 1) // block_size_q
        cu_seqblocks_q = torch.cat([torch.zeros(1, dtype=torch.int64, device=dev), torch.cumsum(nblk, 0)])
    r = torch.arange(total_q, device=dev, dtype=torch.int64)
    bi = torch.searchsorted(cu[1:].contiguous(), r, right=True)
    local = r - cu[bi]
    max_slots = k_pay.shape[0] * block_size_k
    # wrapped as the reference wraps it, then kept inside the table (on the device: no synchronization)
    row_req = torch.clamp(torch.remainder(slot_ids.to(torch.int64)[bi], max_slots), max=req_to_token.shape[0] - 1)
    row_qpos = (prefix_lens.to(torch.int64)[bi] + local).to(torch.int32)
    row_seq = torch.clamp(seq_lens.to(torch.int32)[bi], max=req_to_token.shape[1])   # positions within the table
    row_idx = torch.clamp(cu_seqblocks_q.to(torch.int64)[bi] + local // block_size_q,
                          max=topk_idx.shape[1] - 1).to(torch.int32)   # a list row of topk_idx
    if q.stride(-1) != 1:
        q = q.contiguous()
    if out is None:
        out = torch.empty(total_q, qh, d, dtype=q.dtype if q.dtype in _DTYPES else torch.bfloat16, device=dev)
    if req_to_token.dtype != torch.int32 or req_to_token.stride(1) != 1:
        req_to_token = req_to_token.to(torch.int32).contiguous()
    if topk_idx.dtype != torch.int32 or topk_idx.stride(2) != 1:
        topk_idx = topk_idx.to(torch.int32).contiguous()
    q16 = q if q.dtype == torch.bfloat16 else q.to(torch.bfloat16)
    topk = topk_idx.shape[2]
    if splits is None:
        splits = _capture_splits(dev, total_q, qh, d, default_splits(total_q, kh, topk * block_size_k, False),
                                 ws)
    ws = _decode_ws(dev, total_q, qh, d, splits, ws)
    _lib.check(_lib.lib().xt_block_sparse_prefill_nvfp4(
        _ptr(q16), q16.stride(0), q16.stride(1), _ptr(k_pay), _ptr(v_pay), _ptr(k_sc8), _ptr(v_sc8), float(kv_scale),
        k_pay.shape[0], kh, qh, d, int(block_size_k), k_pay.stride(0), k_pay.stride(1), k_pay.stride(2),
        k_sc8.stride(0), k_sc8.stride(1), k_sc8.stride(2), _ptr(req_to_token), req_to_token.stride(0), _ptr(row_req),
        _ptr(row_seq), _ptr(row_qpos), _ptr(topk_idx), topk_idx.stride(0), topk_idx.stride(1), topk, _ptr(row_idx),
        float(sm_scale), _ptr(out), out.stride(0), out.stride(1), _DTYPES[out.dtype], None, total_q, int(splits),
        _ptr(ws), ws.numel(), _stream(q16)), 'fp4_prefill_gqa_share_sparse')
    return out


def dequantize_context(pay, sc, req_to_token, slot_ids, seq_lens, rows_per_req, out=None):
    """BF16 [b * rows_per_req, heads, d] of each request's first seq_lens[b] positions (kv_fp4.py:514-530): pay / sc
    [pages, heads, block, d/2 | d/16] (main) or [pages, block, ...] (the one-head index cache)."""
    if pay.dim() == 3:
        pay, sc = pay.unsqueeze(1), sc.unsqueeze(1)
    pay, sc = _pages(pay, sc, 'dequantize_context')
    pages, heads, block, half = pay.shape
    b = slot_ids.shape[0]
    _need_cuda(pay, sc, req_to_token, slot_ids, seq_lens, out)
    if out is None:
        out = torch.empty(b * rows_per_req, heads, 2 * half, dtype=torch.bfloat16, device=pay.device)
    if out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError('xtier_amd.dequantize_context: a contiguous BF16 output expected')
    if req_to_token.dtype != torch.int32 or req_to_token.stride(1) != 1:
        req_to_token = req_to_token.to(torch.int32).contiguous()
    slot_ids = slot_ids if slot_ids.dtype == torch.int64 else slot_ids.to(torch.int64)
    seq_lens = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
    _lib.check(_lib.lib().xt_dequantize_context_nvfp4(
        _ptr(pay), _ptr(sc), pages, heads, 2 * half, block, pay.stride(0), pay.stride(1) if heads > 1 else 0,
        pay.stride(2), sc.stride(0), sc.stride(1) if heads > 1 else 0, sc.stride(2), _ptr(req_to_token),
        req_to_token.stride(0), _ptr(slot_ids), _ptr(seq_lens), b, int(rows_per_req), _ptr(out), _stream(pay)),
        'dequantize_context')
    return out


# --- split-K decode over packed BF16 rows --------------------------------------------------------------------------

def varlen_workspace_bytes(rows, heads, dim, splits):
    return int(_lib.lib().xt_varlen_decode_workspace_bytes(rows, heads, dim, splits))


def varlen_decode(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal=True,
                  out=None, splits=None, ws=None, **_):
    """flash_attn_varlen_func for decode-shaped calls (qsa_decode.py:89-113): one query per row, which sees all of the
    row's packed keys [cu_seqlens_k[r], cu_seqlens_k[r + 1]). q [rows, heads, dim]; k, v [keys, KV heads, dim], BF16.
    Returns out shaped like q (rows it does not name are left as allocated)."""
    if max_seqlen_q != 1:
        raise NotImplementedError('xtier_amd.varlen_decode takes one query per row')
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    _need_cuda(q, k, v, cu_seqlens_q, cu_seqlens_k, out)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError('xtier_amd.varlen_decode: BF16 q, k, v expected')
    rows = cu_seqlens_q.shape[0] - 1
    heads, dim = q.shape[1], q.shape[2]
    kv_heads = k.shape[1]
    if out is None:
        out = torch.empty_like(q)
    if rows <= 0:
        return out
    cu_q, cu_k = (t if t.dtype == torch.int32 else t.to(torch.int32) for t in (cu_seqlens_q, cu_seqlens_k))
    max_k = max(int(max_seqlen_k), 1)
    if splits is None:
        splits = varlen_splits(rows, kv_heads, heads // kv_heads, max_k)
        need = varlen_workspace_bytes(rows, heads, dim, splits)
        if (splits > 1 and ws is None and torch.cuda.is_current_stream_capturing()
                and _cached_workspace_bytes(q.device) < need):
            splits = _narrowed('varlen_decode', splits, 1, need)
    need = varlen_workspace_bytes(rows, heads, dim, splits)
    if ws is None:
        ws = (workspace(q.device, need) if _cached_workspace_bytes(q.device) >= need
              or not torch.cuda.is_current_stream_capturing()
              else torch.empty(need, dtype=torch.uint8, device=q.device))
    _lib.check(_lib.lib().xt_varlen_decode_bf16(
        _ptr(q), q.stride(0), q.stride(1), _ptr(k), k.stride(0), k.stride(1), _ptr(v), v.stride(0), v.stride(1),
        _ptr(cu_q), _ptr(cu_k), rows, heads, kv_heads, dim, max_k, float(softmax_scale), _ptr(out), out.stride(0),
        out.stride(1), _DTYPES[out.dtype], int(splits), _ptr(ws), ws.numel(), _stream(q)), 'varlen_decode')
    return out


# --- sparse MLA ----------------------------------------------------------------------------------------------------

def _mla_cache(raw):
    """(pay u8 [slots, Dl/2], scales u8 [slots, Dl/16], rope BF16 [slots, Dr], g f32 [1]) -> xt_mla_cache, dims."""
    if hasattr(raw, 'raw'):
        raw = raw.raw
    pay, sc, rope, g = raw
    _need_cuda(pay, sc, rope, g)
    if (pay.dtype != torch.uint8 or sc.dtype != torch.uint8 or rope.dtype != torch.bfloat16 or pay.dim() != 2
            or pay.stride(1) != 1 or sc.stride(1) != 1 or rope.stride(1) != 1 or sc.shape[1] * 8 != pay.shape[1]
            or not (pay.shape[0] == sc.shape[0] == rope.shape[0])):
        raise ValueError('xtier_amd.sparse_mla: cache (pay u8 [slots, latent/2], scales u8 [slots, latent/16], '
                         'rope BF16 [slots, rope_dim], g f32 [1]) with packed rows expected')
    g = g if g.dtype == torch.float32 else g.float()
    c = _lib.MlaCache(_ptr(pay), _ptr(sc), _ptr(rope), _ptr(g), pay.shape[0], pay.stride(0), sc.stride(0),
                      rope.stride(0) * 2)
    return c, pay.shape[1] * 2, rope.shape[1], (pay, sc, rope, g)


V4_ROW_BYTES = 584   # a DeepSeek V4 FP8 token: 448 E4M3 + 128 B rope + 8 B scale row


def is_v4_cache(k_cache):
    """A DeepSeek V4 FP8 page view [pages, page_size, 1, 584] of 1-byte elements (sparse_mla.py:156-160)."""
    return torch.is_tensor(k_cache) and k_cache.dim() >= 2 and k_cache.shape[-1] == V4_ROW_BYTES and \
        k_cache.element_size() == 1


def _v4_cache(cache):
    """A V4 page view -> xt_mla_fp8_cache (page stride from the view, as sparse_mla.py:_views takes it)."""
    _need_cuda(cache)
    raw = cache.view(torch.uint8) if cache.dtype != torch.uint8 else cache
    c = _lib.MlaFp8Cache(_ptr(raw), raw.shape[0], raw.shape[1], raw.stride(0))
    return c, raw


def _mla_keys(indices, lengths, rows):
    indices = indices.reshape(rows, -1)
    if indices.dtype != torch.int32 or indices.stride(-1) != 1:
        indices = indices.to(torch.int32).contiguous()
    if lengths is not None:
        lengths = lengths.reshape(rows)
        if lengths.dtype != torch.int32:
            lengths = lengths.to(torch.int32)
        lengths = lengths.contiguous()
    _need_cuda(indices, lengths)
    return _lib.MlaKeys(_ptr(indices), indices.stride(0), indices.shape[1], _ptr(lengths)), (indices, lengths)


def default_mla_splits(rows, topk, v4=False):
    """Key splits per row for sparse MLA: about one workgroup per CU and at least 256 keys per split, and at least
    enough that a split's slot list fits in LDS beside the key and query tiles."""
    fit = math.ceil(topk / _lib.lib().xt_sparse_mla_max_split_keys(int(v4)))
    return min(64, max(1, min(math.ceil(device_cus() / max(1, rows)), max(1, topk // 256), 64), fit))


def mla_workspace_bytes(rows, heads, splits, v4=False):
    if v4:
        return int(_lib.lib().xt_sparse_mla_fp8_workspace_bytes(rows, heads, splits))
    return int(_lib.lib().xt_sparse_mla_workspace_bytes(rows, heads, splits))


def sparse_mla(q, k_cache, indices, topk_length, attn_sink, softmax_scale, extra_k_cache=None, extra_indices=None,
               extra_topk_length=None, out=None, lse=None, splits=None, ws=None):
    """sparse_mla (xtier/packs/deepseek_v4/sparse_mla.py:167-217): q [rows, 1, heads, D] (or [rows, heads, D]) BF16,
    indices [rows, 1, topk] slots of k_cache (-1: none), optional extra_* into a second cache, attn_sink [heads] FP32
    or None. k_cache: DeepSeek V4 FP8 pages [pages, page_size, 1, 584] (D = 512, value = key, the reference's own
    layout), or an NVFP4 latent cache (a LatentPool or (pay, scales, rope, g); D = 576, value = the 512-wide latent).
    Returns (out [rows, 1, heads, 512] BF16, lse [rows, heads, 1] FP32, natural log of the keys' sum) as the reference
    does."""
    shape4 = q.dim() == 4
    if shape4:
        rows, s_q, heads, dim = q.shape
        if s_q != 1:
            raise NotImplementedError(f'xtier_amd.sparse_mla: one query per row expected, not {tuple(q.shape)}')
        q = q.reshape(rows, heads, dim)
    else:
        rows, heads, dim = q.shape
    v4 = is_v4_cache(k_cache)
    if v4:
        cache, keep = _v4_cache(k_cache)
        dl, dr = 512, 0
        if dim != 512:
            raise NotImplementedError(f'xtier_amd.sparse_mla: V4 pages take head dim 512, not {tuple(q.shape)}')
    else:
        cache, dl, dr, keep = _mla_cache(k_cache)
        if dim != dl + dr:
            raise NotImplementedError(f'xtier_amd.sparse_mla: q head size {dim} != latent {dl} + rope {dr}')
    _need_cuda(q, attn_sink, out, lse)
    if q.dtype != torch.bfloat16 or q.stride(-1) != 1:
        q = q.to(torch.bfloat16).contiguous()
    keys, keep_k = _mla_keys(indices, topk_length, rows)
    extra = extra_k_cache is not None and extra_indices is not None
    cache2 = keys2 = None
    if extra:
        if v4 != is_v4_cache(extra_k_cache):
            raise ValueError('xtier_amd.sparse_mla: both caches must have the same format')
        if v4:
            cache2, keep2 = _v4_cache(extra_k_cache)
        else:
            cache2, dl2, dr2, keep2 = _mla_cache(extra_k_cache)
            if (dl2, dr2) != (dl, dr):
                raise ValueError('xtier_amd.sparse_mla: both caches must have the same latent and rope widths')
        keys2, keep_k2 = _mla_keys(extra_indices, extra_topk_length, rows)
    if out is None:
        out = torch.empty((rows, heads, dl), dtype=torch.bfloat16, device=q.device)
    if lse is None:
        lse = torch.empty((rows, heads), dtype=torch.float32, device=q.device)
    if attn_sink is not None and (attn_sink.dtype != torch.float32 or not attn_sink.is_contiguous()):
        attn_sink = attn_sink.float().contiguous()
    topk_all = keys.topk + (keys2.topk if extra else 0)
    if splits is None:
        splits = default_mla_splits(rows, topk_all, v4)
        fewest = default_mla_splits(1 << 20, topk_all, v4)   # the LDS bound alone
        need = mla_workspace_bytes(rows, heads, splits, v4)
        if ws is None and torch.cuda.is_current_stream_capturing() and rows and splits > fewest and \
                _cached_workspace_bytes(q.device) < need:
            splits = _narrowed('sparse_mla', splits, fewest, need)
    need = mla_workspace_bytes(rows, heads, splits, v4)
    if ws is None:
        ws = (workspace(q.device, need) if _cached_workspace_bytes(q.device) >= need
              or not torch.cuda.is_current_stream_capturing()
              else torch.empty(need, dtype=torch.uint8, device=q.device))
    if v4:
        status = _lib.lib().xt_sparse_mla_fp8(
            _ptr(q), q.stride(0), q.stride(1), heads, ctypes.byref(cache), ctypes.byref(keys),
            ctypes.byref(cache2) if extra else None, ctypes.byref(keys2) if extra else None, _ptr(attn_sink),
            float(softmax_scale), _ptr(out), out.stride(0), out.stride(1), _DTYPES[out.dtype], _ptr(lse), rows,
            int(splits), _ptr(ws), ws.numel(), _stream(q))
    else:
        status = _lib.lib().xt_sparse_mla_nvfp4(
            _ptr(q), q.stride(0), q.stride(1), heads, dl, dr, ctypes.byref(cache), ctypes.byref(keys),
            ctypes.byref(cache2) if extra else None, ctypes.byref(keys2) if extra else None, _ptr(attn_sink),
            float(softmax_scale), _ptr(out), out.stride(0), out.stride(1), _DTYPES[out.dtype], _ptr(lse), rows,
            int(splits), _ptr(ws), ws.numel(), _stream(q))
    _lib.check(status, 'sparse_mla')
    return (out.unsqueeze(1), lse.unsqueeze(-1)) if shape4 else (out, lse)


def clock_mhz(device='cuda', iters=20000):
    """The shader clock in MHz while one wavefront runs (xt_clock_probe: core clock ticks over 100 MHz ticks)."""
    out = torch.zeros(3, dtype=torch.int64, device=device)
    _lib.check(_lib.lib().xt_clock_probe(_ptr(out), int(iters), _stream(out)), 'clock_probe')
    core, real, _ = out.tolist()
    return 100.0 * core / real if real > 0 else None


TIMELINE_PHASES = ('entry', 'slot list ready', 'first step computed', 'main loop done', 'slices merged',
                   'partials issued', 'arrival counted', 'split merge done')


def decode_shape(rows, kv_heads, splits, dim=128, shared_lists=True):
    """The decode kernel's launch shape for these sizes, as xt_sparse_decode_nvfp4 derives it: (KV heads per
    workgroup, waves per workgroup, workgroups). 4 KV heads when that alone fills the CUs, else 2, else 1 (per-head
    index lists: 1); 8 waves while the workgroups fit one round on the CUs (head size 256: always 4)."""
    cus = device_cus()
    if not shared_lists:
        hpw = 1
    elif kv_heads % 4 == 0 and rows * (kv_heads // 4) * splits >= cus:
        hpw = 4
    elif kv_heads % 2 == 0 and rows * (kv_heads // 2) * splits >= cus:
        hpw = 2
    else:
        hpw = 1
    units = rows * -(-kv_heads // hpw) * splits
    return hpw, (4 if units > cus or dim == 256 else 8), units


MLA_TIMELINE_PHASES = ('entry', 'slot list ready', 'query ready', 'first key tile ready', 'main loop done',
                       'outputs or partials issued', 'outputs staged (one split)', '(unused)')


class decode_timeline:
    """Per-wave timeline of the decode launches made inside the block (xt_decode_timeline):

        with ops.decode_timeline(max_waves) as tl:
            ops.sparse_decode(...)
        tl.stamps   # int64 [max_waves, 8]: row g * W + w is wave w of workgroup g (W waves per workgroup: 8 for
                    # decode batches that fit one round of workgroups, else 4), column i the 100 MHz clock at
                    # TIMELINE_PHASES[i] of the last launch (0: not reached; rows past the launch's waves: 0)

    kind='mla': the sparse MLA launches instead (xt_mla_timeline; W = 8, phases MLA_TIMELINE_PHASES)."""

    def __init__(self, max_waves, device='cuda', kind='decode'):
        self._buf = torch.zeros(max_waves, len(TIMELINE_PHASES), dtype=torch.int64, device=device)
        self._set = 'xt_mla_timeline' if kind == 'mla' else 'xt_decode_timeline'
        self.stamps = None

    def __enter__(self):
        _lib.check(getattr(_lib.lib(), self._set)(_ptr(self._buf), self._buf.numel() * 8), self._set)
        return self

    def __exit__(self, *exc):
        torch.cuda.synchronize(self._buf.device)
        _lib.check(getattr(_lib.lib(), self._set)(None, 0), self._set)
        self.stamps = self._buf.cpu().numpy()
        return False


def ceiling_mfma(iters, blocks, device='cuda'):
    """The sustained MFMA rate alone (xt_ceiling_mfma): `blocks` x 4 wavefronts x `iters` x 4 independent
    v_mfma_f32_32x32x16_f16 (32768 flops each). Returns the per-thread check values, 64 * iters each."""
    out = torch.empty(int(blocks) * 256, dtype=torch.float32, device=device)
    _lib.check(_lib.lib().xt_ceiling_mfma(_ptr(out), int(iters), int(blocks), _stream(out)), 'ceiling_mfma')
    return out


def ceiling_gather(pool, page_table, indices, page_size, sink=None):
    """The fused decode's HBM access pattern alone (xt_ceiling_gather): pool uint8 [records, record_bytes] (one slot
    record per row, e.g. the interleaved KV pool's 576-byte records), page_table int32 [batch, pages], indices int32
    [batch, topk] positions. Every listed record is read whole and folded by XOR into one word per thread of the
    returned sink."""
    if pool.dtype != torch.uint8 or pool.dim() != 2 or not pool.is_contiguous():
        raise ValueError('xtier_amd.ceiling_gather: pool must be contiguous uint8 [records, record_bytes]')
    page_table, indices = page_table.int().contiguous(), indices.int().contiguous()
    batch, topk = indices.shape
    words = int(_lib.lib().xt_ceiling_gather_sink_words(batch, topk))
    if sink is None or sink.numel() < words:
        sink = torch.empty(max(1, words), dtype=torch.int32, device=pool.device)
    status = _lib.lib().xt_ceiling_gather(_ptr(pool), pool.shape[1], pool.shape[0], _ptr(page_table),
                                          page_table.stride(0), int(page_size), page_table.shape[1], _ptr(indices),
                                          batch, topk, _ptr(sink), _stream(pool))
    _lib.check(status, 'ceiling_gather')
    return sink


def ceiling_gather_pieces(pool, page_table, indices, page_size, splits=2, sink=None):
    """The fused decode's own gather decomposition alone (xt_ceiling_gather_pieces) on the interleaved pool's 576-byte
    records (4 KV heads x D = 128): one workgroup per (row, KV head, key split) reading its head's pieces of every
    key. Returns the sink (512 words per workgroup)."""
    if pool.dtype != torch.uint8 or pool.dim() != 2 or pool.shape[1] != 576 or not pool.is_contiguous():
        raise ValueError('xtier_amd.ceiling_gather_pieces: pool must be contiguous uint8 [records, 576]')
    page_table, indices = page_table.int().contiguous(), indices.int().contiguous()
    batch, topk = indices.shape
    words = batch * 4 * splits * 512
    if sink is None or sink.numel() < words:
        sink = torch.empty(words, dtype=torch.int32, device=pool.device)
    status = _lib.lib().xt_ceiling_gather_pieces(_ptr(pool), pool.shape[0], _ptr(page_table), page_table.stride(0),
                                                 int(page_size), page_table.shape[1], _ptr(indices), batch, topk, 4,
                                                 int(splits), _ptr(sink), _stream(pool))
    _lib.check(status, 'ceiling_gather_pieces')
    return sink


def ceiling_launch(blocks=256, device='cuda'):
    """An empty kernel of `blocks` workgroups of 512 threads (xt_ceiling_launch): the cost of a launch alone."""
    dev = torch.device(device)
    _lib.check(_lib.lib().xt_ceiling_launch(int(blocks), torch.cuda.current_stream(dev).cuda_stream),
               'ceiling_launch')


def ceiling_split_merge(part, counters, out, splits, bytes_per_split, blocks, fenced=False):
    """The decode kernels' split arrival alone (xt_ceiling_split_merge): part uint8 >= blocks * bytes_per_split,
    counters int32 >= blocks / splits (zero before and after), out int32 >= blocks / splits * 512 (the merged sums)."""
    if part.numel() < blocks * bytes_per_split or counters.numel() < blocks // max(1, splits) or \
            out.numel() < blocks // max(1, splits) * 512:
        raise ValueError('xtier_amd.ceiling_split_merge: buffers too small')
    _lib.check(_lib.lib().xt_ceiling_split_merge(_ptr(part), int(bytes_per_split), _ptr(counters), _ptr(out),
                                                 int(splits), int(blocks), int(bool(fenced)), _stream(part)),
               'ceiling_split_merge')


def topk_rows(x, topk, out=None):
    """xt_topk_rows: x FP32 [rows, cols] (unit column stride) -> int32 [rows, topk]: per row the positions of the topk
    largest finite values, ascending, ties toward the lower position, -1 padded."""
    if x.dtype != torch.float32 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError('xtier_amd.topk_rows: x must be float32 [rows, cols] with contiguous rows')
    rows, cols = x.shape
    if out is None:
        out = torch.empty((rows, topk), dtype=torch.int32, device=x.device)
    elif out.dtype != torch.int32 or out.shape != (rows, topk) or out.stride(1) != 1:
        raise ValueError('xtier_amd.topk_rows: out must be int32 [rows, topk] with contiguous rows')
    _lib.check(_lib.lib().xt_topk_rows(_ptr(x), x.stride(0), rows, cols, int(topk), _ptr(out), out.stride(0),
                                       _stream(x)), 'topk_rows')
    return out


def qsa_indexer_logits(q, k, row_starts, row_ends, score_scale=None):
    """The QSA indexer logits (qsa_prefill.py:77-102, with SGLang's mask): q [rows, heads, dim] and k [keys, 1, dim]
    (or [keys, dim]) BF16 / FP16, row_starts / row_ends [rows] -> FP32 [rows, keys]: sum_h ReLU(q . k) / score_scale
    (default sqrt(dim)) inside [start, end), -inf outside."""
    if k.dim() == 3:
        k = k[:, 0]
    rows, heads, dim = q.shape
    keys = k.shape[0]
    if q.dtype not in _DTYPES or k.dtype != q.dtype:
        raise ValueError('xtier_amd.qsa_indexer_logits: q and k must both be BF16 or both FP16')
    if q.stride(-1) != 1 or k.stride(-1) != 1:
        raise ValueError('xtier_amd.qsa_indexer_logits: q and k need a contiguous last dimension')
    starts = row_starts.to(device=q.device, dtype=torch.int32).contiguous()
    ends = row_ends.to(device=q.device, dtype=torch.int32).contiguous()
    logits = torch.empty((rows, keys), dtype=torch.float32, device=q.device)
    scale = float(score_scale or math.sqrt(dim))
    status = _lib.lib().xt_qsa_indexer_logits(_ptr(q), q.stride(0), q.stride(1), rows, heads, dim, _ptr(k), k.stride(0),
                                              keys, _ptr(starts), _ptr(ends), scale, _DTYPES[q.dtype], _ptr(logits),
                                              logits.stride(0), _stream(q))
    _lib.check(status, 'qsa_indexer_logits')
    return logits


def _fp8(t, what):
    if t.dtype == torch.float8_e4m3fn:
        return t
    if t.dtype == torch.uint8:
        return t.view(torch.float8_e4m3fn)
    raise ValueError(f'xtier_amd.{what}: FP8 E4M3 tensors expected, not {t.dtype}')


def dsa_mqa_logits(q_fp8, kv, weights, ks, ke, clean_logits=False, max_seqlen_k=0):
    """fp8_mqa_logits (indexer_torch.py:28-45): q [num_q, heads, dim] E4M3, kv = (k [num_kv, dim] E4M3, k_scale
    [num_kv] FP32), weights [num_q, heads], ks / ke [num_q] -> FP32 [num_q, num_kv], a view of rows padded to a
    multiple of 4 columns (the stride SGLang's top-k expects): sum_h w ReLU(q_h . k) * k_scale inside [ks, ke), 0
    (or -inf when clean_logits) elsewhere."""
    k_fp8, k_scale = kv
    q_fp8, k_fp8 = _fp8(q_fp8, 'dsa_mqa_logits'), _fp8(k_fp8, 'dsa_mqa_logits')
    num_q, heads, dim = q_fp8.shape
    num_kv = k_fp8.shape[0]
    k2 = k_fp8.reshape(num_kv, dim)
    if q_fp8.stride(-1) != 1 or k2.stride(-1) != 1:
        raise ValueError('xtier_amd.dsa_mqa_logits: q and k need a contiguous last dimension')
    w = weights.float().contiguous()
    sc = k_scale.reshape(num_kv).float().contiguous()
    storage = torch.zeros(num_q, (num_kv + 3) // 4 * 4, dtype=torch.float32, device=q_fp8.device)
    ks32 = ks.to(device=q_fp8.device, dtype=torch.int32).contiguous()
    ke32 = ke.to(device=q_fp8.device, dtype=torch.int32).contiguous()
    status = _lib.lib().xt_dsa_mqa_logits(_ptr(q_fp8), q_fp8.stride(0), q_fp8.stride(1), num_q, heads, dim, _ptr(k2),
                                          k2.stride(0), _ptr(sc), num_kv, _ptr(w), w.stride(0), _ptr(ks32), _ptr(ke32),
                                          int(bool(clean_logits)), _ptr(storage), storage.stride(0), _stream(q_fp8))
    _lib.check(status, 'dsa_mqa_logits')
    return storage[:, :num_kv]


def dsa_paged_mqa_logits(q_fp8, kvcache_fp8, weights, context_lens, block_table, schedule_metadata, max_seq_len,
                         clean_logits=False, indices=None):
    """fp8_paged_mqa_logits (indexer_torch.py:48-72): q [batch, 1, heads, dim] E4M3, the paged cache [pages, block, 1,
    dim + 4] bytes (block x dim E4M3 values, then block FP32 scales per page), weights [batch, heads], context_lens
    [batch] (or [batch, 1]), block_table [batch, pages] -> FP32 [batch, max_seq_len]."""
    if indices is not None:
        raise NotImplementedError('xtier_amd.dsa_paged_mqa_logits: no index tensor is taken')
    if context_lens.dim() == 2:
        if context_lens.shape[1] != 1:
            raise NotImplementedError('xtier_amd.dsa_paged_mqa_logits: one query per row (next_n 1)')
        context_lens = context_lens[:, 0]
    q = _fp8(q_fp8, 'dsa_paged_mqa_logits')
    batch, _, heads, dim = q.shape
    block = kvcache_fp8.shape[1]
    cache = kvcache_fp8.view(torch.uint8) if kvcache_fp8.dtype != torch.uint8 else kvcache_fp8
    page_bytes = cache.stride(0) * cache.element_size()
    w = weights.float().contiguous()
    lens = context_lens.to(device=q.device, dtype=torch.int32).contiguous()
    table = block_table.to(device=q.device, dtype=torch.int32).contiguous()
    out = torch.empty((batch, int(max_seq_len)), dtype=torch.float32, device=q.device)
    status = _lib.lib().xt_dsa_paged_mqa_logits(_ptr(q), q.stride(0), q.stride(2), batch, heads, dim, _ptr(cache),
                                                cache.shape[0], page_bytes, block, _ptr(table), table.stride(0), table.shape[1],
                                                _ptr(lens), _ptr(w), w.stride(0), int(max_seq_len),
                                                int(bool(clean_logits)), _ptr(out), out.stride(0), _stream(q))
    _lib.check(status, 'dsa_paged_mqa_logits')
    return out


_SCORE_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _f32(x):
    return ctypes.c_float(float(x)).value


def minimax_score_factor(sm_scale, k_scale):
    """The FP32 factor of the MiniMax index scores, formed as the reference's kernels form it:
    (sm_scale * 1.4426950409) * k_scale, each product rounded to FP32 (kv_fp4.py:181, :208)."""
    return _f32(_f32(_f32(sm_scale) * _f32(1.4426950409)) * _f32(k_scale))


def _index_bits(*arrays):
    """The index_int64 mask of the block-score entry points: bit i set when array i is int64 (else int32)."""
    bits = 0
    for i, t in enumerate(arrays):
        if t is None:
            continue
        if t.dtype == torch.int64:
            bits |= 1 << i
        elif t.dtype != torch.int32:
            raise ValueError(f'xtier_amd.minimax scores: index arrays are int32 or int64, got {t.dtype}')
    return bits


def _index_pool(pay, sc, what):
    """The MiniMax index pool views: payload [pages, 128, dim/2] and scale bytes [pages, 128, dim/16], unit stride
    within a slot row."""
    sc = sc.view(torch.uint8) if sc.dtype != torch.uint8 else sc
    pay = pay.view(torch.uint8) if pay.dtype != torch.uint8 else pay
    if (pay.dim() != 3 or sc.dim() != 3 or pay.shape[:2] != sc.shape[:2] or pay.shape[1] != 128
            or pay.stride(2) != 1 or sc.stride(2) != 1 or sc.shape[2] * 8 != pay.shape[2]):
        raise ValueError(f'xtier_amd.{what}: index pool views [pages, 128, dim/2] and [pages, 128, dim/16] expected, '
                         f'got {tuple(pay.shape)} and {tuple(sc.shape)}')
    _need_cuda(pay, sc)
    return pay, sc


def minimax_decode_scores(q, idx_pay, idx_sc, req_to_token, score, seq_lens, slot_ids, block_size, sm_scale, k_scale,
                          init_blocks, local_blocks, score_type='max', skip_topk=None, heads=None, batch=None,
                          q_strides=None, r2t_stride=None, score_strides=None):
    """The MiniMax decode index scores (_fp4_decode_score_kernel, kv_fp4.py:168-222) into ``score``
    [heads, batch, blocks] (FP32 / BF16 / FP16): q [batch, heads, dim] BF16 / FP16 against the NVFP4 index pool.
    Strides default to the tensors' own; ``skip_topk``: requests with at most that many blocks get no scores."""
    pay, sc = _index_pool(idx_pay, idx_sc, 'minimax_decode_scores')
    if q.dtype not in _DTYPES or score.dtype not in _SCORE_DTYPES:
        raise ValueError('xtier_amd.minimax_decode_scores: BF16 / FP16 queries and FP32 / BF16 / FP16 scores')
    if score_type not in ('max', 'lse'):
        raise ValueError(f'xtier_amd.minimax_decode_scores: score_type {score_type!r} (max or lse)')
    _need_cuda(q, req_to_token, score, seq_lens, slot_ids)
    batch = q.shape[0] if batch is None else int(batch)
    dim = q.shape[2]
    heads = q.shape[1] if heads is None else int(heads)
    sq = q_strides or q.stride()
    if sq[2] != 1:
        raise ValueError('xtier_amd.minimax_decode_scores: the query head dimension must be contiguous')
    ss = score_strides or score.stride()
    hint = -(-req_to_token.shape[1] // int(block_size))
    status = _lib.lib().xt_minimax_decode_scores(
        _ptr(q), sq[0], sq[1], batch, heads, dim, _DTYPES[q.dtype], _ptr(pay), pay.stride(0), pay.stride(1), _ptr(sc),
        sc.stride(0), sc.stride(1), pay.shape[0] * 128, _ptr(req_to_token),
        req_to_token.stride(0) if r2t_stride is None else r2t_stride, _ptr(seq_lens), _ptr(slot_ids),
        _index_bits(req_to_token, seq_lens, slot_ids), int(block_size), minimax_score_factor(sm_scale, k_scale),
        int(init_blocks), int(local_blocks), -1 if skip_topk is None else int(skip_topk), int(score_type == 'lse'),
        _ptr(score), _SCORE_DTYPES[score.dtype], ss[0], ss[1], ss[2], hint, _stream(q))
    _lib.check(status, 'minimax_decode_scores')
    return score


def minimax_prefill_scores(q, idx_pay, idx_sc, req_to_token, score, cu_seqlens, seq_lens, prefix_lens, slot_ids,
                           block_size, sm_scale, k_scale, max_q_len, heads=None, q_strides=None, r2t_stride=None,
                           score_strides=None):
    """The MiniMax prefill index scores (_fp4_index_score_kernel, kv_fp4.py:407-446) into ``score``
    [heads, total_q, blocks]: q [total_q, heads, dim] BF16 / FP16; causal, each row's blocks bounded by its 64-row
    tile. ``max_q_len`` bounds every request's query count."""
    pay, sc = _index_pool(idx_pay, idx_sc, 'minimax_prefill_scores')
    if q.dtype not in _DTYPES or score.dtype not in _SCORE_DTYPES:
        raise ValueError('xtier_amd.minimax_prefill_scores: BF16 / FP16 queries and FP32 / BF16 / FP16 scores')
    _need_cuda(q, req_to_token, score, cu_seqlens, seq_lens, prefix_lens, slot_ids)
    dim = q.shape[2]
    heads = q.shape[1] if heads is None else int(heads)
    sq = q_strides or q.stride()
    if sq[2] != 1:
        raise ValueError('xtier_amd.minimax_prefill_scores: the query head dimension must be contiguous')
    ss = score_strides or score.stride()
    status = _lib.lib().xt_minimax_prefill_scores(
        _ptr(q), sq[0], sq[1], cu_seqlens.shape[0] - 1, heads, dim, _DTYPES[q.dtype], int(max_q_len), _ptr(pay),
        pay.stride(0), pay.stride(1), _ptr(sc), sc.stride(0), sc.stride(1), pay.shape[0] * 128, _ptr(req_to_token),
        req_to_token.stride(0) if r2t_stride is None else r2t_stride, _ptr(cu_seqlens), _ptr(seq_lens),
        _ptr(prefix_lens), _ptr(slot_ids), _index_bits(req_to_token, seq_lens, slot_ids, prefix_lens, cu_seqlens),
        int(block_size), minimax_score_factor(sm_scale, k_scale), _ptr(score), _SCORE_DTYPES[score.dtype], ss[0],
        ss[1], ss[2], _stream(q))
    _lib.check(status, 'minimax_prefill_scores')
    return score
