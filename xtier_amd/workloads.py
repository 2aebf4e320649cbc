"""Seeded synthetic inputs for the sparse-attention workloads (bf16 activations, NVFP4 paged KV pools, page tables
and top-k index lists), generated with torch on any device from a torch.Generator.

Generators (the same rules for every workload):
- K/V and latents: bf16 N(0, 1) with round(1% of heads * dim) channels (at least one) multiplied by 8, chosen once
  per tensor;
- the global scale of a tensor is amax / (6 * 448) (NVFP4 with its own amax);
- page tables: each request owns ctx / page pages of the pool, in a random permutation;
- index lists: unique positions, sorted, int32.
"""
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class DecodeWorkload:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    dim: int
    ctx: int
    topk: int
    page: int = 64
    index_mode: str = 'uniform'     # 'uniform' | 'recent_half'
    q_std: float = 1.0

    @property
    def slots(self):
        return self.batch * self.ctx

    def algorithmic_bytes(self):
        """Gathered KV payload plus scales: batch * topk * kv_heads * 2 * (dim/2 + dim/16)."""
        return self.batch * self.topk * self.kv_heads * 2 * (self.dim // 2 + self.dim // 16)

    def flops(self):
        return self.batch * self.q_heads * self.topk * 4 * self.dim


WORKLOADS = {
    # 1 request, 8 q heads / 1 KV head, d 128, context 4096, top-512 uniform (the CPU-reference case)
    'cpu_ref_decode': DecodeWorkload('cpu_ref_decode', 1, 8, 1, 128, 4096, 512),
    # batch 32, 32 q / 4 KV heads, d 128, context 32768, top-2048 sorted unique per request, page 64
    'gqa_decode_b32': DecodeWorkload('gqa_decode_b32', 32, 32, 4, 128, 32768, 2048),
    # batch 4, context 524288, top-2048: half from the last 4096 tokens, half uniform over the rest
    'long_ctx_decode_b4': DecodeWorkload('long_ctx_decode_b4', 4, 32, 4, 128, 524288, 2048,
                                         index_mode='recent_half'),
}


@dataclass(frozen=True)
class PrefillWorkload:
    """One request: `chunk` new tokens appended after `ctx0` context tokens; query t (position ctx0 + t) attends to
    its own top-k causal positions (the `recent` most recent, itself included, plus uniform ones below them); the step
    also quantizes the chunk's K/V rows into the pool."""
    name: str
    q_heads: int
    kv_heads: int
    dim: int
    ctx0: int
    chunk: int
    topk: int
    recent: int = 128
    page: int = 64

    @property
    def ctx(self):
        return self.ctx0 + self.chunk

    @property
    def slots(self):
        return self.ctx

    def algorithmic_bytes(self):
        """Gathered KV payload plus scales over all queries (most are cache hits: the unique set is the pool)."""
        return self.chunk * self.topk * self.kv_heads * 2 * (self.dim // 2 + self.dim // 16)

    def flops(self):
        return self.chunk * self.q_heads * self.topk * 4 * self.dim


PREFILL_WORKLOADS = {
    # 4096 query tokens appended at 65536 (context 69632), 32 q / 4 KV heads, d 128, top-2048 causal per query
    'gqa_prefill_chunk4096': PrefillWorkload('gqa_prefill_chunk4096', 32, 4, 128, 65536, 4096, 2048),
}


@dataclass(frozen=True)
class MlaWorkload:
    """Sparse MLA, DeepSeek-style: `heads` query heads share one latent key per token (latent NVFP4 + rope BF16).
    Decode: `rows` requests, one query each, top-k uniform over the request's context. Prefill (causal): one request,
    the last `rows` positions of its context as queries, each with its own causal top-k (the `recent` most recent
    included)."""
    name: str
    rows: int
    heads: int
    ctx: int
    topk: int
    causal: bool = False
    latent: int = 512
    rope: int = 64
    q_std: float = 0.5
    recent: int = 128
    page: int = 64
    fmt: str = 'nvfp4'          # 'nvfp4' (latent + rope, value = latent) or 'fp8_v4' (DeepSeek V4 pages, value = key)

    @property
    def requests(self):
        return 1 if self.causal else self.rows

    @property
    def slots(self):
        return self.requests * self.ctx

    def algorithmic_bytes(self):
        """Gathered key bytes: NVFP4, rows * topk * (latent/2 + latent/16 + 2 * rope); V4, rows * topk * (448 E4M3 +
        7 scale bytes + 128 rope bytes)."""
        if self.fmt == 'fp8_v4':
            return self.rows * self.topk * (448 + 7 + 128)
        return self.rows * self.topk * (self.latent // 2 + self.latent // 16 + 2 * self.rope)

    def flops(self):
        """q.k over the key and p.v over the value: NVFP4 rows * heads * topk * (2 (Dl + Dr) + 2 Dl); V4 (key = value
        = 512 wide) rows * heads * topk * 4 * 512."""
        if self.fmt == 'fp8_v4':
            return self.rows * self.heads * self.topk * 4 * 512
        return self.rows * self.heads * self.topk * (2 * (self.latent + self.rope) + 2 * self.latent)


MLA_WORKLOADS = {
    # 64 requests decoding at context 131072, 128 heads, top-2048 uniform
    'mla_decode_b64': MlaWorkload('mla_decode_b64', 64, 128, 131072, 2048),
    # a 2048-token prefill chunk at the end of a 131072-token context, top-2048 causal per query
    'mla_prefill_2048': MlaWorkload('mla_prefill_2048', 2048, 128, 131072, 2048, causal=True),
    # the decode workload on DeepSeek V4 FP8 pages (pages of 64 tokens)
    'mla_v4_decode_b64': MlaWorkload('mla_v4_decode_b64', 64, 128, 131072, 2048, fmt='fp8_v4'),
}


@dataclass(frozen=True)
class BlockDecodeWorkload:
    """Block-sparse decode over head-major NVFP4 pages (the MiniMax cache layout): each (request, KV head) attends to
    `topk_blocks` distinct blocks of `block` tokens of its context (one block = one page row range), chosen uniformly
    per KV head; the pool has a unit global scale."""
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    dim: int
    ctx: int
    topk_blocks: int
    block: int = 128
    q_std: float = 1.0

    @property
    def pages(self):
        return self.batch * (self.ctx // self.block)

    @property
    def keys(self):
        return self.topk_blocks * self.block

    def algorithmic_bytes(self):
        """Read KV payload plus scales: batch * kv_heads * keys * 2 * (dim/2 + dim/16)."""
        return self.batch * self.kv_heads * self.keys * 2 * (self.dim // 2 + self.dim // 16)

    def flops(self):
        return self.batch * self.q_heads * self.keys * 4 * self.dim


BLOCK_WORKLOADS = {
    # batch 32, 64 q / 4 KV heads, d 128, context 32768, 16 blocks of 128 tokens per KV head (2048 keys)
    'minimax_decode_b32': BlockDecodeWorkload('minimax_decode_b32', 32, 64, 4, 128, 32768, 16),
}


@dataclass(frozen=True)
class BlockPrefillWorkload:
    """Causal block-sparse prefill over head-major NVFP4 pages (the MiniMax cache layout): one request appends a chunk
    of `q_len` queries after `prefix` tokens; each query (query blocks of one, as the NVFP4 prefill runs them) and KV
    head lists `topk_blocks` blocks of `block` tokens: its own block and topk_blocks - 1 distinct earlier ones."""
    name: str
    q_len: int
    prefix: int
    q_heads: int
    kv_heads: int
    dim: int
    topk_blocks: int
    block: int = 128

    @property
    def ctx(self):
        return self.prefix + self.q_len

    @property
    def pages(self):
        return self.ctx // self.block

    def algorithmic_bytes(self):
        """KV payload plus scales the queries read, counting whole listed blocks: q_len * kv_heads * topk_blocks *
        block * 2 * (dim/2 + dim/16)."""
        return self.q_len * self.kv_heads * self.topk_blocks * self.block * 2 * (self.dim // 2 + self.dim // 16)

    def flops(self):
        return self.q_len * self.q_heads * self.topk_blocks * self.block * 4 * self.dim

    def copy_bytes(self):
        """The BF16 context copy of main K, V (kv_heads) and index K (one head): per token read dim/2 + dim/16 and
        write 2 * dim bytes per head."""
        return self.ctx * (2 * self.kv_heads + 1) * (self.dim // 2 + self.dim // 16 + 2 * self.dim)


BLOCK_PREFILL_WORKLOADS = {
    # a 4096-query chunk after 61440 tokens (context 65536), 64 q / 4 KV heads, d 128, 16 blocks of 128 per query
    'minimax_prefill_chunk4096': BlockPrefillWorkload('minimax_prefill_chunk4096', 4096, 61440, 64, 4, 128, 16),
}


@dataclass(frozen=True)
class VarlenWorkload:
    """Decode over packed BF16 rows (the gathered top-k rows of every request, one query per row)."""
    name: str
    rows: int
    q_heads: int
    kv_heads: int
    dim: int
    keys: int

    def algorithmic_bytes(self):
        """K and V rows read: rows * keys * kv_heads * 2 * dim * 2 bytes."""
        return self.rows * self.keys * self.kv_heads * 2 * self.dim * 2

    def flops(self):
        return self.rows * self.q_heads * self.keys * 4 * self.dim


VARLEN_WORKLOADS = {
    # 32 rows, 32 q / 4 KV heads, d 128, 2048 packed keys per row (the gathered top-2048 of the decode workload)
    'qsa_varlen_b32': VarlenWorkload('qsa_varlen_b32', 32, 32, 4, 128, 2048),
}


def generator(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def kv_tensor(n, heads, dim, gen, device, outlier_frac=0.01, outlier_scale=8.0):
    """bf16 [n, heads, dim] N(0, 1) with round(outlier_frac * heads * dim) channels (>= 1) scaled by outlier_scale."""
    x = torch.randn(n, heads, dim, generator=gen, device=device, dtype=torch.float32)
    channels = heads * dim
    k = max(1, round(outlier_frac * channels))
    pick = torch.randperm(channels, generator=gen, device=device)[:k]
    scale = torch.ones(channels, device=device)
    scale[pick] = outlier_scale
    x.mul_(scale.view(1, heads, dim))
    return x.to(torch.bfloat16)


def page_table(batch, ctx, page, gen, device):
    """int32 [batch, ctx/page]: every request's pages, the pool's pages in a random order."""
    n_pages = batch * (ctx // page)
    return torch.randperm(n_pages, generator=gen, device=device).to(torch.int32).view(batch, ctx // page)


def token_table(pt, page):
    """The token-granular form of a page table (SGLang's req_to_token): int32 [batch, ctx]."""
    batch, pages = pt.shape
    off = torch.arange(page, device=pt.device, dtype=torch.int32)
    return (pt[:, :, None] * page + off[None, None, :]).reshape(batch, pages * page)


def index_lists(batch, ctx, topk, gen, device, mode='uniform'):
    """int32 [batch, topk] sorted unique positions below ctx."""
    out = torch.empty(batch, topk, dtype=torch.int32, device=device)
    for b in range(batch):
        if mode == 'uniform':
            pick = torch.randperm(ctx, generator=gen, device=device)[:topk]
        elif mode == 'recent_half':
            recent = min(4096, ctx)
            half = topk // 2
            a = ctx - recent + torch.randperm(recent, generator=gen, device=device)[:half]
            rest = torch.randperm(ctx - recent, generator=gen, device=device)[:topk - half]
            pick = torch.cat([rest, a])
        else:
            raise ValueError(mode)
        out[b] = torch.sort(pick).values.to(torch.int32)
    return out


def causal_index_lists(q_positions, topk, recent, gen, device):
    """Per query position p: the `recent` most recent positions (p-recent+1 .. p) and topk-recent uniform ones below
    p-recent+1, sorted; int32 [n, topk]."""
    n = q_positions.numel()
    out = torch.empty(n, topk, dtype=torch.int32, device=device)
    for i, p in enumerate(q_positions.tolist()):
        lo = p - recent + 1
        far = torch.randperm(lo, generator=gen, device=device)[:topk - recent]
        near = torch.arange(lo, p + 1, device=device)
        out[i] = torch.sort(torch.cat([far, near])).values.to(torch.int32)
    return out


@dataclass
class DecodeInputs:
    workload: DecodeWorkload
    q: torch.Tensor            # bf16 [batch, q_heads, dim]
    k: torch.Tensor            # bf16 [slots, kv_heads, dim] (None when not kept)
    v: torch.Tensor
    page_table: torch.Tensor   # int32 [batch, ctx/page]
    indices: torch.Tensor      # int32 [batch, topk]
    seq_lens: torch.Tensor     # int32 [batch]


def decode_inputs(w, seed, device='cpu', batch=None):
    """Seeded activations and index lists of a decode workload (optionally with fewer requests)."""
    b = w.batch if batch is None else batch
    gen = generator(device, seed)
    slots = b * w.ctx
    k = kv_tensor(slots, w.kv_heads, w.dim, gen, device)
    v = kv_tensor(slots, w.kv_heads, w.dim, gen, device)
    q = (torch.randn(b, w.q_heads, w.dim, generator=gen, device=device) * w.q_std).to(torch.bfloat16)
    pt = page_table(b, w.ctx, w.page, gen, device)
    idx = index_lists(b, w.ctx, w.topk, gen, device, w.index_mode)
    seq = torch.full((b,), w.ctx, dtype=torch.int32, device=device)
    return DecodeInputs(w, q, k, v, pt, idx, seq)


@dataclass
class PrefillInputs:
    workload: PrefillWorkload
    q: torch.Tensor            # bf16 [chunk, q_heads, dim]
    k: torch.Tensor            # bf16 [ctx, kv_heads, dim]: context rows then the chunk's rows
    v: torch.Tensor
    page_table: torch.Tensor   # int32 [1, ctx/page]
    indices: torch.Tensor      # int32 [chunk, topk]
    q_pos: torch.Tensor        # int32 [chunk]: ctx0 + t


def prefill_inputs(w, seed, device='cpu'):
    """Seeded activations, page table and per-query causal index lists of a prefill workload."""
    gen = generator(device, seed)
    k = kv_tensor(w.ctx, w.kv_heads, w.dim, gen, device)
    v = kv_tensor(w.ctx, w.kv_heads, w.dim, gen, device)
    q = torch.randn(w.chunk, w.q_heads, w.dim, generator=gen, device=device).to(torch.bfloat16)
    pt = page_table(1, w.ctx, w.page, gen, device)
    q_pos = torch.arange(w.ctx0, w.ctx, dtype=torch.int32, device=device)
    idx = causal_index_lists(q_pos, w.topk, w.recent, gen, device)
    return PrefillInputs(w, q, k, v, pt, idx, q_pos)


@dataclass
class MlaInputs:
    workload: MlaWorkload
    q: torch.Tensor            # bf16 [rows, heads, latent + rope]
    slots: torch.Tensor        # int32 [rows, topk]: cache slots of each row's keys
    positions: torch.Tensor    # int32 [rows, topk]: their positions in the request's context


def mla_cache_rows(w, gen, device, start, n):
    """Latent BF16 [n, latent] (N(0,1), 1% outlier channels x8) and rope BF16 [n, rope] (N(0,1)) for cache rows
    start .. start+n-1 of a workload's pool (generated in order from `gen`)."""
    lat = kv_tensor(n, 1, w.latent, gen, device).view(n, w.latent)
    rope = torch.randn(n, w.rope, generator=gen, device=device).to(torch.bfloat16)
    return lat, rope


def mla_inputs(w, seed, device='cpu'):
    """Seeded queries and key lists of an MLA workload (the cache rows come from mla_cache_rows)."""
    gen = generator(device, seed)
    dim = 512 if w.fmt == 'fp8_v4' else w.latent + w.rope
    q = (torch.randn(w.rows, w.heads, dim, generator=gen, device=device) * w.q_std).to(torch.bfloat16)
    pt = page_table(w.requests, w.ctx, w.page, gen, device)
    if w.causal:
        q_pos = torch.arange(w.ctx - w.rows, w.ctx, dtype=torch.int32, device=device)
        pos = causal_index_lists(q_pos, w.topk, w.recent, gen, device)
        req = torch.zeros(w.rows, dtype=torch.long, device=device)
    else:
        pos = index_lists(w.rows, w.ctx, w.topk, gen, device)
        req = torch.arange(w.rows, device=device)
    slots = (pt[req[:, None], (pos // w.page).long()].long() * w.page + pos % w.page).to(torch.int32)
    return MlaInputs(w, q, slots, pos)


@dataclass
class BlockDecodeInputs:
    workload: BlockDecodeWorkload
    q: torch.Tensor            # bf16 [batch, q_heads, dim]
    req_to_token: torch.Tensor  # int32 [batch, ctx]: block-aligned page rows, pages in a random order
    slot_ids: torch.Tensor     # int64 [batch]
    topk_idx: torch.Tensor     # int32 [kv_heads, batch, topk_blocks]: sorted distinct block ids
    seq_lens: torch.Tensor     # int32 [batch]


def block_decode_inputs(w, seed, device='cpu', batch=None):
    """Seeded queries, request tables and per-KV-head block lists of a block-sparse decode workload."""
    b = w.batch if batch is None else batch
    gen = generator(device, seed)
    q = (torch.randn(b, w.q_heads, w.dim, generator=gen, device=device) * w.q_std).to(torch.bfloat16)
    pt = page_table(b, w.ctx, w.block, gen, device)
    r2t = token_table(pt, w.block)
    nb = w.ctx // w.block
    idx = torch.empty(w.kv_heads, b, w.topk_blocks, dtype=torch.int32, device=device)
    for h in range(w.kv_heads):
        for r in range(b):
            idx[h, r] = torch.sort(torch.randperm(nb, generator=gen, device=device)[:w.topk_blocks]).values
    seq = torch.full((b,), w.ctx, dtype=torch.int32, device=device)
    return BlockDecodeInputs(w, q, r2t, torch.arange(b, dtype=torch.int64, device=device), idx, seq)


@dataclass
class BlockPrefillInputs:
    workload: BlockPrefillWorkload
    q: torch.Tensor            # bf16 [q_len, q_heads, dim]
    req_to_token: torch.Tensor  # int32 [1, ctx]: pages of `block` tokens in a random order
    slot_ids: torch.Tensor     # int64 [1]
    topk_idx: torch.Tensor     # int32 [kv_heads, q_len, topk_blocks]: the query's block first, then earlier ones
    cu_seqlens: torch.Tensor   # int32 [2]
    seq_lens: torch.Tensor     # int32 [1]
    prefix_lens: torch.Tensor  # int32 [1]


def block_prefill_inputs(w, seed, device='cpu'):
    """Seeded queries, a token table over the pool's pages in a random order (as a page allocator hands them out), and
    per-(KV head, query) block lists."""
    gen = generator(device, seed)
    q = torch.randn(w.q_len, w.q_heads, w.dim, generator=gen, device=device).to(torch.bfloat16)
    r2t = token_table(page_table(1, w.ctx, w.block, gen, device), w.block)
    own = (w.prefix + torch.arange(w.q_len, device=device)) // w.block
    nb = w.ctx // w.block
    score = torch.rand(w.kv_heads, w.q_len, nb, generator=gen, device=device)
    score = torch.where(torch.arange(nb, device=device)[None, None, :] < own[None, :, None], score, -1.0)
    far = torch.topk(score, w.topk_blocks - 1, dim=2).indices
    idx = torch.cat([own[None, :, None].expand(w.kv_heads, -1, 1), far], dim=2).to(torch.int32).contiguous()
    i32 = lambda v: torch.tensor(v, dtype=torch.int32, device=device)
    return BlockPrefillInputs(w, q, r2t, torch.zeros(1, dtype=torch.int64, device=device), idx, i32([0, w.q_len]),
                              i32([w.ctx]), i32([w.prefix]))


def head_major_pages(x_pay, x_sc, block):
    """Token-major pool bytes [slots, heads, n] (slot = page * block + row) -> head-major pages [pages, heads, block,
    n] (the MiniMax cache layout)."""
    slots, heads, n = x_pay.shape
    pay = x_pay.view(slots // block, block, heads, n).permute(0, 2, 1, 3).contiguous()
    m = x_sc.shape[2]
    sc = x_sc.view(slots // block, block, heads, m).permute(0, 2, 1, 3).contiguous()
    return pay, sc


def v4_pages(tokens, page_size, gen, device):
    """DeepSeek V4 FP8 pages [pages, page_size, 1, 584] of random valid content: E4M3 bytes other than NaN, UE8M0
    exponents 120 .. 130 (scales 2^-7 .. 2^3), BF16 N(0, 1) rope values."""
    pages = tokens // page_size
    buf = torch.randint(0, 256, (pages, page_size * 584), generator=gen, device=device, dtype=torch.uint8)
    data = buf[:, :page_size * 576].view(pages, page_size, 576)
    nope = data[..., :448]
    nope.copy_(torch.where((nope & 0x7F) == 0x7F, nope ^ 1, nope))
    rope = torch.randn(pages, page_size, 64, generator=gen, device=device).to(torch.bfloat16)
    data[..., 448:] = rope.view(torch.uint8).view(pages, page_size, 128)
    sc = buf[:, page_size * 576:].view(pages, page_size, 8)
    sc.copy_(torch.randint(120, 131, (pages, page_size, 8), generator=gen, device=device, dtype=torch.uint8))
    sc[..., 7] = 0
    return buf.as_strided((pages, page_size, 1, 584), (page_size * 584, 584, 584, 1))
