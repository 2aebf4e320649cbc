"""A layer's paged NVFP4 KV pool in HBM, in either of two layouts:

- 'interleaved' (this library's layout): one uint8 buffer [slots, 2 * heads * (dim/2 + dim/16)]. Each slot holds, per
  KV head, the head's K payload row then its V payload row, and after them, per KV head, its K scales then its V
  scales. A key's K and V (576 bytes at 4 heads x 128) are one contiguous record, so a sparse gather reads one burst
  per key instead of four scattered ones, and the K and V payload of one head (128 bytes) sit side by side, where one
  workgroup reads both.
- 'split': SGLang's NVFP4 pool buffers (xtier/packs/qwen4_exp/qsa_fp4.py:43-58): k, v uint8 [slots, heads, dim/2] and
  k_sf, v_sf uint8 [slots, heads, dim/16], each contiguous.

Either way ``raw`` is the reference's tuple (k_pay, v_pay, k_scales, v_scales, gk, gv), the payload and scale entries
being uint8 views [slots, heads, width] with strided slots and heads. The decode, prefill and quantize entry points
of xtier_amd.ops take both layouts; the QSA gather and pack keep the reference's packed-buffer precondition.
"""
import torch

from . import ops


class KVPool:
    def __init__(self, slots, kv_heads, dim, device='cuda', layout='interleaved', gk=None, gv=None):
        if dim % 32 or dim & (dim - 1):
            raise ValueError(f'head size {dim}: a power of 2, multiple of 32 expected')
        self.slots, self.kv_heads, self.dim, self.layout = slots, kv_heads, dim, layout
        half, blocks = kv_heads * dim // 2, kv_heads * dim // 16
        device = torch.device(device)
        if layout == 'interleaved':
            self.buffer = torch.zeros(slots, 2 * (half + blocks), dtype=torch.uint8, device=device)
            pay = self.buffer[:, :2 * half].unflatten(1, (kv_heads, dim))        # per head [K row | V row]
            sf = self.buffer[:, 2 * half:].unflatten(1, (kv_heads, dim // 8))    # per head [K scales | V scales]
            self.k_pay, self.v_pay = pay[:, :, :dim // 2], pay[:, :, dim // 2:]
            self.k_sf, self.v_sf = sf[:, :, :dim // 16], sf[:, :, dim // 16:]
        elif layout == 'split':
            self.buffer = None
            self.k_pay = torch.zeros(slots, kv_heads, dim // 2, dtype=torch.uint8, device=device)
            self.v_pay = torch.zeros_like(self.k_pay)
            self.k_sf = torch.zeros(slots, kv_heads, dim // 16, dtype=torch.uint8, device=device)
            self.v_sf = torch.zeros_like(self.k_sf)
        else:
            raise ValueError(f'layout {layout!r}')
        one = lambda: torch.ones(1, dtype=torch.float32, device=device)
        self.gk = gk if gk is not None else one()
        self.gv = gv if gv is not None else one()

    @property
    def raw(self):
        return (self.k_pay, self.v_pay, self.k_sf, self.v_sf, self.gk, self.gv)

    def nbytes(self):
        return sum(t.numel() for t in (self.k_pay, self.v_pay, self.k_sf, self.v_sf))

    def set_global_scales(self, k, v):
        """The per-tensor global scales amax / (6 * 448) of K and V (formats.py:122), computed on the device."""
        ops.global_scale(k, out=self.gk)
        ops.global_scale(v, out=self.gv)

    def append(self, k, v, slots, saturate=True):
        """NVFP4 quantize-on-append of K and V rows [n, kv_heads, dim] (BF16) at pool slots [n], in one launch."""
        ops.store_kv([(k, self.gk, self.k_pay, self.k_sf), (v, self.gv, self.v_pay, self.v_sf)], slots,
                     saturate=saturate)


class LatentPool:
    """One layer's sparse-MLA cache: per slot an NVFP4 latent row (latent_dim values: payload latent_dim/2 bytes, E4M3
    scales latent_dim/16 bytes, FP32 global scale g on the device) and a BF16 rope row (rope_dim values).

    layout 'interleaved' (default): one buffer, per slot [payload | scales | rope] (416 bytes at 512 + 64), so a key is
    one contiguous record; 'split': three buffers. `raw` is (pay [slots, latent/2], scales [slots, latent/16],
    rope [slots, rope_dim] BF16, g [1]) as strided views either way."""

    def __init__(self, slots, latent_dim=512, rope_dim=64, device='cuda', layout='interleaved', g=None):
        self.slots, self.latent_dim, self.rope_dim, self.layout = slots, latent_dim, rope_dim, layout
        pb, sb, rb = latent_dim // 2, latent_dim // 16, rope_dim * 2
        if layout == 'interleaved':
            rec = pb + sb + rb
            self.buffer = torch.zeros(slots, rec, dtype=torch.uint8, device=device)
            self.pay = self.buffer[:, :pb]
            self.scales = self.buffer[:, pb:pb + sb]
            self.rope = self.buffer[:, pb + sb:].view(torch.bfloat16)
        elif layout == 'split':
            self.buffer = None
            self.pay = torch.zeros(slots, pb, dtype=torch.uint8, device=device)
            self.scales = torch.zeros(slots, sb, dtype=torch.uint8, device=device)
            self.rope = torch.zeros(slots, rope_dim, dtype=torch.bfloat16, device=device)
        else:
            raise ValueError(f'unknown layout {layout!r}')
        self.g = g if g is not None else torch.ones(1, dtype=torch.float32, device=device)

    @property
    def raw(self):
        return (self.pay, self.scales, self.rope, self.g)

    def set_global_scale(self, latent):
        """g = amax(|latent|) / (6 * 448), computed on the device (formats.py:122)."""
        self.g = ops.global_scale(latent.reshape(latent.shape[0], 1, -1))

    def append(self, latent, rope, slots, saturate=True):
        """Quantize BF16 latent rows [n, latent_dim] with the pool's g into `slots` and copy their rope rows, in one
        launch."""
        ops.store_kv([(latent, self.g, self.pay, self.scales), (rope.to(torch.bfloat16), None, self.rope, None)], slots,
                     saturate=saturate)
