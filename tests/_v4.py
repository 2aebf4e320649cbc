"""DeepSeek V4 FP8 KV pages for the tests, built on the CPU from float latents with the format's own rule (the
packing of tests/ds_sparse_mla_check.py:25-41): per token and 64-value group, e = ceil(log2(amax / 448)) clamped to
[-126, 127], the values / 2^e as E4M3 (torch's float8_e4m3fn cast), stored exponent e + 127; the 64 rope values as
BF16. Returns the page view [pages, page_size, 1, 584] and the exact keys in float64."""
import math

import numpy as np
import torch

NOPE, DIM = 448, 512


def pack_v4(latent, page_size, page_stride=None):
    latent = latent.float().cpu()
    tokens = latent.shape[0]
    pages = tokens // page_size
    groups = latent[:, :NOPE].reshape(tokens, NOPE // 64, 64)
    e = torch.ceil(torch.log2(groups.abs().amax(-1).clamp_min(1e-30) / 448)).clamp(-126, 127)
    fp8 = (groups / torch.exp2(e)[..., None]).to(torch.float8_e4m3fn)
    rope = latent[:, NOPE:].to(torch.bfloat16)
    stride = page_stride or math.ceil(page_size * 584 / 256) * 256
    buf = torch.zeros(pages * stride, dtype=torch.uint8)
    for p in range(pages):
        t = slice(p * page_size, (p + 1) * page_size)
        base = p * stride
        data = buf[base:base + page_size * 576].view(page_size, 576)
        data[:, :NOPE] = fp8[t].view(torch.uint8).reshape(page_size, NOPE)
        data[:, NOPE:] = rope[t].view(torch.uint8).reshape(page_size, 128)
        sc = buf[base + page_size * 576:base + page_size * 584].view(page_size, 8)
        sc[:, :7] = (e[t] + 127).to(torch.uint8)
    keys = torch.cat([(fp8.double() * torch.exp2(e.double())[..., None]).reshape(tokens, NOPE), rope.double()], 1)
    view = buf.as_strided((pages, page_size, 1, 584), (stride, 584, 584, 1))
    return view, keys.numpy(), stride
