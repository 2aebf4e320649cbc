"""Shared builders for the GPU parity tests: NVFP4 pools made by the oracle on the CPU (so the GPU reads bytes the
oracle knows), uploaded to the device in the reference's layout."""
import numpy as np
import torch

from oracle import nvfp4
from xtier_amd import workloads


def bf16_numpy(t):
    """A bf16 torch tensor's values as float32 numpy (exact)."""
    return t.float().cpu().numpy()


class Pool:
    """Host (numpy) and device (torch) copies of one layer's pool: payload/scales for K and V, global scales."""

    def __init__(self, k_bf16, v_bf16, device='cuda'):
        self.k_pay, self.k_sf, self.gk = nvfp4.nvfp4_encode(bf16_numpy(k_bf16))
        self.v_pay, self.v_sf, self.gv = nvfp4.nvfp4_encode(bf16_numpy(v_bf16))
        dev = torch.device(device)
        up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.raw = (up(self.k_pay), up(self.v_pay), up(self.k_sf), up(self.v_sf),
                    torch.tensor([self.gk], dtype=torch.float32, device=dev),
                    torch.tensor([self.gv], dtype=torch.float32, device=dev))

    @property
    def host(self):
        return (self.k_pay, self.v_pay, self.k_sf, self.v_sf, self.gk, self.gv)


def random_pool(seed, slots, heads, dim, device='cuda'):
    gen = workloads.generator('cpu', seed)
    k = workloads.kv_tensor(slots, heads, dim, gen, 'cpu')
    v = workloads.kv_tensor(slots, heads, dim, gen, 'cpu')
    return Pool(k, v, device)
