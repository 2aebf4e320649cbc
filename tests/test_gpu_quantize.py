"""NVFP4 quantize-on-append on the GPU against the oracle: payload bytes, scale bytes and the global scale bit for
bit (xtier/backend/formats.py:114-128 semantics)."""
import numpy as np
import pytest
import torch

from oracle import nvfp4
from xtier_amd import ops, workloads
from xtier_amd.pool import KVPool

pytestmark = pytest.mark.gpu


def _kv(seed, n, heads, dim):
    gen = workloads.generator('cpu', seed)
    return workloads.kv_tensor(n, heads, dim, gen, 'cpu')


@pytest.mark.parametrize('n,heads,dim', [(4096, 1, 128), (777, 4, 128), (64, 2, 256), (16, 8, 64)])
def test_encode_bit_exact(n, heads, dim):
    x = _kv(n + heads, n, heads, dim)
    pay, sc, g = ops.nvfp4_encode(x.cuda())
    opay, osc, og = nvfp4.nvfp4_encode(x.float().numpy())
    assert np.float32(g.item()).view(np.uint32) == np.float32(og).view(np.uint32)
    assert np.array_equal(sc.cpu().numpy(), osc)
    assert np.array_equal(pay.cpu().numpy(), opay)


def test_encode_magnitudes_over_decades():
    """Per-token magnitudes over 5 decades (tests/qsa_fp4_check.py:26-34 spreads 3): small blocks hit subnormal
    E4M3 scales."""
    gen = torch.Generator().manual_seed(20261023)
    x = (torch.randn(3000, 2, 128, generator=gen) * 10 ** torch.empty(3000, 1, 1).uniform_(-4, 1, generator=gen))
    x = x.to(torch.bfloat16)
    pay, sc, g = ops.nvfp4_encode(x.cuda())
    opay, osc, og = nvfp4.nvfp4_encode(x.float().numpy())
    assert g.item() == og
    assert np.array_equal(sc.cpu().numpy(), osc) and np.array_equal(pay.cpu().numpy(), opay)
    assert (osc < 8).any()   # subnormal scales occur


def test_append_strided_rows_to_permuted_slots():
    """K as a strided view of a projection output (the MiniMax store check's shape), written to shuffled slots; a
    negative slot skips its row and untouched slots keep their bytes."""
    n, heads, dim, pool_slots = 300, 4, 128, 1024
    gen = torch.Generator().manual_seed(3)
    proj = (torch.randn(n, 3 * heads * dim + 64, generator=gen) * 2).to(torch.bfloat16)
    k = proj[:, heads * dim:2 * heads * dim].view(n, heads, dim)
    slots = torch.randperm(pool_slots, generator=gen)[:n]
    slots[7] = -1
    g = torch.tensor([0.0021], dtype=torch.float32)
    pay = torch.full((pool_slots, heads, dim // 2), 0xAB, dtype=torch.uint8, device='cuda')
    sc = torch.full((pool_slots, heads, dim // 16), 0xCD, dtype=torch.uint8, device='cuda')
    ops.quantize_append(k.cuda(), slots.cuda(), g.cuda(), pay, sc, saturate=True)
    opay, osc = nvfp4.quantize_blocks(k.float().numpy(), np.float32(0.0021), saturate=True)
    want_pay = np.full((pool_slots, heads, dim // 2), 0xAB, np.uint8)
    want_sc = np.full((pool_slots, heads, dim // 16), 0xCD, np.uint8)
    keep = slots.numpy() >= 0
    want_pay[slots.numpy()[keep]] = opay[keep]
    want_sc[slots.numpy()[keep]] = osc[keep]
    assert np.array_equal(pay.cpu().numpy(), want_pay) and np.array_equal(sc.cpu().numpy(), want_sc)


@pytest.mark.parametrize('saturate', [False, True])
def test_fixed_scale_overflow(saturate):
    """Rows far above a fixed global scale: E4M3 NaN scales (the reference's cast) or 448 (saturating)."""
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(64, 2, 128, generator=gen) * 30).to(torch.bfloat16)
    g = np.float32(0.01)
    pay = torch.zeros(64, 2, 64, dtype=torch.uint8, device='cuda')
    sc = torch.zeros(64, 2, 8, dtype=torch.uint8, device='cuda')
    ops.quantize_append(x.cuda(), torch.arange(64).cuda(), torch.tensor([g]).cuda(), pay, sc, saturate=saturate)
    opay, osc = nvfp4.quantize_blocks(x.float().numpy(), g, saturate=saturate)
    assert ((osc & 0x7F) == (0x7E if saturate else 0x7F)).any()
    assert np.array_equal(sc.cpu().numpy(), osc) and np.array_equal(pay.cpu().numpy(), opay)


def test_golden_fixture():
    data = np.load(__import__('pathlib').Path(__file__).parent / 'golden' / 'nvfp4_encode.npz')
    x = torch.from_numpy(data['x_bf16'].view(np.int16)).view(torch.bfloat16)
    pay, sc, g = ops.nvfp4_encode(x.cuda())
    assert np.float32(g.item()) == data['g'][0]
    assert np.array_equal(pay.cpu().numpy(), data['pay']) and np.array_equal(sc.cpu().numpy(), data['sc'])


@pytest.mark.parametrize('layout', ['interleaved', 'split'])
def test_pool_append_layouts(layout):
    """KVPool: device global scales, then K and V appended at shuffled slots; every payload / scale byte equal to the
    oracle's in either layout, the interleaved buffer's bytes in place."""
    n, heads, dim = 500, 4, 128
    gen = workloads.generator('cpu', 17)
    k = workloads.kv_tensor(n, heads, dim, gen, 'cpu')
    v = workloads.kv_tensor(n, heads, dim, gen, 'cpu')
    slots = torch.randperm(1024, generator=gen)[:n]
    pool = KVPool(1024, heads, dim, layout=layout)
    pool.set_global_scales(k.cuda(), v.cuda())
    pool.append(k.cuda(), v.cuda(), slots.cuda())
    for x, pay, sc, g in ((k, pool.k_pay, pool.k_sf, pool.gk), (v, pool.v_pay, pool.v_sf, pool.gv)):
        og = nvfp4.global_scale(x.float().numpy())
        assert np.float32(g.item()) == og
        opay, osc = nvfp4.quantize_blocks(x.float().numpy(), og, saturate=True)
        assert np.array_equal(pay.cpu().numpy()[slots.numpy()], opay)
        assert np.array_equal(sc.cpu().numpy()[slots.numpy()], osc)
    if layout == 'interleaved':
        # per slot: each head's [K row | V row] (128 bytes), then each head's [K scales | V scales] (16 bytes)
        row = pool.buffer[slots[0]].cpu().numpy()
        pairs, scales = row[:512].reshape(heads, 128), row[512:].reshape(heads, 16)
        assert np.array_equal(pairs[:, :64], pool.k_pay[slots[0]].cpu().numpy())
        assert np.array_equal(pairs[:, 64:], pool.v_pay[slots[0]].cpu().numpy())
        assert np.array_equal(scales[:, :8], pool.k_sf[slots[0]].cpu().numpy())
        assert np.array_equal(scales[:, 8:], pool.v_sf[slots[0]].cpu().numpy())
        assert row.size == 576 and pool.k_pay.stride()[:2] == (576, 128) and pool.k_sf.stride()[:2] == (576, 16)
