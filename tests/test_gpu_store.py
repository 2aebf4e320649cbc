"""The fused KV-write epilogue (xt_nvfp4_store_kv: K, V and a third tensor in one launch) on the GPU against the oracle's
quantizer (xtier/backend/formats.py:114-128) byte for byte: token-major pools in both layouts, the MiniMax head-major
pages with the index K (the call of tests/minimax_kv_fp4_check.py:152-175), a latent cache's latent plus rope copy, and
blocks built to land exactly on the E2M1 midpoints or to hold non-finite values."""
import numpy as np
import pytest
import torch

from oracle import nvfp4
from xtier_amd import minimax, ops
from xtier_amd.pool import KVPool, LatentPool

pytestmark = pytest.mark.gpu


def _proj(n, heads, dim, seed):
    """K and V as strided views of one projection output, as a model's KV projection hands them over."""
    gen = torch.Generator().manual_seed(seed)
    proj = (torch.randn(n, (2 * heads + 1) * dim + 64, generator=gen) * 2).to(torch.bfloat16).cuda()
    k = proj[:, :heads * dim].view(n, heads, dim)
    v = proj[:, heads * dim:2 * heads * dim].view(n, heads, dim)
    ik = proj[:, 2 * heads * dim:(2 * heads + 1) * dim]
    return k, v, ik


@pytest.mark.parametrize('layout', ['interleaved', 'split'])
@pytest.mark.parametrize('n', [1, 37, 4096])
def test_kv_append_in_one_launch_equals_the_oracle(layout, n):
    heads, dim, slots = 4, 128, 8192
    k, v, _ = _proj(n, heads, dim, n)
    loc = torch.randperm(slots, generator=torch.Generator().manual_seed(n))[:n].cuda()
    if n > 1:
        loc[n // 2] = -1                      # a skipped row
    pool = KVPool(slots, heads, dim, layout=layout, gk=torch.tensor([0.0123], device='cuda'),
                  gv=torch.tensor([0.0456], device='cuda'))
    canary = [t.clone().fill_(0xA5) for t in (pool.k_pay, pool.v_pay, pool.k_sf, pool.v_sf)]
    for t, c in zip((pool.k_pay, pool.v_pay, pool.k_sf, pool.v_sf), canary):
        t.copy_(c)
    pool.append(k, v, loc)
    keep = (loc >= 0).cpu().numpy()
    sl = loc.cpu().numpy()[keep]
    for x, g, pay, sc in ((k, 0.0123, pool.k_pay, pool.k_sf), (v, 0.0456, pool.v_pay, pool.v_sf)):
        opay, osc = nvfp4.quantize_blocks(x.float().cpu().numpy(), np.float32(g), saturate=True)
        want_pay = np.full(tuple(pay.shape), 0xA5, np.uint8)
        want_sc = np.full(tuple(sc.shape), 0xA5, np.uint8)
        want_pay[sl], want_sc[sl] = opay[keep], osc[keep]
        assert np.array_equal(pay.cpu().numpy(), want_pay) and np.array_equal(sc.cpu().numpy(), want_sc)


@pytest.mark.parametrize('n', [1, 6, 12, 1000, 4096])
def test_minimax_store_into_head_major_pages(n):
    """Main K, V (4 heads x 128) and index K (one head) into head-major pages of 128 rows at random token slots, with
    the pool's unit global scale: every byte as the oracle places it, other rows untouched."""
    kh, d, page, pages = 4, 128, 128, 64
    k, v, ik = _proj(n, kh, d, 100 + n)
    loc = torch.randperm(pages * page, generator=torch.Generator().manual_seed(n))[:n].cuda()
    kpay, vpay = (torch.full((pages, kh, page, d // 2), 0x5A, dtype=torch.uint8, device='cuda') for _ in range(2))
    ksc, vsc = (torch.full((pages, kh, page, d // 16), 0x5A, dtype=torch.uint8, device='cuda') for _ in range(2))
    ipay = torch.full((pages, page, d // 2), 0x5A, dtype=torch.uint8, device='cuda')
    isc = torch.full((pages, page, d // 16), 0x5A, dtype=torch.uint8, device='cuda')
    g = torch.ones(1, device='cuda')
    ops.nvfp4_store_kv_index(k, v, ik, kpay, ksc.view(torch.float8_e4m3fn), vpay, vsc.view(torch.float8_e4m3fn),
                             ipay, isc.view(torch.float8_e4m3fn), loc, g, page_size=page)
    p, r = (loc // page).cpu().numpy(), (loc % page).cpu().numpy()
    for x, pay, sc in ((k, kpay, ksc), (v, vpay, vsc)):
        opay, osc = nvfp4.quantize_blocks(x.float().cpu().numpy(), np.float32(1.0), saturate=True)
        want_pay = np.full(tuple(pay.shape), 0x5A, np.uint8)
        want_sc = np.full(tuple(sc.shape), 0x5A, np.uint8)
        for h in range(kh):
            want_pay[p, h, r], want_sc[p, h, r] = opay[:, h], osc[:, h]
        assert np.array_equal(pay.cpu().numpy(), want_pay) and np.array_equal(sc.cpu().numpy(), want_sc)
    opay, osc = nvfp4.quantize_blocks(ik.float().cpu().numpy(), np.float32(1.0), saturate=True)
    want_pay = np.full(tuple(ipay.shape), 0x5A, np.uint8)
    want_sc = np.full(tuple(isc.shape), 0x5A, np.uint8)
    want_pay[p, r], want_sc[p, r] = opay, osc
    assert np.array_equal(ipay.cpu().numpy(), want_pay) and np.array_equal(isc.cpu().numpy(), want_sc)


def test_minimax_store_hook_falls_through_off_gpu_and_runs_the_store_on_it():
    seen = []
    original = lambda *a, **kw: seen.append(a) or 'original'
    cpu = torch.zeros(2, 4, 128, dtype=torch.bfloat16)
    assert minimax.store_kv_index(original, cpu, cpu, cpu[:, 0], *([None] * 6), None, None) == 'original'
    kh, d, page, pages = 2, 128, 128, 4
    k, v, ik = _proj(3, kh, d, 9)
    bufs = [torch.zeros(pages, kh, page, w, dtype=torch.uint8, device='cuda') for w in (64, 8, 64, 8)]
    ib = [torch.zeros(pages, page, w, dtype=torch.uint8, device='cuda') for w in (64, 8)]
    loc = torch.tensor([5, 300, 129], device='cuda')
    minimax.store_kv_index(original, k, v, ik, bufs[0], bufs[1], bufs[2], bufs[3], ib[0], ib[1], loc,
                           torch.ones(1, device='cuda'), page_size=page)
    assert len(seen) == 1 and bufs[0][0, 0, 5].any() and ib[0][2, 44].any()   # slot 300: page 2, row 44


@pytest.mark.parametrize('layout', ['interleaved', 'split'])
def test_latent_append_quantizes_latent_and_copies_rope(layout):
    n, slots = 500, 4096
    gen = torch.Generator().manual_seed(4)
    lat = (torch.randn(n, 512, generator=gen)).to(torch.bfloat16).cuda()
    rope = (torch.randn(n, 64, generator=gen)).to(torch.bfloat16).cuda()
    loc = torch.randperm(slots, generator=gen)[:n].cuda()
    pool = LatentPool(slots, layout=layout, g=torch.tensor([0.0031], device='cuda'))
    pool.append(lat, rope, loc)
    opay, osc = nvfp4.quantize_blocks(lat.float().cpu().numpy(), np.float32(0.0031), saturate=True)
    sl = loc.cpu().numpy()
    assert np.array_equal(pool.pay.cpu().numpy()[sl], opay) and np.array_equal(pool.scales.cpu().numpy()[sl], osc)
    assert torch.equal(pool.rope[loc].view(torch.int16), rope.view(torch.int16))
    others = np.setdiff1d(np.arange(slots), sl)
    assert not pool.pay.cpu().numpy()[others].any() and not pool.rope.float().cpu().numpy()[others].any()


@pytest.mark.parametrize('saturate', [True, False])
def test_blocks_on_the_midpoints_and_non_finite_blocks(saturate):
    """Blocks whose values divide by the block's d = 1.125 (scale 1.125, g = 1) exactly onto the E2M1 midpoints (a
    value on a midpoint takes the smaller magnitude) and one BF16 step either side, in both signs; a block scale that
    rounds past 448; and blocks with inf and NaN values."""
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32) * np.float32(1.125)
    bf = lambda a: nvfp4.f32_to_bf16_f32(np.asarray(a, np.float32))
    assert np.array_equal(bf(mids), mids)                    # the products are BF16 values
    bits = nvfp4.bf16_bits(mids).astype(np.int32)
    up = nvfp4.bf16_to_f32((bits + 1).astype(np.uint16))     # one BF16 step above each midpoint product
    dn = nvfp4.bf16_to_f32((bits - 1).astype(np.uint16))     # and one below
    vals = np.concatenate([mids, up, dn, -mids, -up, -dn])
    blocks = []
    for i in range(0, len(vals), 15):
        b = np.zeros(16, np.float32)
        b[0] = 6.75                                          # block amax 6.75: scale e4m3(6.75 / 6) = 1.125
        chunk = vals[i:i + 15]
        b[1:1 + len(chunk)] = chunk
        blocks.append(b)
    big = np.full(16, 3000.0, np.float32)                    # 3000 / 6 = 500 > 448: NaN scale or saturated
    inf = np.zeros(16, np.float32)
    inf[3], inf[4] = np.inf, -2.0
    nan = np.zeros(16, np.float32)
    nan[5], nan[6], nan[7] = np.nan, 1.0, -np.nan        # a NaN of either sign codes 7, without the sign bit
    x = np.stack(blocks + [big, inf, nan]).reshape(-1, 1, 16)
    x = np.concatenate([x, np.zeros((x.shape[0], 1, 112), np.float32)], -1)    # rows of 128
    xt = torch.from_numpy(x).to(torch.bfloat16).cuda()
    n = xt.shape[0]
    pay = torch.zeros(n, 1, 64, dtype=torch.uint8, device='cuda')
    sc = torch.zeros(n, 1, 8, dtype=torch.uint8, device='cuda')
    ops.store_kv([(xt, torch.ones(1, device='cuda'), pay, sc)], torch.arange(n, device='cuda'), saturate=saturate)
    opay, osc = nvfp4.quantize_blocks(xt.float().cpu().numpy(), np.float32(1.0), saturate=saturate)
    assert np.array_equal(sc.cpu().numpy(), osc) and np.array_equal(pay.cpu().numpy(), opay)
    assert (osc[:len(blocks), 0, 0] == 0x39).all()           # E4M3 1.125
