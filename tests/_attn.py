"""Attention references for the GPU parity tests: FP64 softmax and the flash-precision reference over the pool bytes
the GPU holds (tests/qsa_decode_check.py:14-45), and the tolerance check (max-abs 2e-2 / mean-abs 2e-3 in BF16, and the
flash kernels' precision class of tests/qsa_decode_check.py:82)."""
import numpy as np
import torch

from oracle import attention, nvfp4

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def host_rows(raw_dev, slots):
    """Host copies of the pool rows at `slots` (unique) and the map slot -> compact row."""
    uniq = np.unique(slots[slots >= 0])
    sel = torch.from_numpy(uniq).cuda()
    host = tuple(t.index_select(0, sel).cpu().numpy() for t in raw_dev[:4]) + (raw_dev[4].item(), raw_dev[5].item())
    return host, uniq


def oracle(raw_dev, q, table, page, rows_req, idx, counts, seq, scale, qpos=None):
    """FP64 and flash-precision references for every row, from the pool bytes the GPU holds."""
    table = np.asarray(table)
    nrows = q.shape[0]
    all_slots = np.full(idx.shape, -1, np.int64)
    valid = np.zeros(idx.shape, bool)
    for r in range(nrows):
        v = attention.key_validity(idx[r], counts[r] if counts is not None else idx.shape[1], seq[r],
                                   None if qpos is None else qpos[r])
        valid[r] = v
        if v.any():
            all_slots[r, v] = attention.slots_of(table, rows_req[r], idx[r][v], page)
    host, uniq = host_rows(raw_dev, all_slots)
    k_pay, v_pay, k_sf, v_sf, gk, gv = host
    ref = np.zeros(q.shape)
    flash = np.zeros(q.shape)
    lse = np.full(q.shape[:2], -np.inf)
    qf = q.astype(np.float32)
    for r in range(nrows):
        n = int(valid[r].sum())
        if n == 0:
            continue
        pos = np.searchsorted(uniq, all_slots[r][valid[r]])
        k = nvfp4.dequant(k_pay[pos], k_sf[pos], gk)
        v = nvfp4.dequant(v_pay[pos], v_sf[pos], gv)
        ones = np.ones(n, bool)
        ref[r] = attention.softmax_attention(qf[r], k, v, ones, scale)
        flash[r] = attention.flash_precision_attention(qf[r], k, v, ones, scale)
        group = q.shape[1] // k.shape[1]
        for h in range(q.shape[1]):
            s = k[:, h // group].astype(np.float64) @ qf[r, h].astype(np.float64) * scale
            lse[r, h] = s.max() + np.log(np.exp(s - s.max()).sum())
    return ref, flash, lse


def check(got, ref, flash, nonempty=None, strict=False):
    """Tolerances: mean |err| <= 2e-3; max |err| <= 2e-2 beyond the BF16 rounding of the reference value (strict:
    2e-2 absolute, for the workloads whose outputs are small averages); and the precision class of the flash
    kernels (max <= 1.5x, mean <= 1.25x the flash-precision reference's error)."""
    g = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(g - ref)
    fe = np.abs(flash - ref)
    half_ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 8)
    if nonempty is not None:
        err, fe, half_ulp = err[nonempty], fe[nonempty], half_ulp[nonempty]
    assert np.isfinite(g).all()
    assert err.mean() <= MEAN_ABS, err.mean()
    assert (err - (0 if strict else half_ulp)).max() <= MAX_ABS, err.max()
    assert err.max() <= 1.5 * fe.max() + 1e-6 and err.mean() <= 1.25 * fe.mean() + 1e-7, (err.max(), fe.max(),
                                                                                           err.mean(), fe.mean())
    return err
