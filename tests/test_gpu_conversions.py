"""Device known-answer test of the hardware conversions the attention kernels use, every byte against the format
tables (the method of tests/fp8_decode_check.py:28-45 and tests/fp4_decode_check.py:67-107): E4M3 -> FP16 from either
half of a dword (v_cvt_scalef32_pk_f16_fp8), two E2M1 codes -> FP16 and FP32 from each byte position
(v_cvt_scalef32_pk_{f16,f32}_fp4), and E4M3 times a power-of-2 V4 scale -> BF16 (v_cvt_scalef32_pk_bf16_fp8)."""
import numpy as np
import pytest
import torch

from oracle import nvfp4
from xtier_amd import _lib

pytestmark = pytest.mark.gpu

ALL = np.arange(256, dtype=np.uint8)


def _run():
    lib = _lib.lib()
    n = lib.xt_selftest_conversions_bytes()
    buf = torch.full((n // 2,), 0x5A5A, dtype=torch.int16, device='cuda')
    _lib.check(lib.xt_selftest_conversions(buf.data_ptr(), torch.cuda.current_stream().cuda_stream), 'selftest')
    torch.cuda.synchronize()
    return buf.cpu().numpy().view(np.uint16)


def _f16(bits):
    return bits.view(np.float16).astype(np.float64)


def _same(got, want):
    """Equal values, NaN where NaN is expected, and the sign of zero kept."""
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.array_equal(np.signbit(got[~nan]), np.signbit(want[~nan]))


def test_e4m3_to_f16_every_byte():
    out = _run()
    want = nvfp4.e4m3_decode(ALL).astype(np.float64)
    _same(_f16(out[:256]), want)          # low half of the dword
    _same(_f16(out[256:512]), want)       # high half


def test_e2m1_pairs_to_f16_and_f32_every_byte_position():
    out = _run()
    table = nvfp4.e2m1_decode(np.arange(16, dtype=np.uint8)).astype(np.float64)
    want = np.stack([table[ALL & 15], table[ALL >> 4]], 1).reshape(-1)   # low nibble first
    f32 = out[3328:3328 + 2 * 2048].copy().view(np.float32).astype(np.float64)
    for sel in range(4):
        _same(_f16(out[512 + sel * 512:512 + (sel + 1) * 512]), want)
        _same(f32[sel * 512:(sel + 1) * 512], want)


def test_e4m3_with_v4_scale_to_bf16_every_byte():
    out = _run()
    e4m3 = nvfp4.e4m3_decode(ALL).astype(np.float64)
    for i, e in enumerate((120, 127, 134)):
        got = nvfp4.bf16_to_f32(out[2560 + i * 256:2560 + (i + 1) * 256]).astype(np.float64)
        _same(got, e4m3 * 2.0 ** (e - 127))   # exact in BF16: 3 mantissa bits, exponents in range
