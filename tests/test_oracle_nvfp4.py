"""The CPU oracle's NVFP4 arithmetic pinned against the reference's tables, torch's FP8 conversions (the library
routines the reference quantizer calls) and independent brute force."""
import numpy as np
import pytest
import torch

from oracle import nvfp4

# the table the reference's own tests hold (tests/draft_bf16_check.py:25, tests/fp4_decode_check.py:15)
REF_E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def test_e2m1_table_all_bytes():
    want = np.array(REF_E2M1, dtype=np.float32)
    assert np.array_equal(nvfp4.E2M1_TABLE.view(np.uint32), want.view(np.uint32))   # -0.0 for code 8 included
    b = np.arange(256, dtype=np.uint8)
    codes = nvfp4.unpack_codes(b[:, None])
    assert np.array_equal(nvfp4.e2m1_decode(codes[:, 0]).view(np.uint32), want[b & 15].view(np.uint32))
    assert np.array_equal(nvfp4.e2m1_decode(codes[:, 1]).view(np.uint32), want[b >> 4].view(np.uint32))


def test_e4m3_decode_matches_torch_all_bytes():
    want = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    got = nvfp4.e4m3_decode(np.arange(256))
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _encode_grid():
    """tests/fp8_encode_check.py:29-37: every FP32 top-20-bit pattern with low bits 0, 7FF, 800, 801, FFF, random
    values over the range, and the edge list (both signs)."""
    top = np.arange(1 << 20, dtype=np.int64) << 12
    grid = np.concatenate([top, top | 0x7FF, top | 0x800, top | 0x801, top | 0xFFF]).astype(np.uint32).view(np.float32)
    rng = np.random.default_rng(20261029)
    rand = (rng.standard_normal(1 << 20) * np.logspace(-6, 3, 1 << 20)).astype(np.float32)
    edges = np.array([0.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -6, 2.0 ** -6 - 2.0 ** -10, 448.0, 449.0,
                      463.9, 464.0, 464.1, 479.0, 480.0, 1e30, np.inf, np.nan], dtype=np.float32)
    return np.concatenate([grid, rand, edges, -edges])


def test_e4m3_encode_matches_torch_cast():
    x = _encode_grid()
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = nvfp4.e4m3_encode(x, saturate=False)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7F) == 0x7F) and np.all((want[nan] & 0x7F) == 0x7F)


def test_e4m3_encode_saturating():
    x = _encode_grid()
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    nan = np.isnan(x)
    # satfinite (xtier/arch.py:57-75): where torch's cast overflows to NaN, 448 with the sign
    want = np.where(((ref & 0x7F) == 0x7F) & ~nan, (ref & 0x80) | 0x7E, ref).astype(np.uint8)
    got = nvfp4.e4m3_encode(x, saturate=True)
    assert np.array_equal(got[~nan], want[~nan])
    assert nvfp4.e4m3_encode(np.float32(np.inf), True) == 0x7E and nvfp4.e4m3_encode(np.float32(-np.inf), True) == 0xFE


def _nearest_codes(q):
    """Brute force: the E2M1 magnitude nearest to min(|q|, 6), the smaller one on a tie; sign when q < 0 and the
    magnitude is not 0."""
    mag = np.minimum(np.abs(q), 6.0)
    d = np.abs(mag[..., None].astype(np.float64) - nvfp4.E2M1_MAGNITUDES.astype(np.float64))
    code = np.argmin(d, -1).astype(np.uint8)      # first minimum = the smaller magnitude
    code = np.where(np.isnan(q), 7, code).astype(np.uint8)
    return code | (((q < 0) & (code > 0)).astype(np.uint8) << 3)


def _quotients(x, g):
    blocks = x.reshape(-1, x.shape[-1] // 16, 16)
    s = nvfp4.e4m3_decode(nvfp4.e4m3_encode(np.abs(blocks).max(-1) / (np.float32(6) * g)))
    return blocks / np.maximum(s * g, np.float32(1e-30))[..., None]


@pytest.mark.parametrize('seed', [0, 1, 2])
def test_quantize_codes_brute_force(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((512, 128)) * 10.0 ** rng.uniform(-3, 2, (512, 1))).astype(np.float32)
    x = nvfp4.f32_to_bf16_f32(x)
    pay, sc, g = nvfp4.nvfp4_encode(x)
    want = _nearest_codes(_quotients(x, g)).reshape(512, 128)
    assert np.array_equal(nvfp4.unpack_codes(pay), want)


def test_quantize_matches_torch_primitives():
    """The same quotients bucketized by torch.bucketize and scales cast by torch (the reference's primitives)."""
    rng = np.random.default_rng(7)
    x = nvfp4.f32_to_bf16_f32((rng.standard_normal((256, 64)) * 3).astype(np.float32))
    pay, sc, g = nvfp4.nvfp4_encode(x)
    w = torch.from_numpy(x)
    tg = (w.abs().amax() / (6 * 448)).clamp_min(1e-12)
    assert np.float32(tg.item()) == g
    blocks = w.unflatten(-1, (-1, 16))
    s = (blocks.abs().amax(-1) / (6 * tg)).to(torch.float8_e4m3fn)
    q = (blocks / (s.float() * tg).clamp_min(1e-30).unsqueeze(-1)).flatten(-2)
    code = torch.bucketize(q.abs().clamp(max=6.0), torch.tensor(nvfp4.E2M1_BOUNDS.tolist())).to(torch.uint8)
    code |= ((q < 0) & (code > 0)).to(torch.uint8) << 3
    assert np.array_equal(sc, s.view(torch.uint8).numpy())
    assert np.array_equal(pay, (code[:, 0::2] | (code[:, 1::2] << 4)).numpy())


def test_quantize_round_trip_within_one_block_scale():
    """tests/draft_bf16_check.py:41-44: every value within one block scale of its input."""
    rng = np.random.default_rng(0)
    x = nvfp4.f32_to_bf16_f32((rng.standard_normal((64, 4096)) * rng.random((64, 1)) * 0.05).astype(np.float32))
    pay, sc, g = nvfp4.nvfp4_encode(x)
    back = nvfp4.dequant(pay, sc, g)
    bound = np.repeat(nvfp4.e4m3_decode(sc), 16, -1) * g
    assert (np.abs(back - x) / np.maximum(bound, 1e-30)).max() <= 1.0 + 1e-6


def test_quantize_special_cases():
    g = np.float32(1.0)
    # block amax 6: the scale is 1 and quotients are the values themselves; midpoints take the smaller magnitude
    row = np.array([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -0.2, -0.0, 0.0, -6.0, 0.26, 4.99, 5.01],
                   dtype=np.float32)
    pay, sc = nvfp4.quantize_blocks(row[None], g)
    assert sc[0, 0] == 0x38                                   # E4M3 1.0
    codes = nvfp4.unpack_codes(pay)[0].tolist()
    assert codes == [7, 0, 1, 2, 3, 4, 5, 6, 0, 0, 0, 0, 15, 1, 6, 7]
    # a zero block: scale 0, every code 0
    pay, sc = nvfp4.quantize_blocks(np.zeros((1, 16), np.float32), g)
    assert sc[0, 0] == 0 and not pay.any()
    # the global scale's clamp
    assert nvfp4.global_scale(np.zeros(16, np.float32)) == np.float32(1e-12)
    assert nvfp4.global_scale(np.full(16, 2688.0, np.float32)) == np.float32(1.0)


def test_quantize_fixed_scale_overflow_rules():
    """A block far above the fixed global scale: NaN scale with the reference's cast, 448 when saturating."""
    x = np.full((1, 16), 1000.0, np.float32)
    pay_nan, sc_nan = nvfp4.quantize_blocks(x, np.float32(0.1), saturate=False)
    pay_sat, sc_sat = nvfp4.quantize_blocks(x, np.float32(0.1), saturate=True)
    assert sc_nan[0, 0] == 0x7F and np.all(nvfp4.unpack_codes(pay_nan) == 7)   # NaN quotients bucketize to 7
    assert sc_sat[0, 0] == 0x7E and np.all(nvfp4.unpack_codes(pay_sat) == 7)   # 1000 / 44.8 clamps to 6


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([(rng.standard_normal(1 << 16) * 10.0 ** rng.uniform(-30, 30, 1 << 16)).astype(np.float32),
                        np.array([np.inf, -np.inf, 3.3895314e38, -0.0], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(nvfp4.bf16_bits(x), want)
