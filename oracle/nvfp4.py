"""NVFP4 format arithmetic on the CPU (numpy): the oracle for the quantizer, the dequantizer and the byte layouts.

Test infrastructure only (see the package docstring for what pins each function).

Format (reference: xtier/packs/qwen4_exp/qsa_fp4.py:3-4, :94-101; xtier/backend/formats.py:114-128):
- payload byte i of a row holds element 2i in bits 0-3 and element 2i+1 in bits 4-7;
- an E2M1 code is a sign (bit 3) and a magnitude index into {0, .5, 1, 1.5, 2, 3, 4, 6}; code 8 is -0.0;
- one OCP E4M3 ("fn") scale byte per 16 consecutive elements;
- value = (e2m1 * e4m3) * g in FP32, g the per-tensor FP32 global scale.
"""
import numpy as np

E2M1_MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
# code -> value, sign in bit 3 (tests/draft_bf16_check.py:25): code 8 is -0.0
E2M1_TABLE = np.concatenate([E2M1_MAGNITUDES, -E2M1_MAGNITUDES]).astype(np.float32)
# midpoints between consecutive E2M1 magnitudes (xtier/backend/formats.py:111)
E2M1_BOUNDS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)
GLOBAL_DIVISOR = 6 * 448       # E2M1 max * E4M3 max (formats.py:122)
F32 = np.float32


def e2m1_decode(codes):
    """E2M1 codes (low 4 bits of ``codes``) -> float32 (qsa_fp4.py:81-86; arch.py:30-37 gives the same values)."""
    return E2M1_TABLE[np.asarray(codes).astype(np.int64) & 15]


def _e4m3_table():
    """Value of each of the 256 E4M3 (fn) bytes (arch.py:40-54): exponent field e, mantissa m; e > 0 is
    2^(e-7) * (1 + m/8); e = 0 is m * 2^-9; 0x7F and 0xFF are NaN; bit 7 is the sign."""
    b = np.arange(256, dtype=np.int64)
    e = (b >> 3) & 15
    m = b & 7
    mag = np.where(e == 0, m * 2.0 ** -9, 2.0 ** (e - 7) * (1.0 + m / 8.0))
    mag = np.where((b & 0x7F) == 0x7F, np.nan, mag)
    return np.where((b & 0x80) != 0, -mag, mag).astype(np.float32)


E4M3_TABLE = _e4m3_table()


def e4m3_decode(bytes_):
    """E4M3 bytes -> float32."""
    return E4M3_TABLE[np.asarray(bytes_).astype(np.int64) & 255]


def e4m3_encode(x, saturate=False):
    """float32 -> E4M3 (fn) byte, round to nearest even.

    saturate=False: torch's float8_e4m3fn cast, which the reference quantizer uses (formats.py:124): a magnitude that
    rounds above 448 (from 464 up, infinities included) becomes NaN (0x7F with the sign).
    saturate=True: the satfinite conversion of arch.py:57-75 (cvt.rn.satfinite): such magnitudes become 448 (0x7E).
    NaN becomes 0x7F with its sign either way.
    Below 2^-6 the value is |x| * 2^9 subnormal steps rounded to even; from 2^-6 up the FP32 bits are rounded at
    mantissa bit 20 (a carry moves into the exponent)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = x.view(np.uint32).astype(np.int64)
    sign = (bits >> 24) & 0x80
    a = bits & 0x7FFFFFFF
    with np.errstate(over='ignore', invalid='ignore'):
        t = (a.astype(np.uint32).view(np.float32) * F32(512.0)).astype(np.float64)   # exact: power-of-two scaling
    lo = np.floor(np.where(a < 0x3C800000, t, 0.0))
    steps = lo.astype(np.int64)
    half = np.where(a < 0x3C800000, t, 0.0) - lo
    steps = steps + ((half > 0.5) | ((half == 0.5) & ((steps & 1) == 1))).astype(np.int64)
    r = a + 0x7FFFF + ((a >> 20) & 1)
    normal = (((r >> 23) - 120) << 3) | ((r >> 20) & 7)
    code = np.where(a < 0x3C800000, steps, normal)
    over = code > 0x7E
    code = np.where(over, 0x7E if saturate else 0x7F, code)
    code = np.where(a > 0x7F800000, 0x7F, code)   # NaN
    return (code | sign).astype(np.uint8)


def bf16_bits(x):
    """float32 -> bfloat16 bits, round to nearest even (torch's .to(torch.bfloat16)); NaN -> 0x7FC0 with its sign."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    return np.where(nan, ((b >> 16) & 0x8000).astype(np.uint16) | np.uint16(0x7FC0), r).astype(np.uint16)


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_f32(x):
    """float32 rounded to bfloat16 and back (RNE)."""
    return bf16_to_f32(bf16_bits(x))


def global_scale(x):
    """Per-tensor FP32 global scale of formats.py:122: max(amax / (6 * 448), 1e-12), all in FP32."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max() if x.size else F32(0.0)
    return max(F32(amax) / F32(GLOBAL_DIVISOR), F32(1e-12))


def quantize_blocks(x, g, saturate=False):
    """Rows x [..., K] (K a multiple of 16, float32) with the FP32 global scale g -> (payload uint8 [..., K/2],
    scale bytes uint8 [..., K/16]). formats.py:123-128:
      s = e4m3(blockamax / (6 * g));  q = x / max(s * g, 1e-30);
      code = bucketize(min(|q|, 6), E2M1_BOUNDS) (a value on a midpoint takes the smaller magnitude);
      the sign bit is set when q < 0 and the code is not 0; element 2i goes to the low nibble of byte i.
    ``saturate`` selects the E4M3 overflow rule (see e4m3_encode); the reference's cast is saturate=False."""
    x = np.asarray(x, dtype=np.float32)
    g = F32(g)
    shape = x.shape
    k = shape[-1]
    if k % 16:
        raise ValueError(f'row length {k} is not a multiple of 16')
    blocks = x.reshape(-1, k // 16, 16)
    bamax = np.abs(blocks).max(-1)
    s_bytes = e4m3_encode(bamax / (F32(6.0) * g), saturate=saturate)
    denom = np.maximum(e4m3_decode(s_bytes) * g, F32(1e-30))
    with np.errstate(invalid='ignore', divide='ignore'):
        q = blocks / denom[..., None]
    mag = np.minimum(np.abs(q), F32(6.0))     # NaN stays NaN
    code = np.searchsorted(E2M1_BOUNDS, mag.ravel(), side='left').reshape(mag.shape).astype(np.uint8)
    code |= (((q < 0) & (code > 0)).astype(np.uint8) << 3)
    code = code.reshape(-1, k)
    pay = (code[:, 0::2] | (code[:, 1::2] << 4)).astype(np.uint8)
    return pay.reshape(*shape[:-1], k // 2), s_bytes.reshape(*shape[:-1], k // 16)


def nvfp4_encode(x):
    """formats.py:114-128 on a matrix/tensor x (last dim a multiple of 16): (payload, scale bytes, g)."""
    x = np.asarray(x, dtype=np.float32)
    g = global_scale(x)
    pay, sc = quantize_blocks(x, g, saturate=False)
    return pay, sc, g


def unpack_codes(pay):
    """payload [..., K/2] -> codes [..., K] (element 2i = low nibble of byte i)."""
    pay = np.asarray(pay, dtype=np.uint8)
    return np.stack([pay & 15, pay >> 4], -1).reshape(*pay.shape[:-1], pay.shape[-1] * 2)


def dequant(pay, sc, g=1.0):
    """(e2m1 * e4m3) * g in FP32, in this order (qsa_fp4.py:96-101): float32 [..., K]."""
    vals = e2m1_decode(unpack_codes(pay))
    scales = np.repeat(e4m3_decode(sc), 16, axis=-1)
    with np.errstate(invalid='ignore'):
        return (vals * scales) * F32(g)


def dequant_unscaled(pay, sc):
    """e2m1 * e4m3 (no global scale): exact in float16 and bfloat16 (at most 6 significant bits, 2^-10 .. 2688)."""
    return dequant(pay, sc, 1.0)
