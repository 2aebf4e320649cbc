// NVFP4 quantization on the device: the per-tensor global scale and quantize-on-append into the paged pool.
//
// Rounding follows xtier/backend/formats.py:114-128 step by step in FP32 with IEEE division (no reciprocal
// approximation, no contraction): g = max(amax / 2688, 1e-12); s = e4m3(blockamax / (6 * g));
// q = x / max(s * g, 1e-30); code = number of E2M1 midpoints {.25, .75, 1.25, 1.75, 2.5, 3.5, 5} strictly below |q|
// (torch.bucketize: a value on a midpoint takes the smaller magnitude; NaN gives 7); sign when q < 0 and code > 0.
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

__global__ void amax_init_kernel(uint32_t* ws) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *ws = 0u;
}

// Maximum of |x| over a strided BF16 tensor as FP32 bits (non-negative floats order as unsigned integers; NaN's bits
// exceed every finite value's, so a NaN wins as in torch's amax).
__global__ void amax_kernel(const uint16_t* __restrict__ src, int64_t n_rows, int heads, int dim, int64_t rs,
                            int64_t hs, uint32_t* __restrict__ ws) {
  const int chunks = dim / 8;
  const int64_t total = n_rows * heads * chunks;
  uint32_t m = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % chunks);
    const int64_t rh = i / chunks;
    const int h = (int)(rh % heads);
    const int64_t r = rh / heads;
    const uint4 v = *reinterpret_cast<const uint4*>(src + r * rs + (int64_t)h * hs + c * 8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      m = max(m, (w[k] & 0x7FFFu) << 16);
      m = max(m, (w[k] >> 16 & 0x7FFFu) << 16);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off));
  if ((threadIdx.x & 63) == 0 && m != 0) atomicMax(ws, m);
}

__global__ void global_scale_kernel(const uint32_t* __restrict__ ws, float* __restrict__ g) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const uint32_t bits = *ws;
    float amax;
    __builtin_memcpy(&amax, &bits, 4);
    const float v = amax / 2688.0f;
    *g = (v < 1e-12f) ? 1e-12f : v;   // a NaN stays NaN, as torch's clamp_min
  }
}

// One thread per 16-element block: read 32 bytes of BF16, write 8 bytes of payload and one scale byte.
__global__ void quantize_append_kernel(const uint16_t* __restrict__ src, int64_t n_rows, int heads, int dim,
                                       int64_t rs, int64_t hs, const int64_t* __restrict__ slots,
                                       const float* __restrict__ gp, uint8_t* __restrict__ pay,
                                       uint8_t* __restrict__ sf, int64_t pool_slots, int64_t pay_stride,
                                       int64_t sf_stride, int64_t pay_hs, int64_t sf_hs, int saturate) {
  const int blocks = dim / 16;
  const int64_t total = n_rows * heads * blocks;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int blk = (int)(i % blocks);
  const int64_t rh = i / blocks;
  const int h = (int)(rh % heads);
  const int64_t r = rh / heads;
  const int64_t slot = slots[r];
  if (slot < 0 || slot >= pool_slots) return;
  const uint16_t* p = src + r * rs + (int64_t)h * hs + blk * 16;
  const uint4 a = reinterpret_cast<const uint4*>(p)[0];
  const uint4 b = reinterpret_cast<const uint4*>(p)[1];
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float x[16];
  uint32_t amax_bits = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    x[2 * k] = bf16_bits_to_f32(w[k] & 0xFFFFu);
    x[2 * k + 1] = bf16_bits_to_f32(w[k] >> 16);
    amax_bits = max(amax_bits, w[k] & 0x7FFFu);
    amax_bits = max(amax_bits, (w[k] >> 16) & 0x7FFFu);
  }
  const float g = *gp;
  const float six_g = 6.0f * g;
  const float bamax = bf16_bits_to_f32(amax_bits);
  const uint32_t sbyte = e4m3_encode(bamax / six_g, saturate != 0);
  float denom = e4m3_decode(sbyte) * g;
  denom = (denom < 1e-30f) ? 1e-30f : denom;
  uint32_t packed[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float q = x[e] / denom;
    const float a_ = __builtin_fabsf(q);
    uint32_t code = (uint32_t)(a_ > 0.25f) + (uint32_t)(a_ > 0.75f) + (uint32_t)(a_ > 1.25f) +
                    (uint32_t)(a_ > 1.75f) + (uint32_t)(a_ > 2.5f) + (uint32_t)(a_ > 3.5f) + (uint32_t)(a_ > 5.0f);
    if (q != q) code = 7u;
    if (q < 0.0f && code > 0u) code |= 8u;
    packed[e >> 3] |= code << (4 * (e & 7));
  }
  uint2 outw;
  outw.x = packed[0];
  outw.y = packed[1];
  *reinterpret_cast<uint2*>(pay + slot * pay_stride + h * pay_hs + blk * 8) = outw;
  sf[slot * sf_stride + h * sf_hs + blk] = (uint8_t)sbyte;
}

int check_src(const char* what, const void* src, int64_t n_rows, int heads, int dim, int64_t rs, int64_t hs) {
  if (n_rows < 0 || heads <= 0 || dim <= 0 || dim % 16 != 0)
    return fail(XT_EINVAL, "%s: bad shape n_rows=%lld heads=%d dim=%d (dim must be a positive multiple of 16)", what,
                (long long)n_rows, heads, dim);
  if (n_rows > 0 && (src == nullptr || !aligned(src, 16) || rs % 8 != 0 || hs % 8 != 0 || rs < 0 || hs < 0))
    return fail(XT_EINVAL, "%s: source rows must be 16-byte aligned (strides %lld, %lld elements)", what,
                (long long)rs, (long long)hs);
  return XT_OK;
}

}  // namespace
}  // namespace xt

using namespace xt;

extern "C" int xt_nvfp4_global_scale(const void* src, int64_t n_rows, int heads, int dim, int64_t src_row_stride,
                                     int64_t src_head_stride, float* g_out, void* workspace, xt_stream_t stream) {
  const char* what = "xt_nvfp4_global_scale";
  if (int e = check_src(what, src, n_rows, heads, dim, src_row_stride, src_head_stride)) return e;
  if (g_out == nullptr || workspace == nullptr || !aligned(workspace, 4))
    return fail(XT_EINVAL, "%s: g_out and a 4-byte aligned workspace are required", what);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint32_t* ws = static_cast<uint32_t*>(workspace);
  hipLaunchKernelGGL(amax_init_kernel, dim3(1), dim3(64), 0, s, ws);
  const int64_t total = n_rows * heads * (dim / 8);
  if (total > 0) {
    const int64_t blocks = std::min<int64_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(amax_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<const uint16_t*>(src),
                       n_rows, heads, dim, src_row_stride, src_head_stride, ws);
  }
  hipLaunchKernelGGL(global_scale_kernel, dim3(1), dim3(64), 0, s, ws, g_out);
  return check_launch(what);
}

extern "C" int xt_nvfp4_quantize_append(const void* src, int64_t n_rows, int heads, int dim, int64_t src_row_stride,
                                        int64_t src_head_stride, const int64_t* slots, const float* g, uint8_t* pay,
                                        uint8_t* scales, int64_t pool_slots, int64_t pay_stride, int64_t sf_stride,
                                        int64_t pay_head_stride, int64_t sf_head_stride, int saturate,
                                        xt_stream_t stream) {
  const char* what = "xt_nvfp4_quantize_append";
  if (int e = check_src(what, src, n_rows, heads, dim, src_row_stride, src_head_stride)) return e;
  if (n_rows == 0) return ok();
  if (slots == nullptr || g == nullptr || pay == nullptr || scales == nullptr || pool_slots <= 0)
    return fail(XT_EINVAL, "%s: slots, g, payload and scales are required (pool_slots %lld)", what,
                (long long)pool_slots);
  if (pay_head_stride == 0) pay_head_stride = dim / 2;
  if (sf_head_stride == 0) sf_head_stride = dim / 16;
  if (pay_stride == 0) pay_stride = (int64_t)heads * pay_head_stride;
  if (sf_stride == 0) sf_stride = (int64_t)heads * sf_head_stride;
  if (!aligned(pay, 8) || pay_stride % 8 || pay_head_stride % 8 || pay_head_stride < dim / 2 ||
      sf_head_stride < dim / 16 || pay_stride < (int64_t)(heads - 1) * pay_head_stride + dim / 2 ||
      sf_stride < (int64_t)(heads - 1) * sf_head_stride + dim / 16)
    return fail(XT_EINVAL, "%s: payload must be 8-byte aligned with slot and head strides (%lld, %lld) that are "
                "multiples of 8 and hold the heads' rows; scale strides %lld, %lld", what, (long long)pay_stride,
                (long long)pay_head_stride, (long long)sf_stride, (long long)sf_head_stride);
  const int64_t total = n_rows * heads * (dim / 16);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7FFFFFFF) return fail(XT_EUNSUPPORTED, "%s: %lld rows is too many for one launch", what,
                                       (long long)n_rows);
  hipLaunchKernelGGL(quantize_append_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(src), n_rows, heads, dim,
                     src_row_stride, src_head_stride, slots, g, pay, scales, pool_slots, pay_stride, sf_stride,
                     pay_head_stride, sf_head_stride, saturate);
  return check_launch(what);
}
