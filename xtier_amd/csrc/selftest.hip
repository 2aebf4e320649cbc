// Known-answer test of the hardware conversions the attention kernels rely on: every E4M3 byte and every byte of two
// E2M1 codes through exactly the helpers and builtins the kernels call, written to a caller buffer for the host to
// compare with the format tables.
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

// V4 scale exponents checked for the scaled E4M3 -> BF16 conversion (2^(e - 127): 2^-7, 1, 2^7).
__constant__ uint32_t kV4Exps[3] = {120, 127, 134};

// One workgroup of 256 threads, thread b = byte b. Output (uint16 units):
//   [0, 256)        fp8x2_to_f16<false>(b).x           (E4M3 byte in the low half)
//   [256, 512)      fp8x2_to_f16<true>(b << 16).x      (E4M3 byte in the high half)
//   [512, 2560)     fp4x2_to_f16<SEL>(b << 8 SEL), SEL = 0..3: the result dword of each (element 0 first)
//   [2560, 3328)    cvt_scalef32_pk_bf16_fp8(b, 2^(e - 127)) for the three exponents above
// then FP32 (two uint16 units each) at [3328, 3328 + 2 * 2048): fp4x2_to_f32<SEL>(b << 8 SEL), SEL = 0..3.
__global__ __launch_bounds__(256) void conversions_kernel(uint16_t* out) {
  const uint32_t b = threadIdx.x;
  out[b] = __builtin_bit_cast(uint16_t, fp8x2_to_f16<false>(b).x);
  out[256 + b] = __builtin_bit_cast(uint16_t, fp8x2_to_f16<true>(b << 16).x);
  const half2_t h[4] = {fp4x2_to_f16<0>(b), fp4x2_to_f16<1>(b << 8), fp4x2_to_f16<2>(b << 16),
                        fp4x2_to_f16<3>(b << 24)};
  uint32_t* pairs = reinterpret_cast<uint32_t*>(out + 512);   // each pair stored as the dword the conversion wrote
#pragma unroll
  for (int s = 0; s < 4; ++s) pairs[s * 256 + b] = __builtin_bit_cast(uint32_t, h[s]);
#pragma unroll
  for (int e = 0; e < 3; ++e) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t p = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(b, __uint_as_float(kV4Exps[e] << 23), false);
    out[2560 + e * 256 + b] = __builtin_bit_cast(uint16_t, p.x);
  }
  float* f = reinterpret_cast<float*>(out + 3328);
  const float2_t v[4] = {fp4x2_to_f32<0>(b), fp4x2_to_f32<1>(b << 8), fp4x2_to_f32<2>(b << 16),
                         fp4x2_to_f32<3>(b << 24)};
#pragma unroll
  for (int s = 0; s < 4; ++s) reinterpret_cast<float2_t*>(f)[s * 256 + b] = v[s];
}

}  // namespace
}  // namespace xt

extern "C" size_t xt_selftest_conversions_bytes(void) { return (3328 + 2 * 2048) * sizeof(uint16_t); }

extern "C" int xt_selftest_conversions(void* out, xt_stream_t stream) {
  if (!out || !xt::aligned(out, 16)) return xt::fail(XT_EINVAL, "xt_selftest_conversions: a 16-byte aligned buffer");
  hipLaunchKernelGGL(xt::conversions_kernel, dim3(1), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<uint16_t*>(out));
  return xt::check_launch("xt_selftest_conversions");
}
