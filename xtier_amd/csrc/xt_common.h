// Device helpers shared by the NVFP4 kernels (gfx950 only).
//
// NVFP4 as stored in the KV pool: payload byte i of a head row holds element 2i in bits 0-3 and element 2i+1 in
// bits 4-7 (an E2M1 code: sign bit 3, magnitude index into {0, .5, 1, 1.5, 2, 3, 4, 6}); one OCP E4M3 scale byte per
// 16 elements; value = (e2m1 * e4m3) * g with g the per-tensor FP32 global scale.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/xtier_amd.h"

namespace xt {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef short short2_t __attribute__((ext_vector_type(2)));
typedef uint32_t xt_u32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// FP32 -> E4M3 (fn) byte with round-to-nearest-even. Below 2^-6 the magnitude is rounded in subnormal steps of
// 2^-9; from 2^-6 up the FP32 bits are rounded at mantissa bit 20, a carry moving into the exponent. A magnitude
// that rounds above 448 becomes 448 (saturate) or NaN 0x7F (as torch's float8_e4m3fn cast); NaN becomes 0x7F.
// The sign bit is kept in every case.
__host__ __device__ inline uint32_t e4m3_encode(float x, bool saturate) {
  uint32_t bits;
  __builtin_memcpy(&bits, &x, 4);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t a = bits & 0x7FFFFFFFu;
  uint32_t code;
  if (a > 0x7F800000u) {
    code = 0x7Fu;
  } else if (a < 0x3C800000u) {
    float f;
    __builtin_memcpy(&f, &a, 4);
    code = (uint32_t)__builtin_rintf(f * 512.0f);   // exact scaling; rint rounds half to even
  } else {
    const uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
    code = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
    if (code > 0x7Eu) code = saturate ? 0x7Eu : 0x7Fu;
  }
  return code | sign;
}

// E4M3 (fn) byte -> FP32: e > 0 is 2^(e-7) * (1 + m/8), e = 0 is m * 2^-9, 0x7F / 0xFF are NaN.
__host__ __device__ inline float e4m3_decode(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float mag;
  if ((b & 0x7Fu) == 0x7Fu) {
    mag = __builtin_nanf("");
  } else if (e == 0) {
    mag = (float)m * 0.001953125f;
  } else {
    const uint32_t fb = ((e + 120u) << 23) | (m << 20);
    __builtin_memcpy(&mag, &fb, 4);
  }
  return (b & 0x80u) ? -mag : mag;
}

#if defined(__HIP_DEVICE_COMPILE__)
// Two E2M1 codes (byte `sel` of `packed`: low nibble first) -> two exact FP32 values. The conversion's scale operand
// contributes only its exponent, so it is 1.0 here and block scales are applied separately.
template <int SEL>
__device__ inline float2_t fp4x2_to_f32(uint32_t packed) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(packed, 1.0f, SEL);
}
template <int SEL>
__device__ inline half2_t fp4x2_to_f16(uint32_t packed) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(packed, 1.0f, SEL);
}
// Two E4M3 bytes (bytes 0,1 or 2,3 of `packed`) -> two exact FP16 values (every E4M3 value is an FP16 value).
template <bool HI>
__device__ inline half2_t fp8x2_to_f16(uint32_t packed) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(packed, 1.0f, HI);
}
// Eight E4M3 bytes (low byte first) -> eight exact FP16 values in the same order.
__device__ inline half8_t fp8x8_to_f16(uint64_t v) {
  const half2_t a = fp8x2_to_f16<false>((uint32_t)v), b = fp8x2_to_f16<true>((uint32_t)v);
  const half2_t c = fp8x2_to_f16<false>((uint32_t)(v >> 32)), d = fp8x2_to_f16<true>((uint32_t)(v >> 32));
  return half8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
// A load through the scalar cache (the constant address space) of memory no launch writes: uniform per-row values.
__device__ inline int32_t uniform_load(const int32_t* p) {
  return *(const __attribute__((address_space(4))) int32_t*)(p);
}
__device__ inline float uniform_load_f32(const float* p) {
  return *(const __attribute__((address_space(4))) float*)(p);
}
// Maxima of scores as single instructions. fmaxf first quiets each operand (v_max_f32 x, x) wherever the compiler
// cannot prove it already canonical (results of permutes, values merged from branches); attention scores are never
// signalling NaNs, so these skip that step. The operands must be results of ordinary VALU instructions: the compiler
// inserts no wait states in front of inline asm, so an MFMA accumulator read here could still be in flight.
__device__ inline float max2_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ inline float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// Maximum and sum of x over lanes l, l ^ 16 and l ^ 32 (the four lanes 16 apart), in VALU permutes: with x as both
// operands, v_permlane16_swap / v_permlane32_swap hand every lane the pair (x[l], x[l ^ 16]) / (x[l], x[l ^ 32]),
// in an order that does not matter here (ds_bpermute would take two LDS round trips).
__device__ inline float max4_lanes16(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = max2_raw(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return max2_raw(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float sum4_lanes16(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// The power of two 2^e that brings a head's largest query magnitude `qmax` into [2^10, 2^11): the query enters FP16
// MFMA operands as q * 2^-e, exactly for every element down to 2^-24 of qmax (BF16's 8 significant bits fit FP16's
// 11 within its normal range; smaller elements weigh less than that in any score), and 2^e multiplies the FP32
// scores. Zero, subnormal, infinite or NaN maxima give e = 0; e is kept
// in [-100, 100]. Returns {2^-e, 2^e}.
__device__ inline float2_t pow2_query_scale(float qmax) {
  const int biased = (int)(__float_as_uint(qmax) >> 23) & 0xFF;
  int e = (biased == 0 || biased == 255) ? 0 : biased - 127 - 10;
  e = e < -100 ? -100 : e > 100 ? 100 : e;
  return float2_t{__uint_as_float((uint32_t)(127 - e) << 23), __uint_as_float((uint32_t)(127 + e) << 23)};
}
// Split arrival: the workgroups of one output (key splits of a row) leave partial results in a workspace and count
// their arrivals; the last to arrive merges. The protocol keeps every access to the shared partials coherent by
// itself, so no fence has to write back or invalidate a whole L2 (an agent-scope release fence is a buffer_wbl2 and
// an acquire a buffer_inv; on the batch-32 decode's 256 workgroups the two cost 2.4 us per launch):
//   1. every thread stores its pieces of the partial with sc1 (written through to memory, the coherence point of all
//      XCDs; the bits of an agent-scope atomic store), then waits for their completion (s_waitcnt vmcnt(0));
//   2. a workgroup barrier, then thread 0 counts the arrival with a system-scope atomic add (sc1: performed at memory,
//      coherent whichever XCD the workgroups ran on); it is issued after every store of the workgroup completed;
//   3. the workgroup that sees the count reach splits - 1 passes a second barrier and reads the partials with sc0 sc1
//      (missing L1 and any L2 copy, so the reads come from memory), issued after the count returned.
// Every partial a last arriver reads was therefore complete in memory before its count, and the count is what the
// last arriver waited for. The last arriver resets the counter (a system-scope store) for the next call.
__device__ inline void store_partial(__amdgpu_buffer_rsrc_t r, int byte_off, float4_t v) {
  const xt_u32x4_t w = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  __builtin_amdgcn_raw_buffer_store_b128(w, r, byte_off, 0, 16 /* sc1 */);
}
__device__ inline float4_t load_partial(__amdgpu_buffer_rsrc_t r, int byte_off) {
  const xt_u32x4_t w = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 17 /* sc0 sc1 */);
  return float4_t{__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]), __uint_as_float(w[3])};
}
// The same for four values held as FP16 (8 bytes): RNE on the way out, exact on the way back.
__device__ inline void store_partial_h4(__amdgpu_buffer_rsrc_t r, int byte_off, float4_t v) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  const half2_t a = __builtin_convertvector(float2_t{v[0], v[1]}, half2_t);
  const half2_t b = __builtin_convertvector(float2_t{v[2], v[3]}, half2_t);
  const u32x2_t w = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
  __builtin_amdgcn_raw_buffer_store_b64(w, r, byte_off, 0, 16 /* sc1 */);
}
__device__ inline float4_t load_partial_h4(__amdgpu_buffer_rsrc_t r, int byte_off) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  const u32x2_t w = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 17 /* sc0 sc1 */);
  // (the words go through scalars: a bit cast of a vector element directly has read element 0 here)
  const uint32_t w0 = w[0], w1 = w[1];
  const half2_t a = __builtin_bit_cast(half2_t, w0), b = __builtin_bit_cast(half2_t, w1);
  return float4_t{(float)a[0], (float)a[1], (float)b[0], (float)b[1]};
}
// Called by every thread after its partial stores. True in every thread of the workgroup that arrived last among
// `splits`. `flag` is a __shared__ int of the caller.
__device__ inline bool arrive_last(int32_t* counter, int splits, int* flag) {
  __builtin_amdgcn_s_waitcnt(0);   // this thread's partial stores are complete
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == splits - 1;
  __syncthreads();
  return *flag;
}
__device__ inline void reset_counter(int32_t* counter) {
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
#else
// The host pass parses device code without the gfx950 builtins; these declarations are never code-generated.
__device__ float2_t pow2_query_scale(float qmax);
__device__ void store_partial(__amdgpu_buffer_rsrc_t r, int byte_off, float4_t v);
__device__ float4_t load_partial(__amdgpu_buffer_rsrc_t r, int byte_off);
__device__ void store_partial_h4(__amdgpu_buffer_rsrc_t r, int byte_off, float4_t v);
__device__ float4_t load_partial_h4(__amdgpu_buffer_rsrc_t r, int byte_off);
__device__ bool arrive_last(int32_t* counter, int splits, int* flag);
__device__ void reset_counter(int32_t* counter);
template <int SEL>
__device__ float2_t fp4x2_to_f32(uint32_t packed);
template <int SEL>
__device__ half2_t fp4x2_to_f16(uint32_t packed);
template <bool HI>
__device__ half2_t fp8x2_to_f16(uint32_t packed);
__device__ half8_t fp8x8_to_f16(uint64_t v);
__device__ float max2_raw(float a, float b);
__device__ float max3_raw(float a, float b, float c);
__device__ float max4_lanes16(float x);
__device__ int32_t uniform_load(const int32_t* p);
__device__ float uniform_load_f32(const float* p);
__device__ float sum4_lanes16(float x);
#endif

// FP32 -> BF16 bits, round to nearest even; NaN -> a quiet NaN with its sign. On the device this is gfx950's
// v_cvt_pk_bf16_f32 (one instruction, two values when the compiler pairs the calls; denormals kept, as the kernels
// run with FP32 denormals on), whose NaN keeps the top of its payload; the host spells the rounding out and returns
// the canonical 0x7FC0.
__host__ __device__ inline uint32_t f32_to_bf16_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  uint32_t b;
  __builtin_memcpy(&b, &f, 4);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return ((b >> 16) & 0x8000u) | 0x7FC0u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
#endif
}
__host__ __device__ inline float bf16_bits_to_f32(uint32_t h) {
  const uint32_t b = h << 16;
  float f;
  __builtin_memcpy(&f, &b, 4);
  return f;
}
__host__ __device__ inline uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}
// Two FP32 values -> two BF16 (BF) or FP16 values, round to nearest even, `lo` in bits 0..15. On the device: one
// v_cvt_pk_bf16_f32, or two v_cvt_f16_f32 and a pack.
template <bool BF>
__host__ __device__ inline uint32_t pack2_16(float lo, float hi) {
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (BF) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, bf16x2_t));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, half2_t));
  }
#else
  return BF ? f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16) : f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
#endif
}

}  // namespace xt
