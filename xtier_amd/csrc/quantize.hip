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

// The E2M1 code of q = x / d as formats.py:124-127 computes it, without the division. For a midpoint m of the code
// table, fl(|x| / d) > m holds exactly when |x| / d > m + ulp(m) / 2 (every midpoint has an even last mantissa bit, so
// the tie rounds down to m), i.e. when |x| > t_m * d. That product (25 by 24 significant bits) is exact in FP64, and a
// BF16 |x| exceeds a real T exactly when it exceeds T rounded toward -inf to BF16. So the seven thresholds of a block
// are formed once as BF16 bit patterns: the FP64 product truncated to BF16 precision (rounding a positive value
// toward -inf), capped at the largest finite BF16. d must be positive and finite (d >= 1e-30 keeps every product a
// normal BF16 magnitude).
__device__ inline void block_thresholds(float d, uint32_t (&t2)[7]) {
  // m + ulp(m) / 2 for m = 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5 (ulp(m) = 2^(e - 23), e the exponent of m)
  constexpr double kMid[7] = {0.25 + 0x1p-26, 0.75 + 0x1p-25, 1.25 + 0x1p-24, 1.75 + 0x1p-24, 2.5 + 0x1p-23,
                              3.5 + 0x1p-23, 5.0 + 0x1p-22};
  const double dd = (double)d;
#pragma unroll
  for (int i = 0; i < 7; ++i) {
    const uint32_t hi = (uint32_t)((uint64_t)__double_as_longlong(kMid[i] * dd) >> 32);
    // FP64 high word: exponent (bias 1023) in bits 20-30 and the top 20 mantissa bits; BF16: exponent (bias 127)
    // in bits 7-14 and the top 7 mantissa bits
    const uint32_t tb = min((hi >> 13) - ((1023u - 127u) << 7), 0x7F7Fu);
    t2[i] = tb | (tb << 16);
  }
}

// Per 16-bit half: 0xFFFF where the half, as a signed integer, is negative, else 0. Written as inline asm so that the
// compiler keeps the masks as data for single-instruction bitfield selects (it would otherwise rebuild each select
// as two per-half compares and selects and a permute). The operand must be an ordinary VALU result.
__device__ inline uint32_t pk_neg_mask(uint32_t x) {
  uint32_t r;
  asm("v_pk_ashrrev_i16 %0, 15, %1 op_sel_hi:[0,1]" : "=v"(r) : "v"(x));   // the constant 15 for both halves
  return r;
}
typedef short short2v __attribute__((ext_vector_type(2)));
typedef unsigned short ushort2v __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pk_sub16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2v, a) - __builtin_bit_cast(short2v, b));
}
__device__ inline uint32_t select_bits(uint32_t m, uint32_t a, uint32_t b) { return (m & a) | (~m & b); }

// Two E2M1 codes at once from one dword of two BF16 values, with the thresholds of block_thresholds. Non-negative
// BF16 values order as their bit patterns, so |x| > T holds exactly when bits(T) - bits(|x|) is negative (both below
// 2^15); the code is a three-level search over the seven thresholds on both 16-bit halves at once, each level's
// threshold picked by a bitfield select under the masks of the levels above. The sign bit goes with a code above 0
// when x < 0. No value is a NaN here: a NaN anywhere in a block makes its scale, hence d, a NaN, and such a block
// takes the division form. An infinite value exceeds every (finite) threshold and codes 7. Returns the byte of the two
// codes (first value in the low nibble).
__device__ inline uint32_t e2m1_pair(uint32_t w, const uint32_t (&t2)[7]) {
  const uint32_t a = w & 0x7FFF7FFFu;
  const uint32_t m4 = pk_neg_mask(pk_sub16(t2[3], a));
  const uint32_t m2 = pk_neg_mask(pk_sub16(select_bits(m4, t2[5], t2[1]), a));
  const uint32_t t1 = select_bits(m4, select_bits(m2, t2[6], t2[4]), select_bits(m2, t2[2], t2[0]));
  const uint32_t m1 = pk_neg_mask(pk_sub16(t1, a));
  const uint32_t code = (m4 & 0x00040004u) | (m2 & 0x00020002u) | (m1 & 0x00010001u);
  const uint32_t c = code | ((w >> 12) & 0x00080008u & (m4 | m2 | m1));
  return (c & 0xFu) | ((c >> 12) & 0xF0u);
}

// The division form, for a block whose d is not finite (a NaN or infinite global scale, or a NaN in the block).
__device__ inline uint32_t e2m1_code_div(float x, float d) {
  const float q = x / d;
  const float a_ = __builtin_fabsf(q);
  uint32_t code = (uint32_t)(a_ > 0.25f) + (uint32_t)(a_ > 0.75f) + (uint32_t)(a_ > 1.25f) + (uint32_t)(a_ > 1.75f) +
                  (uint32_t)(a_ > 2.5f) + (uint32_t)(a_ > 3.5f) + (uint32_t)(a_ > 5.0f);
  if (q != q) code = 7u;
  if (q < 0.0f && code > 0u) code |= 8u;
  return code;
}

// 16 BF16 values (eight dwords) -> eight payload bytes (two dwords) and the E4M3 scale byte, with global scale g.
// The block maximum is a packed 16-bit maximum of the magnitudes' bit patterns (a NaN's exceeds every finite one's, so
// a NaN wins as in torch's amax); the scale byte's value comes from the hardware E4M3 -> FP16 conversion (exact for
// every byte, NaN for 0x7F / 0xFF).
__device__ inline void quantize_block(const uint32_t (&w)[8], float g, bool saturate, uint32_t (&packed)[2],
                                      uint32_t& sbyte) {
  ushort2v mx = {0, 0};
#pragma unroll
  for (int k = 0; k < 8; ++k) mx = __builtin_elementwise_max(mx, __builtin_bit_cast(ushort2v, w[k] & 0x7FFF7FFFu));
  const float bamax = bf16_bits_to_f32(max((uint32_t)mx.x, (uint32_t)mx.y));
  sbyte = e4m3_encode(bamax / (6.0f * g), saturate);
  float d = (float)fp8x2_to_f16<false>(sbyte).x * g;
  d = (d < 1e-30f) ? 1e-30f : d;
  packed[0] = packed[1] = 0u;
  if (__builtin_isfinite(d)) {
    uint32_t t2[7];
    block_thresholds(d, t2);
#pragma unroll
    for (int k = 0; k < 8; ++k) packed[k >> 2] |= e2m1_pair(w[k], t2) << (8 * (k & 3));
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float x = bf16_bits_to_f32(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xFFFFu);
      packed[e >> 3] |= e2m1_code_div(x, d) << (4 * (e & 7));
    }
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
  uint32_t packed[2], sbyte;
  quantize_block(w, *gp, saturate != 0, packed, sbyte);
  uint2 outw;
  outw.x = packed[0];
  outw.y = packed[1];
  *reinterpret_cast<uint2*>(pay + slot * pay_stride + h * pay_hs + blk * 8) = outw;
  sf[slot * sf_stride + h * sf_hs + blk] = (uint8_t)sbyte;
}

// One launch writes every tensor of a KV append into its pool at the rows' slots: grid row k (blockIdx.y) is store k,
// so its descriptor is uniform over the workgroup (scalar loads); within a store, units of 16 values (row r, head h,
// block b) are numbered row by row, so consecutive threads read consecutive 32-byte pieces of a row and write its
// consecutive payload pieces and scale bytes. A store with g == NULL copies its BF16 values.
constexpr int kMaxStores = 4;
struct StoreArgs {
  xt_kv_store st[kMaxStores];
  uint64_t head_magic[kMaxStores];       // ceil(2^40 / heads): n / heads = (n * magic) >> 40 for every n < 2^31
  int block_shift[kMaxStores];           // log2(dim / 16)
  int n_stores;
  int64_t n_rows;
  const int64_t* slots;
  int64_t pool_slots;
  int page_shift;                        // log2(rows per page); 0: token-major
  int saturate;
};

// 16-value units per thread, their loads all in flight before the first use. One: the block arithmetic (about 270
// VALU instructions per unit) is the larger cost, so more waves in flight beat more loads per wave (a 4096-row K + V
// append: 4.6 us at one unit per thread, 5.0 at two, 6.0 at four, graph-replayed).
constexpr int kStoreUnits = 1;

// Unit i of a thread is (blockIdx.x * kStoreUnits + i) * 256 + threadIdx.x: one 16-value block (32 source bytes, 8
// payload bytes, a scale byte), consecutive threads taking consecutive blocks of a row.
__global__ __launch_bounds__(256) void store_kv_kernel(const StoreArgs a) {
  const xt_kv_store& st = a.st[blockIdx.y];
  const int bs = a.block_shift[blockIdx.y];
  const uint64_t magic = a.head_magic[blockIdx.y];
  const uint32_t heads = (uint32_t)st.heads;
  const int64_t units = (a.n_rows * st.heads) << bs;
  uint32_t u[kStoreUnits];
  int64_t slot[kStoreUnits];
  uint4 lo[kStoreUnits], hi[kStoreUnits];
#pragma unroll
  for (int i = 0; i < kStoreUnits; ++i) {
    u[i] = (blockIdx.x * kStoreUnits + i) * 256u + threadIdx.x;   // < 2^31, checked on the host
    const bool in = (int64_t)u[i] < units;
    const uint32_t uu = in ? u[i] : 0u;
    const uint32_t b = uu & ((1u << bs) - 1), rh = uu >> bs;
    const uint32_t r = (uint32_t)(((uint64_t)rh * magic) >> 40), h = rh - r * heads;
    slot[i] = in ? a.slots[r] : -1;
    const uint16_t* src =
        static_cast<const uint16_t*>(st.src) + (int64_t)r * st.src_row_stride + (int64_t)h * st.src_head_stride + 16 * b;
    lo[i] = reinterpret_cast<const uint4*>(src)[0];
    hi[i] = reinterpret_cast<const uint4*>(src)[1];
  }
  // the global scale (written by an earlier launch, so a scalar load) joins them; the empty asm takes every load
  // before the slot tests, so none is sunk below a test
  int32_t gbits = st.g ? uniform_load(reinterpret_cast<const int32_t*>(st.g)) : 0;
#pragma unroll
  for (int i = 0; i < kStoreUnits; ++i)
    asm volatile("" : "+v"(slot[i]), "+v"(lo[i].x), "+v"(lo[i].y), "+v"(lo[i].z), "+v"(lo[i].w), "+v"(hi[i].x),
                 "+v"(hi[i].y), "+v"(hi[i].z), "+v"(hi[i].w));
  asm volatile("" : "+s"(gbits));
  const float g = __int_as_float(gbits);
#pragma unroll
  for (int i = 0; i < kStoreUnits; ++i) {
    if (slot[i] < 0 || slot[i] >= a.pool_slots) continue;
    const uint32_t b = u[i] & ((1u << bs) - 1), rh = u[i] >> bs;
    const uint32_t h = rh - (uint32_t)(((uint64_t)rh * magic) >> 40) * heads;
    const int64_t page = slot[i] >> a.page_shift, prow = slot[i] & ((1ll << a.page_shift) - 1);
    uint8_t* pay = st.pay + page * st.pay_page_stride + prow * st.pay_row_stride + (int64_t)h * st.pay_head_stride;
    if (st.g == nullptr) {   // a plain copy of the BF16 values
      reinterpret_cast<uint4*>(pay + 32 * b)[0] = lo[i];
      reinterpret_cast<uint4*>(pay + 32 * b)[1] = hi[i];
      continue;
    }
    const uint32_t w[8] = {lo[i].x, lo[i].y, lo[i].z, lo[i].w, hi[i].x, hi[i].y, hi[i].z, hi[i].w};
    uint32_t packed[2], sbyte;
    quantize_block(w, g, a.saturate != 0, packed, sbyte);
    *reinterpret_cast<uint2*>(pay + 8 * b) = make_uint2(packed[0], packed[1]);
    st.scales[page * st.sf_page_stride + prow * st.sf_row_stride + (int64_t)h * st.sf_head_stride + b] =
        (uint8_t)sbyte;
  }
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

extern "C" int xt_nvfp4_store_kv(const xt_kv_store* stores, int n_stores, int64_t n_rows, const int64_t* slots,
                                 int64_t pool_slots, int page_size, int saturate, xt_stream_t stream) {
  const char* what = "xt_nvfp4_store_kv";
  if (!stores || n_stores < 1 || n_stores > kMaxStores)
    return fail(XT_EINVAL, "%s: 1 to %d stores expected, got %d", what, kMaxStores, n_stores);
  if (n_rows < 0 || page_size <= 0 || (page_size & (page_size - 1)) || pool_slots <= 0)
    return fail(XT_EINVAL, "%s: n_rows %lld, page_size %d (a power of 2), pool_slots %lld", what, (long long)n_rows,
                page_size, (long long)pool_slots);
  if (n_rows == 0) return ok();
  if (!slots) return fail(XT_EINVAL, "%s: slots is null", what);
  StoreArgs a;
  a.n_stores = n_stores;
  a.n_rows = n_rows;
  a.slots = slots;
  a.pool_slots = pool_slots;
  a.page_shift = __builtin_ctz((unsigned)page_size);
  a.saturate = saturate;
  int64_t most = 0;   // 16-value units of the largest store
  for (int k = 0; k < kMaxStores; ++k) {
    if (k >= n_stores) {
      a.st[k] = stores[0];
      a.head_magic[k] = 1ull << 40;
      a.block_shift[k] = 0;
      continue;
    }
    const xt_kv_store& st = stores[k];
    if (int e = check_src(what, st.src, n_rows, st.heads, st.dim, st.src_row_stride, st.src_head_stride)) return e;
    if ((st.dim / 16) & (st.dim / 16 - 1) || st.heads > 512)
      return fail(XT_EINVAL, "%s: store %d: dim %d (dim / 16 must be a power of 2), heads %d (at most 512)", what, k,
                  st.dim, st.heads);
    const bool copy = st.g == nullptr;
    const int64_t row_bytes = copy ? 2 * st.dim : st.dim / 2;
    if (!st.pay || (!copy && !st.scales))
      return fail(XT_EINVAL, "%s: store %d: a payload%s pointer is required", what, k, copy ? "" : " and a scale");
    if (!aligned(st.pay, copy ? 16 : 8) || st.pay_page_stride % 8 || st.pay_row_stride % 8 || st.pay_head_stride % 8 ||
        (copy && (st.pay_page_stride % 16 || st.pay_row_stride % 16 || st.pay_head_stride % 16)))
      return fail(XT_EINVAL, "%s: store %d: payload address and strides must be multiples of %d bytes", what, k,
                  copy ? 16 : 8);
    if (st.pay_page_stride < 0 || st.pay_row_stride < 0 || st.pay_head_stride < 0 || st.sf_page_stride < 0 ||
        st.sf_row_stride < 0 || st.sf_head_stride < 0 ||
        (st.heads > 1 && st.pay_head_stride < row_bytes) ||
        (!copy && st.heads > 1 && st.sf_head_stride < st.dim / 16))
      return fail(XT_EINVAL, "%s: store %d: strides must be non-negative and keep the heads' rows apart", what, k);
    a.st[k] = st;
    a.head_magic[k] = ((1ull << 40) + (uint64_t)st.heads - 1) / (uint64_t)st.heads;
    a.block_shift[k] = __builtin_ctz((unsigned)(st.dim / 16));
    most = std::max<int64_t>(most, n_rows * st.heads * (st.dim / 16));
  }
  if (most > 0x7FFFF000LL) return fail(XT_EUNSUPPORTED, "%s: %lld rows is too many for one launch", what,
                                       (long long)n_rows);
  const int64_t blocks = (most + 256 * kStoreUnits - 1) / (256 * kStoreUnits);
  hipLaunchKernelGGL(store_kv_kernel, dim3((unsigned)blocks, (unsigned)n_stores), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(what);
}
