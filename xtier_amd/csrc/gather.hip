// QSA decode gather and prefill packing over the NVFP4 pool: bit-exact dequantized rows.
//
// Each value is (e2m1 * e4m3) * g computed as two FP32 multiplies in this order and rounded to nearest even into the
// output dtype, as xtier/packs/qwen4_exp/qsa_fp4.py:94-101 and :142-143 compute it. A thread handles 8-value pieces
// (one payload dword and its scale byte in, 16 bytes out), several of them 256 apart with all loads in flight together;
// the pieces of a request are numbered in output order, so a wave's stores cover consecutive bytes.
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

// Eight values of one NVFP4 block (one payload dword, its E4M3 scale byte), (e2m1 * e4m3) * g in FP32 in this order
// (qsa_fp4.py:96-101), rounded to BF16 or FP16 (round to nearest even).
__device__ inline uint4 dequant_piece(uint32_t w, uint32_t sbyte, float g, int out_dtype) {
  const float s = e4m3_decode(sbyte);
  const float2_t v[4] = {fp4x2_to_f32<0>(w), fp4x2_to_f32<1>(w), fp4x2_to_f32<2>(w), fp4x2_to_f32<3>(w)};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = (v[e].x * s) * g, b = (v[e].y * s) * g;
    o[e] = out_dtype == XT_DTYPE_BF16 ? f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16)
                                      : f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Eight E4M3 values (two dwords of an FP8 pool row, qsa_fp4.py:104-116) -> BF16 or FP16: every E4M3 value is exact in
// both, so the conversion is the software decode then the (exact) narrowing; a NaN byte gives a NaN.
__device__ inline uint4 fp8_piece(uint2 w, int out_dtype) {
  const uint32_t b[2] = {w.x, w.y};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t word = b[e >> 1] >> (16 * (e & 1));
    const float a = e4m3_decode(word & 0xFFu), c = e4m3_decode((word >> 8) & 0xFFu);
    o[e] = out_dtype == XT_DTYPE_BF16 ? f32_to_bf16_bits(a) | (f32_to_bf16_bits(c) << 16)
                                      : f32_to_f16_bits(a) | (f32_to_f16_bits(c) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// 8-value output pieces per thread, 256 apart (all loads issued before the first use). Four rather than eight: twice
// the workgroups, more than fit at once, so later ones gather while earlier ones write (gather / pack of config 2:
// 45.2 / 45.0 us at eight, 41.8 / 41.4 us at four, 42.3 / 41.7 us at two).
constexpr int kPieces = 4;

// Decode gather (qsa_fp4.py:119-143): request b = blockIdx.y; its output is a run of 8-value pieces (column c, head h,
// piece) in output order, so every store of a wave writes 1 KiB of consecutive rows. Column c < num_cols is valid when
// c < cu_k[b+1] - cu_k[b], its position indices[b, c] (c < topk) lies in [0, seq_lens[b]) (and below the table's row
// pitch) and the slot
// req_to_token[req_indices[b], pos] in [0, pool_slots); valid columns are dequantized into rows cu_k[b] + c, invalid
// ones are zeros when zero_fill (columns up to num_cols) and skipped otherwise.
template <bool FP8>
__global__ __launch_bounds__(256) void qsa_gather_kernel(
    const uint8_t* __restrict__ k_pay, const uint8_t* __restrict__ v_pay, const uint8_t* __restrict__ k_sf,
    const uint8_t* __restrict__ v_sf, const float* __restrict__ gk, const float* __restrict__ gv, int64_t pool_slots,
    int heads, int piece_shift, const int32_t* __restrict__ req_to_token, int64_t req_stride,
    const int64_t* __restrict__ req_indices, const int32_t* __restrict__ indices, int64_t idx_stride,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ cu_k, uint16_t* __restrict__ out_k,
    uint16_t* __restrict__ out_v, int out_dtype, int topk, int num_cols, int zero_fill) {
  const int b = blockIdx.y;
  const int32_t start = cu_k[b];
  const int32_t valid_count = cu_k[b + 1] - start;
  // positions past the table row's pitch are invalid, whatever seq_lens says (no read past the row)
  const int32_t length = req_stride > 0 ? (int32_t)min((int64_t)seq_lens[b], req_stride) : seq_lens[b];
  const int32_t* tp = req_to_token + req_indices[b] * req_stride;
  const int pieces = 1 << piece_shift;
  const int items = num_cols * heads * pieces;
  int c[kPieces], h[kPieces], pc[kPieces];
  int32_t pos[kPieces];
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const int g = (blockIdx.x * kPieces + u) * 256 + (int)threadIdx.x;
    pc[u] = g & (pieces - 1);
    const int hc = g >> piece_shift;
    c[u] = hc / heads;
    h[u] = hc - c[u] * heads;
    pos[u] = (g < items && c[u] < topk && c[u] < valid_count) ? indices[(int64_t)b * idx_stride + c[u]] : -1;
  }
  int64_t slot[kPieces];
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    slot[u] = (pos[u] >= 0 && pos[u] < length) ? tp[pos[u]] : -1;
  }
  // NVFP4: 4 payload bytes and a scale byte per piece; FP8: 8 bytes of E4M3 values
  constexpr int kPieceBytes = FP8 ? 8 : 4;
  uint2 kw[kPieces], vw[kPieces];
  uint32_t ks[kPieces], vs[kPieces];
  const int64_t row_bytes = (int64_t)heads * (pieces * kPieceBytes), row_scales = (int64_t)heads * (pieces / 2);
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const bool valid = slot[u] >= 0 && slot[u] < pool_slots;   // a slot outside the pool reads as invalid
    const int64_t sl = valid ? slot[u] : 0;
    const int64_t po = sl * row_bytes + (int64_t)h[u] * (pieces * kPieceBytes) + pc[u] * kPieceBytes;
    if constexpr (FP8) {
      kw[u] = valid ? *reinterpret_cast<const uint2*>(k_pay + po) : make_uint2(0u, 0u);
      vw[u] = valid ? *reinterpret_cast<const uint2*>(v_pay + po) : make_uint2(0u, 0u);
    } else {
      const int64_t so = sl * row_scales + (int64_t)h[u] * (pieces / 2) + (pc[u] >> 1);
      kw[u].x = valid ? *reinterpret_cast<const uint32_t*>(k_pay + po) : 0u;
      vw[u].x = valid ? *reinterpret_cast<const uint32_t*>(v_pay + po) : 0u;
      ks[u] = valid ? k_sf[so] : 0u;
      vs[u] = valid ? v_sf[so] : 0u;
    }
    if (!valid) slot[u] = -1;
  }
  const float g_k = FP8 ? 1.0f : *gk, g_v = FP8 ? 1.0f : *gv;
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const int g = (blockIdx.x * kPieces + u) * 256 + (int)threadIdx.x;
    if (g >= items || (slot[u] < 0 && !zero_fill)) continue;
    const int64_t dst = ((int64_t)(start + c[u]) * heads + h[u]) * (pieces * 8) + pc[u] * 8;
    if constexpr (FP8) {
      *reinterpret_cast<uint4*>(out_k + dst) = fp8_piece(kw[u], out_dtype);
      *reinterpret_cast<uint4*>(out_v + dst) = fp8_piece(vw[u], out_dtype);
    } else {
      *reinterpret_cast<uint4*>(out_k + dst) = dequant_piece(kw[u].x, ks[u], g_k, out_dtype);
      *reinterpret_cast<uint4*>(out_v + dst) = dequant_piece(vw[u].x, vs[u], g_v, out_dtype);
    }
  }
}

// Prefix pack (qsa_fp4.py:146-162): request b = blockIdx.y writes its first cu_k[b+1] - cu_k[b] positions, in order,
// into rows cu_k[b] + t, as 8-value pieces in output order (see qsa_gather_kernel); a slot outside the pool reads as
// zeros.
template <bool FP8>
__global__ __launch_bounds__(256) void qsa_pack_kernel(
    const uint8_t* __restrict__ k_pay, const uint8_t* __restrict__ v_pay, const uint8_t* __restrict__ k_sf,
    const uint8_t* __restrict__ v_sf, const float* __restrict__ gk, const float* __restrict__ gv, int64_t pool_slots,
    int heads, int piece_shift, const int32_t* __restrict__ req_to_token, int64_t sr0, int64_t sr1,
    const int64_t* __restrict__ req_indices, const int32_t* __restrict__ cu_k, uint16_t* __restrict__ out_k,
    uint16_t* __restrict__ out_v, int out_dtype) {
  const int b = blockIdx.y;
  const int32_t start = cu_k[b];
  const int pieces = 1 << piece_shift;
  const int items = (cu_k[b + 1] - start) * heads * pieces;
  const int32_t* tp = req_to_token + req_indices[b] * sr0;
  int t[kPieces], h[kPieces], pc[kPieces];
  int64_t slot[kPieces];
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const int g = (blockIdx.x * kPieces + u) * 256 + (int)threadIdx.x;
    pc[u] = g & (pieces - 1);
    const int ht = g >> piece_shift;
    t[u] = ht / heads;
    h[u] = ht - t[u] * heads;
    slot[u] = g < items ? tp[(int64_t)t[u] * sr1] : -1;
  }
  constexpr int kPieceBytes = FP8 ? 8 : 4;
  uint2 kw[kPieces], vw[kPieces];
  uint32_t ks[kPieces], vs[kPieces];
  const int64_t row_bytes = (int64_t)heads * (pieces * kPieceBytes), row_scales = (int64_t)heads * (pieces / 2);
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const bool valid = slot[u] >= 0 && slot[u] < pool_slots;
    const int64_t sl = valid ? slot[u] : 0;
    const int64_t po = sl * row_bytes + (int64_t)h[u] * (pieces * kPieceBytes) + pc[u] * kPieceBytes;
    if constexpr (FP8) {
      kw[u] = valid ? *reinterpret_cast<const uint2*>(k_pay + po) : make_uint2(0u, 0u);
      vw[u] = valid ? *reinterpret_cast<const uint2*>(v_pay + po) : make_uint2(0u, 0u);
    } else {
      const int64_t so = sl * row_scales + (int64_t)h[u] * (pieces / 2) + (pc[u] >> 1);
      kw[u].x = valid ? *reinterpret_cast<const uint32_t*>(k_pay + po) : 0u;
      vw[u].x = valid ? *reinterpret_cast<const uint32_t*>(v_pay + po) : 0u;
      ks[u] = valid ? k_sf[so] : 0u;
      vs[u] = valid ? v_sf[so] : 0u;
    }
  }
  const float g_k = FP8 ? 1.0f : *gk, g_v = FP8 ? 1.0f : *gv;
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const int g = (blockIdx.x * kPieces + u) * 256 + (int)threadIdx.x;
    if (g >= items) continue;
    const int64_t dst = ((int64_t)(start + t[u]) * heads + h[u]) * (pieces * 8) + pc[u] * 8;
    if constexpr (FP8) {
      *reinterpret_cast<uint4*>(out_k + dst) = fp8_piece(kw[u], out_dtype);
      *reinterpret_cast<uint4*>(out_v + dst) = fp8_piece(vw[u], out_dtype);
    } else {
      *reinterpret_cast<uint4*>(out_k + dst) = dequant_piece(kw[u].x, ks[u], g_k, out_dtype);
      *reinterpret_cast<uint4*>(out_v + dst) = dequant_piece(vw[u].x, vs[u], g_v, out_dtype);
    }
  }
}

constexpr int kDequantPieces = 8;

// One request's context from head-major NVFP4 pages into BF16 rows (kv_fp4.py:496-530). Grid (x, request b). The
// output of a request is a sequence of 8-value pieces (position, head, piece; piece fastest); a thread takes
// kDequantPieces of them, 256 apart, so every store of a wave writes 1 KiB of consecutive output and 16 lanes read one
// head's 64-byte row. Token slot s = req_to_token[sid, pos] wrapped into [0, pages * block) as the reference wraps
// it, at page s / block, row s % block (block a power of 2); all loads of a thread issue before the first use. The
// products e2m1 * e4m3 have at most 5 significant bits, so the upper half of their FP32 bits is the BF16 value (NaN
// stays NaN).
__global__ __launch_bounds__(256) void paged_dequant_kernel(
    const uint8_t* __restrict__ pay, const uint8_t* __restrict__ sf, int64_t max_slots, int heads, int piece_shift,
    int block_shift, int64_t page_stride, int64_t head_stride, int64_t row_stride, int64_t sf_page_stride,
    int64_t sf_head_stride, int64_t sf_row_stride, const int32_t* __restrict__ req_to_token, int64_t req_stride,
    const int64_t* __restrict__ slot_ids, const int32_t* __restrict__ seq_lens, int rows_per_req,
    uint16_t* __restrict__ out) {
  constexpr int U = kDequantPieces;
  const int b = blockIdx.y;
  const int len = min(seq_lens[b], rows_per_req);
  int64_t sid = slot_ids[b];
  if ((uint64_t)sid >= (uint64_t)max_slots) sid = (sid % max_slots + max_slots) % max_slots;
  const int32_t* tp = req_to_token + sid * req_stride;
  int pos[U], h[U], pc[U];
  int32_t ent[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int g = (blockIdx.x * U + u) * 256 + (int)threadIdx.x;
    pc[u] = g & ((1 << piece_shift) - 1);
    const int hp = g >> piece_shift;
    pos[u] = hp / heads;
    h[u] = hp - pos[u] * heads;
    ent[u] = pos[u] < len ? tp[pos[u]] : 0;
  }
  uint32_t w[U], sb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int64_t slot = ent[u];
    if ((uint64_t)slot >= (uint64_t)max_slots) slot = (slot % max_slots + max_slots) % max_slots;
    const int64_t page = slot >> block_shift, row = slot & ((1 << block_shift) - 1);
    const uint8_t* p = pay + page * page_stride + (int64_t)h[u] * head_stride + row * row_stride + pc[u] * 4;
    const uint8_t* q = sf + page * sf_page_stride + (int64_t)h[u] * sf_head_stride + row * sf_row_stride + (pc[u] >> 1);
    if (pos[u] >= len) p = pay, q = sf;     // a valid address; the values are not stored
    w[u] = *reinterpret_cast<const uint32_t*>(p);
    sb[u] = *q;
  }
  uint16_t* base = out + (int64_t)b * rows_per_req * heads * (8 << piece_shift);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (pos[u] >= len) continue;
    const float s = e4m3_decode(sb[u]);
    const float2_t v[4] = {fp4x2_to_f32<0>(w[u]), fp4x2_to_f32<1>(w[u]), fp4x2_to_f32<2>(w[u]),
                           fp4x2_to_f32<3>(w[u])};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = v[e].x * s, hi = v[e].y * s;
      uint32_t a, bb;
      __builtin_memcpy(&a, &lo, 4);
      __builtin_memcpy(&bb, &hi, 4);
      o[e] = (a >> 16) | (bb & 0xFFFF0000u);
    }
    const int g = (blockIdx.x * U + u) * 256 + (int)threadIdx.x;
    *reinterpret_cast<uint4*>(base + (int64_t)g * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

int check_pool(const char* what, bool fp8, const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_sf,
               const uint8_t* v_sf, const float* gk, const float* gv, int64_t pool_slots, int heads, int dim) {
  // the reference's precondition (qsa_fp4.py:165-171): a power-of-2 head size, a multiple of 32
  if (heads <= 0 || dim < 32 || (dim & (dim - 1)) != 0)
    return fail(XT_EINVAL, "%s: packed [m, heads, %s] rows with a power-of-2 head size >= 32 expected, got "
                "heads=%d dim=%d", what, fp8 ? "dim" : "dim/2", heads, dim);
  if (!k_pay || !v_pay || (!fp8 && (!k_sf || !v_sf || !gk || !gv)) || pool_slots <= 0)
    return fail(XT_EINVAL, "%s: pool buffers%s are required (pool_slots %lld)", what,
                fp8 ? "" : " and global scales", (long long)pool_slots);
  if (!aligned(k_pay, 8) || !aligned(v_pay, 8)) return fail(XT_EINVAL, "%s: payload must be 8-byte aligned", what);
  return XT_OK;
}

}  // namespace
}  // namespace xt

using namespace xt;

template <bool FP8>
static int gather_impl(const char* what, const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                       const uint8_t* v_scales, const float* gk, const float* gv, int64_t pool_slots, int heads, int dim,
                       const int32_t* req_to_token, int64_t req_stride, const int64_t* req_indices,
                       const int32_t* indices, int64_t idx_stride, const int32_t* seq_lens, const int32_t* cu_k,
                       void* out_k, void* out_v, int out_dtype, int batch, int topk, int zero_fill_cols,
                       xt_stream_t stream) {
  if (int e = check_pool(what, FP8, k_pay, v_pay, k_scales, v_scales, gk, gv, pool_slots, heads, dim)) return e;
  if (out_dtype != XT_DTYPE_BF16 && out_dtype != XT_DTYPE_F16)
    return fail(XT_EINVAL, "%s: output dtype must be BF16 or FP16", what);
  if (batch < 0 || topk < 0 || zero_fill_cols < 0) return fail(XT_EINVAL, "%s: negative batch/topk/zero_fill", what);
  const int num_cols = zero_fill_cols > 0 ? zero_fill_cols : topk;
  if (batch == 0 || num_cols == 0) return ok();
  if (!req_to_token || !req_indices || !indices || !seq_lens || !cu_k || !out_k || !out_v)
    return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (!aligned(out_k, 16) || !aligned(out_v, 16)) return fail(XT_EINVAL, "%s: outputs must be 16-byte aligned", what);
  const int64_t per_req = (int64_t)num_cols * heads * (dim / 8);
  if (per_req > 0x7FFFFFFFLL - 256 * kPieces || batch > 65535)
    return fail(XT_EUNSUPPORTED, "%s: %lld pieces per request or %d requests", what, (long long)per_req, batch);
  const dim3 grid((unsigned)((per_req + 256 * kPieces - 1) / (256 * kPieces)), (unsigned)batch);
  hipLaunchKernelGGL(qsa_gather_kernel<FP8>, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), k_pay, v_pay,
                     k_scales, v_scales, gk, gv, pool_slots, heads, __builtin_ctz((unsigned)(dim / 8)), req_to_token,
                     req_stride, req_indices, indices, idx_stride, seq_lens, cu_k, static_cast<uint16_t*>(out_k),
                     static_cast<uint16_t*>(out_v), out_dtype, topk, num_cols, zero_fill_cols > 0 ? 1 : 0);
  return check_launch(what);
}

template <bool FP8>
static int pack_impl(const char* what, const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                     const uint8_t* v_scales, const float* gk, const float* gv, int64_t pool_slots, int heads, int dim,
                     const int32_t* req_to_token, int64_t sr0, int64_t sr1, const int64_t* req_indices, int batch,
                     const int32_t* cu_k, int max_k, void* out_k, void* out_v, int out_dtype, xt_stream_t stream) {
  if (int e = check_pool(what, FP8, k_pay, v_pay, k_scales, v_scales, gk, gv, pool_slots, heads, dim)) return e;
  if (out_dtype != XT_DTYPE_BF16 && out_dtype != XT_DTYPE_F16)
    return fail(XT_EINVAL, "%s: output dtype must be BF16 or FP16", what);
  if (batch < 0 || max_k < 0) return fail(XT_EINVAL, "%s: negative batch/max_k", what);
  if (batch == 0 || max_k == 0) return ok();
  if (!req_to_token || !req_indices || !cu_k || !out_k || !out_v)
    return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (!aligned(out_k, 16) || !aligned(out_v, 16)) return fail(XT_EINVAL, "%s: outputs must be 16-byte aligned", what);
  const int64_t per_req = (int64_t)max_k * heads * (dim / 8);
  if (per_req > 0x7FFFFFFFLL - 256 * kPieces || batch > 65535)
    return fail(XT_EUNSUPPORTED, "%s: %lld pieces per request or %d requests", what, (long long)per_req, batch);
  const dim3 grid((unsigned)((per_req + 256 * kPieces - 1) / (256 * kPieces)), (unsigned)batch);
  hipLaunchKernelGGL(qsa_pack_kernel<FP8>, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), k_pay, v_pay,
                     k_scales, v_scales, gk, gv, pool_slots, heads, __builtin_ctz((unsigned)(dim / 8)), req_to_token,
                     sr0, sr1, req_indices, cu_k, static_cast<uint16_t*>(out_k), static_cast<uint16_t*>(out_v),
                     out_dtype);
  return check_launch(what);
}

extern "C" int xt_qsa_gather_nvfp4(const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                                   const uint8_t* v_scales, const float* gk, const float* gv, int64_t pool_slots,
                                   int heads, int dim, const int32_t* req_to_token, int64_t req_stride,
                                   const int64_t* req_indices, const int32_t* indices, int64_t idx_stride,
                                   const int32_t* seq_lens, const int32_t* cu_k, void* out_k, void* out_v,
                                   int out_dtype, int batch, int topk, int zero_fill_cols, xt_stream_t stream) {
  if (!aligned(k_pay, 8) || !aligned(v_pay, 8))
    return fail(XT_EINVAL, "xt_qsa_gather_nvfp4: payload must be 8-byte aligned");
  return gather_impl<false>("xt_qsa_gather_nvfp4", k_pay, v_pay, k_scales, v_scales, gk, gv, pool_slots, heads, dim,
                            req_to_token, req_stride, req_indices, indices, idx_stride, seq_lens, cu_k, out_k, out_v,
                            out_dtype, batch, topk, zero_fill_cols, stream);
}

extern "C" int xt_qsa_gather_fp8(const uint8_t* k, const uint8_t* v, int64_t pool_slots, int heads, int dim,
                                 const int32_t* req_to_token, int64_t req_stride, const int64_t* req_indices,
                                 const int32_t* indices, int64_t idx_stride, const int32_t* seq_lens,
                                 const int32_t* cu_k, void* out_k, void* out_v, int out_dtype, int batch, int topk,
                                 int zero_fill_cols, xt_stream_t stream) {
  if (!aligned(k, 8) || !aligned(v, 8)) return fail(XT_EINVAL, "xt_qsa_gather_fp8: K / V must be 8-byte aligned");
  return gather_impl<true>("xt_qsa_gather_fp8", k, v, nullptr, nullptr, nullptr, nullptr, pool_slots, heads, dim,
                           req_to_token, req_stride, req_indices, indices, idx_stride, seq_lens, cu_k, out_k, out_v,
                           out_dtype, batch, topk, zero_fill_cols, stream);
}

extern "C" int xt_qsa_pack_nvfp4(const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                                 const uint8_t* v_scales, const float* gk, const float* gv, int64_t pool_slots,
                                 int heads, int dim, const int32_t* req_to_token, int64_t sr0, int64_t sr1,
                                 const int64_t* req_indices, int batch, const int32_t* cu_k, int max_k, void* out_k,
                                 void* out_v, int out_dtype, xt_stream_t stream) {
  if (!aligned(k_pay, 8) || !aligned(v_pay, 8))
    return fail(XT_EINVAL, "xt_qsa_pack_nvfp4: payload must be 8-byte aligned");
  return pack_impl<false>("xt_qsa_pack_nvfp4", k_pay, v_pay, k_scales, v_scales, gk, gv, pool_slots, heads, dim,
                          req_to_token, sr0, sr1, req_indices, batch, cu_k, max_k, out_k, out_v, out_dtype, stream);
}

extern "C" int xt_qsa_pack_fp8(const uint8_t* k, const uint8_t* v, int64_t pool_slots, int heads, int dim,
                               const int32_t* req_to_token, int64_t sr0, int64_t sr1, const int64_t* req_indices,
                               int batch, const int32_t* cu_k, int max_k, void* out_k, void* out_v, int out_dtype,
                               xt_stream_t stream) {
  if (!aligned(k, 8) || !aligned(v, 8)) return fail(XT_EINVAL, "xt_qsa_pack_fp8: K / V must be 8-byte aligned");
  return pack_impl<true>("xt_qsa_pack_fp8", k, v, nullptr, nullptr, nullptr, nullptr, pool_slots, heads, dim,
                         req_to_token, sr0, sr1, req_indices, batch, cu_k, max_k, out_k, out_v, out_dtype, stream);
}

// Per-row count of valid top-k entries (0 <= index < seq_lens[b]) and their running sum cu[0] = 0, cu[b + 1] =
// cu[b] + count[b]: one workgroup, a wave per row, then a scan over the rows in LDS.
__global__ __launch_bounds__(1024) void valid_counts_kernel(const int32_t* __restrict__ seq_lens,
                                                            const int32_t* __restrict__ indices, int64_t idx_stride,
                                                            int batch, int topk, int32_t* __restrict__ counts,
                                                            int32_t* __restrict__ cu) {
  __shared__ int32_t part[1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int r = wave; r < batch; r += 16) {
    const int32_t len = seq_lens[r];
    int n = 0;
    for (int c = lane; c < topk; c += 64) {
      const int32_t i = indices[(int64_t)r * idx_stride + c];
      n += (i >= 0 && i < len);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) n += __shfl_xor(n, off);
    if (lane == 0) counts[r] = n;
  }
  __syncthreads();
  // each thread sums a contiguous run of rows, the runs are scanned across the workgroup, then written out
  const int per = (batch + 1023) / 1024;
  const int r0 = threadIdx.x * per, r1 = min(batch, r0 + per);
  int local = 0;
  for (int r = r0; r < r1; ++r) local += counts[r];
  part[threadIdx.x] = local;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int add = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
    __syncthreads();
    part[threadIdx.x] += add;
    __syncthreads();
  }
  int run = part[threadIdx.x] - local;   // rows before r0
  if (threadIdx.x == 0) cu[0] = 0;
  for (int r = r0; r < r1; ++r) {
    run += counts[r];
    cu[r + 1] = run;
  }
}

extern "C" int xt_qsa_valid_counts(const int32_t* seq_lens, const int32_t* indices, int64_t idx_stride, int batch,
                                   int topk, int32_t* valid_counts, int32_t* cu_seqlens_k, xt_stream_t stream) {
  const char* what = "xt_qsa_valid_counts";
  if (batch < 0 || topk < 0) return fail(XT_EINVAL, "%s: negative batch / topk", what);
  if (!cu_seqlens_k || (batch > 0 && (!seq_lens || !valid_counts || (topk > 0 && !indices))))
    return fail(XT_EINVAL, "%s: a required pointer is null", what);
  hipLaunchKernelGGL(valid_counts_kernel, dim3(1), dim3(1024), 0, reinterpret_cast<hipStream_t>(stream), seq_lens,
                     indices, idx_stride, batch, topk, valid_counts, cu_seqlens_k);
  return check_launch(what);
}

extern "C" int xt_dequantize_context_nvfp4(const uint8_t* pay, const uint8_t* scales, int64_t pages, int heads,
                                           int dim, int block_size, int64_t page_stride, int64_t head_stride,
                                           int64_t row_stride, int64_t sf_page_stride, int64_t sf_head_stride,
                                           int64_t sf_row_stride, const int32_t* req_to_token, int64_t req_stride,
                                           const int64_t* slot_ids, const int32_t* seq_lens, int batch,
                                           int rows_per_req, void* out, xt_stream_t stream) {
  const char* what = "xt_dequantize_context_nvfp4";
  if (heads <= 0 || dim < 32 || (dim & (dim - 1)) || block_size <= 0 || (block_size & (block_size - 1)) ||
      pages <= 0 || batch < 0 || rows_per_req < 0)
    return fail(XT_EINVAL, "%s: bad heads %d / dim %d / block %d (a power of 2) / pages %lld / batch / rows", what, heads, dim,
                block_size, (long long)pages);
  if (row_stride < dim / 2 || sf_row_stride < dim / 16 || row_stride % 8 || page_stride < (int64_t)block_size *
      row_stride || sf_page_stride < (int64_t)block_size * sf_row_stride || head_stride < 0 || sf_head_stride < 0)
    return fail(XT_EINVAL, "%s: pool strides do not describe [pages, heads, %d, dim/2] pages", what, block_size);
  if (batch == 0 || rows_per_req == 0) return ok();
  if (!pay || !scales || !req_to_token || !slot_ids || !seq_lens || !out || !aligned(pay, 8) || !aligned(out, 16))
    return fail(XT_EINVAL, "%s: a required pointer is null or misaligned", what);
  const int64_t per_req = (int64_t)rows_per_req * heads * (dim / 8);
  if (per_req > 0x7FFFFFFFLL - 256 * kDequantPieces || batch > 65535)
    return fail(XT_EUNSUPPORTED, "%s: %lld pieces per request or %d requests", what, (long long)per_req, batch);
  const dim3 grid((unsigned)((per_req + 256 * kDequantPieces - 1) / (256 * kDequantPieces)), (unsigned)batch);
  hipLaunchKernelGGL(paged_dequant_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), pay, scales,
                     pages * block_size, heads, __builtin_ctz((unsigned)(dim / 8)),
                     __builtin_ctz((unsigned)block_size), page_stride, head_stride, row_stride, sf_page_stride,
                     sf_head_stride, sf_row_stride, req_to_token, req_stride, slot_ids, seq_lens, rows_per_req,
                     static_cast<uint16_t*>(out));
  return check_launch(what);
}
