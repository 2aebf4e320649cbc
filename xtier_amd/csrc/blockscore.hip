// MiniMax index block scores over the NVFP4 index K: the scores SGLang's top-k selection of KV blocks reads
// (kv_fp4.py:168-222 decode, :407-446 prefill). The index pool holds one key head per slot: payload bytes
// [pages, 128 slots, d/2] (element 2i in the low nibble of byte i) and E4M3 scale bytes [pages, 128, d/16]
// (element j uses scale j / 16), unit global scale; a slot s lives on page s / 128, row s % 128.
//
//   score of key position p for head h = (q_h . k_p) * c with c = (sm_scale * log2(e)) * k_scale in FP32.
//   decode: per request, head and block of block_size positions, the maximum (or log2-sum-exp2) of the scores of the
//     block's positions below seq_len; the last local_blocks blocks read 1e29, else the first init_blocks 1e30.
//   prefill: per query row, head and block, the maximum over the block's positions at or before the row's own
//     position (prefix_len + row), -inf when there are none; a row gets the blocks below
//     min(seq_len, prefix_len + 64 (row / 64 + 1)), the 64-row tile bound of the reference's grid.
//
// Numerics: e2m1 * e4m3 has at most 6 significant bits, so every key value is exact in FP32 and in BF16 (FP16 for an
// FP16 query); v_mfma_f32_32x32x16_{bf16,f16} sums the exact products in FP32. The MFMA takes keys as rows
// (A = 32 keys x 16 dims) and query columns as columns (B = 16 dims x 32 columns); a lane then holds 16 keys of one
// column, so the block maximum is 15 VALU maxima in the lane and one exchange with the lane 32 apart. The dims of a
// lane half h are h d/2 .. h d/2 + d/2 - 1 (k-step kk covers h d/2 + 8 kk .. + 7 in both operands), so a lane reads
// one contiguous run of each key's payload.
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

typedef float float16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kPoolRows = 128;   // slots per page of the index pool
constexpr int kScoreWaves = 4;

// index arrays given as int32 or int64 (bit i of `wide` set: argument i is int64)
enum : int { kWideR2t = 1, kWideSeq = 2, kWideSlot = 4, kWidePrefix = 8, kWideCu = 16 };

__device__ inline int64_t load_index(const void* p, int64_t i, bool wide) {
  return wide ? static_cast<const int64_t*>(p)[i] : (int64_t) static_cast<const int32_t*>(p)[i];
}

// slot -> [0, max_slots): (s + max_slots) % max_slots for the reference's range s >= -max_slots, and kept in range
// for any other value
__device__ inline int64_t wrap_slot(int64_t s, int64_t max_slots) {
  const int64_t r = s % max_slots;
  return r < 0 ? r + max_slots : r;
}

struct ScoreArgs {
  const uint16_t* q;          // decode [batch, heads, d]; prefill [total_q, heads, d] (BF16 / FP16, d contiguous)
  int64_t q_ns, q_hs;         // element strides of a row (request / token) and a head
  const uint8_t* pay;         // index payload
  int64_t pay_ps, pay_rs;     // byte strides of a page and a slot row
  const uint8_t* sc;          // index scale bytes
  int64_t sc_ps, sc_rs;
  int64_t max_slots;          // pages * 128
  const void* r2t;            // req_to_token [reqs, width]
  int64_t r2t_stride;
  const void* seq_lens;
  const void* slot_ids;
  const void* prefix_lens;    // prefill
  const void* cu_seqlens;     // prefill [batch + 1]
  int wide;
  void* score;                // decode [heads, batch, blocks]; prefill [heads, total_q, blocks] (element strides)
  int64_t s_hs, s_ns, s_ks;
  int out_dtype;              // 0 FP32, 1 BF16, 2 FP16
  int batch, heads, block_size;
  float c;
  int init_blocks, local_blocks;
  int skip_topk;              // decode: a request with at most this many blocks gets no scores (-1: none skipped)
  int lse;                    // decode: log2-sum-exp2 instead of the maximum
  int chunks;                 // prefill: block ranges per row tile (grid x = row tiles * chunks)
  int chunk_blocks;           // prefill: blocks per range
};

__device__ inline void store_score(const ScoreArgs& a, int64_t at, float v) {
  if (a.out_dtype == 0)
    static_cast<float*>(a.score)[at] = v;
  else if (a.out_dtype == 1)
    static_cast<uint16_t*>(a.score)[at] = (uint16_t)f32_to_bf16_bits(v);
  else
    static_cast<uint16_t*>(a.score)[at] = (uint16_t)f32_to_f16_bits(v);
}

// Eight E2M1 codes (one dword, low nibble first) times the FP32 scale `sf`, as eight exact 16-bit values.
template <bool BF>
__device__ inline u32x4_t fp4x8_scaled(uint32_t w, float sf) {
  u32x4_t r;
  if constexpr (BF) {
    // the products are exact in FP32 with zero low halves, so their high halves are the BF16 values
#define XT_PAIR(E)                                                                                                 \
  {                                                                                                                \
    const float2_t v = fp4x2_to_f32<E>(w);                                                                         \
    r[E] = __builtin_amdgcn_perm(__float_as_uint(v.y * sf), __float_as_uint(v.x * sf), 0x07060302u);              \
  }
    XT_PAIR(0) XT_PAIR(1) XT_PAIR(2) XT_PAIR(3)
#undef XT_PAIR
  } else {
    const half2_t s2 = {(_Float16)sf, (_Float16)sf};
    r[0] = __builtin_bit_cast(uint32_t, fp4x2_to_f16<0>(w) * s2);
    r[1] = __builtin_bit_cast(uint32_t, fp4x2_to_f16<1>(w) * s2);
    r[2] = __builtin_bit_cast(uint32_t, fp4x2_to_f16<2>(w) * s2);
    r[3] = __builtin_bit_cast(uint32_t, fp4x2_to_f16<3>(w) * s2);
  }
  return r;
}

template <bool BF>
__device__ inline float16_t mfma16(u32x4_t a, u32x4_t b, float16_t c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                  0, 0, 0);
}

__device__ inline float scale_of(uint32_t byte) {
  return (float)fp8x2_to_f16<false>(byte)[0];
}

__device__ inline float swap32_max(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ inline float swap32_sum(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// ---------------------------------------------------------------------------------------------------------------
// Decode: grid (x, request b, head group of 32); wavefront w of workgroup x takes blocks x * 4 + w, + 4 gridDim.x,
// ... of its request; T = block_size / 32 key tiles per block, all held until the block's reduction.

template <int NK, int T, bool BF>
__global__ __launch_bounds__(64 * kScoreWaves) void decode_scores_kernel(const ScoreArgs a) {
  constexpr int D = 16 * NK;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  const int b = blockIdx.y;
  const int64_t seq = load_index(a.seq_lens, b, a.wide & kWideSeq);
  const int64_t nb = (seq + 32 * T - 1) / (32 * T);
  if (a.skip_topk >= 0 && nb <= a.skip_topk) return;
  int64_t blk = (int64_t)blockIdx.x * kScoreWaves + wave;
  if (blk >= nb) return;   // no barrier below
  const int64_t sid = wrap_slot(load_index(a.slot_ids, b, a.wide & kWideSlot), a.max_slots);
  const int head = 32 * blockIdx.z + j;
  const bool live_head = head < a.heads;
  // B = this lane's query column (head), dims h d/2 + 8 kk .. + 7
  u32x4_t qv[NK];
  {
    const uint16_t* qp = a.q + (int64_t)b * a.q_ns + (int64_t)(live_head ? head : 0) * a.q_hs + h * (D / 2);
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      qv[kk] = live_head ? *reinterpret_cast<const u32x4_t*>(qp + 8 * kk) : u32x4_t{0, 0, 0, 0};
  }
  const int64_t local_start = nb - a.local_blocks > 0 ? nb - a.local_blocks : 0;
  const bool wide_r2t = a.wide & kWideR2t;
  for (; blk < nb; blk += (int64_t)gridDim.x * kScoreWaves) {
    float16_t acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t pos = blk * (32 * T) + 32 * t + j;
      const int64_t slot = pos < seq ? wrap_slot(load_index(a.r2t, sid * a.r2t_stride + pos, wide_r2t), a.max_slots) : 0;
      const uint8_t* pp = a.pay + (slot >> 7) * a.pay_ps + (slot & (kPoolRows - 1)) * a.pay_rs + h * (D / 4);
      const uint8_t* sp = a.sc + (slot >> 7) * a.sc_ps + (slot & (kPoolRows - 1)) * a.sc_rs + h * (D / 32);
      uint32_t pw[NK];
#pragma unroll
      for (int i = 0; i < NK / 4; ++i) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(pp + 16 * i);
        pw[4 * i] = v[0]; pw[4 * i + 1] = v[1]; pw[4 * i + 2] = v[2]; pw[4 * i + 3] = v[3];
      }
      uint64_t sw;
      if constexpr (NK == 4) sw = *reinterpret_cast<const uint16_t*>(sp);
      else if constexpr (NK == 8) sw = *reinterpret_cast<const uint32_t*>(sp);
      else sw = *reinterpret_cast<const uint64_t*>(sp);
      float16_t s = {};
#pragma unroll
      for (int kk = 0; kk < NK; ++kk)
        s = mfma16<BF>(fp4x8_scaled<BF>(pw[kk], scale_of((uint32_t)(sw >> (8 * (kk / 2))) & 0xFFu)), qv[kk], s);
      acc[t] = s;
    }
    // C rows: keys 32 t + 8 (r / 4) + 4 h + r % 4 of the block; scaled, -inf at and past seq_len
    float m = -__builtin_inff();
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t pos = blk * (32 * T) + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
        acc[t][r] = pos < seq ? acc[t][r] * a.c : -__builtin_inff();
        m = fmaxf(m, acc[t][r]);
      }
    m = swap32_max(m);
    float score = m;
    if (a.lse) {
      float sum = 0.0f;
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) sum += exp2f(acc[t][r] - m);
      score = m + log2f(swap32_sum(sum));
      if (score != score) score = -__builtin_inff();
    }
    if (blk >= local_start) score = 1e29f;
    else if (blk < a.init_blocks) score = 1e30f;
    if (h == 0 && live_head) store_score(a, (int64_t)head * a.s_hs + (int64_t)b * a.s_ns + blk * a.s_ks, score);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Prefill: grid (row tile x block range, request b, head group of HPW heads); a workgroup covers R = 256 / HPW query
// rows of request b and one range of chunk_blocks blocks (the per-block results are independent, so ranges split a
// long prompt's work over many workgroups). Column j of wavefront w's column group g is (row (32 / HPW)(2 w + g) + j / HPW, head j % HPW).
// Key chunks of S = min(block_size, 128) positions are staged as 16-bit values in LDS by the whole workgroup (once
// for its 256 columns), then each wavefront runs its two column groups over them. Chunks wholly at or below every
// row's position skip the causal test and scale once after the maximum (c > 0: the maximum commutes with the
// rounding of the product).

constexpr int kStageKeys = 128;

template <int NK, int HPW, bool BF>
__global__ __launch_bounds__(64 * kScoreWaves) void prefill_scores_kernel(const ScoreArgs a) {
  constexpr int D = 16 * NK;
  constexpr int ROW_U32 = D / 2 + 4;          // LDS row: D 16-bit values + 16 bytes of padding
  constexpr int R = 256 / HPW;                // rows per workgroup
  constexpr int RG = 32 / HPW;                // rows per column group
  __shared__ uint32_t lds[kStageKeys * ROW_U32];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5, tid = threadIdx.x;
  const int b = blockIdx.y;
  const int64_t q0 = load_index(a.cu_seqlens, b, a.wide & kWideCu);
  const int64_t q_len = load_index(a.cu_seqlens, b + 1, a.wide & kWideCu) - q0;
  const int tiles = (int)gridDim.x / a.chunks, chunk = (int)blockIdx.x % a.chunks;
  const int64_t row0 = (int64_t)(tiles - 1 - (int)blockIdx.x / a.chunks) * R;   // the longest rows first
  if (row0 >= q_len) return;   // uniform over the workgroup: before every barrier
  const int64_t seq = load_index(a.seq_lens, b, a.wide & kWideSeq);
  const int64_t pre = load_index(a.prefix_lens, b, a.wide & kWidePrefix);
  const int64_t sid = wrap_slot(load_index(a.slot_ids, b, a.wide & kWideSlot), a.max_slots);
  const int bs = a.block_size;
  // rows of this lane's two columns, their heads and block counts
  int64_t row[2], nblk[2];
  bool live[2];
  u32x4_t qv[2][NK];
  const int head = HPW * blockIdx.z + (j % HPW);
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    row[g] = row0 + RG * (2 * wave + g) + j / HPW;
    live[g] = row[g] < q_len && head < a.heads;
    const int64_t hi = min(seq, pre + 64 * (row[g] / 64 + 1));
    nblk[g] = live[g] ? (hi + bs - 1) / bs : 0;
    const uint16_t* qp = a.q + (q0 + (live[g] ? row[g] : 0)) * a.q_ns + (int64_t)(live[g] ? head : 0) * a.q_hs +
                         h * (D / 2);
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      qv[g][kk] = live[g] ? *reinterpret_cast<const u32x4_t*>(qp + 8 * kk) : u32x4_t{0, 0, 0, 0};
  }
  // the workgroup's block count: that of its last live row (block counts grow with the row)
  const int64_t last = min(q_len, row0 + R) - 1;
  const int64_t wg_blocks = (min(seq, pre + 64 * (last / 64 + 1)) + bs - 1) / bs;
  const int64_t blk_lo = (int64_t)chunk * a.chunk_blocks, blk_hi = min(wg_blocks, blk_lo + a.chunk_blocks);
  if (blk_lo >= wg_blocks) return;   // uniform: before every barrier
  const int64_t first_pos = pre + row0;       // every row of the workgroup sees keys at or below this
  const bool wide_r2t = a.wide & kWideR2t;
  const int S = bs < kStageKeys ? bs : kStageKeys;
  const int chunks16 = S * NK;                // 16-value pieces per stage
  for (int64_t blk = blk_lo; blk < blk_hi; ++blk) {
    float m[2] = {-__builtin_inff(), -__builtin_inff()};    // scaled maxima of masked chunks
    float mr[2] = {-__builtin_inff(), -__builtin_inff()};   // raw maxima of unmasked chunks
    for (int sub = 0; sub < bs; sub += S) {
      const int64_t key0 = blk * bs + sub;
      __syncthreads();   // the previous stage's readers are done
      for (int c = tid; c < chunks16; c += 64 * kScoreWaves) {
        const int key = c / NK, kc = c % NK;
        const int64_t pos = key0 + key;
        const int64_t slot =
            pos < seq ? wrap_slot(load_index(a.r2t, sid * a.r2t_stride + pos, wide_r2t), a.max_slots) : 0;
        const uint8_t* pp = a.pay + (slot >> 7) * a.pay_ps + (slot & (kPoolRows - 1)) * a.pay_rs + 8 * kc;
        const uint8_t* sp = a.sc + (slot >> 7) * a.sc_ps + (slot & (kPoolRows - 1)) * a.sc_rs + kc;
        const uint2 w = *reinterpret_cast<const uint2*>(pp);
        const float sf = scale_of(*sp);
        *reinterpret_cast<u32x4_t*>(&lds[key * ROW_U32 + 8 * kc]) = fp4x8_scaled<BF>(w.x, sf);
        *reinterpret_cast<u32x4_t*>(&lds[key * ROW_U32 + 8 * kc + 4]) = fp4x8_scaled<BF>(w.y, sf);
      }
      __syncthreads();
      // every key of the chunk at or below every row's position and below seq_len, and c > 0
      const bool unmasked = key0 + S - 1 <= first_pos && key0 + S <= seq && a.c > 0.0f;
      for (int t = 0; t < S / 32; ++t) {
        float16_t s0 = {}, s1 = {};
        const uint32_t* kp = &lds[(32 * t + j) * ROW_U32 + h * (D / 4)];
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(kp + 4 * kk);
          s0 = mfma16<BF>(kv, qv[0][kk], s0);
          s1 = mfma16<BF>(kv, qv[1][kk], s1);
        }
        if (unmasked) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            mr[0] = fmaxf(mr[0], s0[r]);
            mr[1] = fmaxf(mr[1], s1[r]);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t pos = key0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
            // a key counts for a row at or after it, below seq_len
            m[0] = fmaxf(m[0], pos <= pre + row[0] && pos < seq ? s0[r] * a.c : -__builtin_inff());
            m[1] = fmaxf(m[1], pos <= pre + row[1] && pos < seq ? s1[r] * a.c : -__builtin_inff());
          }
        }
      }
    }
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      // max(round(c x)) = round(c max(x)) for c > 0
      const float v = swap32_max(fmaxf(m[g], mr[g] * a.c));
      if (h == 0 && blk < nblk[g]) store_score(a, (int64_t)head * a.s_hs + (q0 + row[g]) * a.s_ns + blk * a.s_ks, v);
    }
  }
}

}  // namespace
}  // namespace xt

using namespace xt;

namespace {

int score_common(const char* what, ScoreArgs& a, int dim, int q_dtype, const void* q, const void* pay,
                 const void* sc, const void* r2t, int64_t pay_ps, int64_t pay_rs, int64_t sc_ps, int64_t sc_rs,
                 void* scores, int score_dtype) {
  if (!q || !pay || !sc || !r2t || !scores || !a.seq_lens || !a.slot_ids)
    return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (dim != 64 && dim != 128 && dim != 256) return fail(XT_EUNSUPPORTED, "%s: head dim %d (64, 128 or 256)", what, dim);
  if (q_dtype != XT_DTYPE_BF16 && q_dtype != XT_DTYPE_F16) return fail(XT_EUNSUPPORTED, "%s: queries must be BF16 or FP16", what);
  if (score_dtype < 0 || score_dtype > 2) return fail(XT_EINVAL, "%s: score dtype %d (0 FP32, 1 BF16, 2 FP16)", what,
                                                      score_dtype);
  // powers of two only, as the reference's tl.arange(0, block_size) requires: the prefill stages 128 keys at a time
  // and masks keys by causality and length, not by the block's end
  if (a.block_size != 32 && a.block_size != 64 && a.block_size != 128 && a.block_size != 256)
    return fail(XT_EUNSUPPORTED, "%s: block size %d (32, 64, 128 or 256)", what, a.block_size);
  if (a.max_slots < kPoolRows || a.max_slots % kPoolRows)
    return fail(XT_EINVAL, "%s: the index pool holds %lld slots (whole pages of 128)", what, (long long)a.max_slots);
  if (!aligned(pay, 16) || pay_ps % 16 || pay_rs % 16 || pay_rs < dim / 2 || !aligned(sc, 8) || sc_rs < dim / 16 ||
      sc_rs % (dim / 32) || sc_ps % (dim / 32) || !aligned(q, 16))
    return fail(XT_EINVAL, "%s: index pool rows must be 16-byte (payload) and %d-byte (scales) aligned", what, dim / 32);
  a.q = static_cast<const uint16_t*>(q);
  a.pay = static_cast<const uint8_t*>(pay);
  a.pay_ps = pay_ps;
  a.pay_rs = pay_rs;
  a.sc = static_cast<const uint8_t*>(sc);
  a.sc_ps = sc_ps;
  a.sc_rs = sc_rs;
  a.r2t = r2t;
  a.score = scores;
  a.out_dtype = score_dtype;
  return XT_OK;
}

template <int NK, bool BF>
int decode_dispatch(int T, const ScoreArgs& a, dim3 grid, hipStream_t st) {
  switch (T) {
    case 1: hipLaunchKernelGGL((decode_scores_kernel<NK, 1, BF>), grid, dim3(64 * kScoreWaves), 0, st, a); break;
    case 2: hipLaunchKernelGGL((decode_scores_kernel<NK, 2, BF>), grid, dim3(64 * kScoreWaves), 0, st, a); break;
    case 4: hipLaunchKernelGGL((decode_scores_kernel<NK, 4, BF>), grid, dim3(64 * kScoreWaves), 0, st, a); break;
    case 8: hipLaunchKernelGGL((decode_scores_kernel<NK, 8, BF>), grid, dim3(64 * kScoreWaves), 0, st, a); break;
    default: return XT_EUNSUPPORTED;
  }
  return XT_OK;
}

template <int NK, bool BF>
void prefill_dispatch(int hpw, const ScoreArgs& a, dim3 grid, hipStream_t st) {
  if (hpw == 1)
    hipLaunchKernelGGL((prefill_scores_kernel<NK, 1, BF>), grid, dim3(64 * kScoreWaves), 0, st, a);
  else if (hpw == 2)
    hipLaunchKernelGGL((prefill_scores_kernel<NK, 2, BF>), grid, dim3(64 * kScoreWaves), 0, st, a);
  else
    hipLaunchKernelGGL((prefill_scores_kernel<NK, 4, BF>), grid, dim3(64 * kScoreWaves), 0, st, a);
}

}  // namespace

extern "C" int xt_minimax_decode_scores(const void* q, int64_t q_batch_stride, int64_t q_head_stride, int batch,
                                        int heads, int dim, int q_dtype, const void* index_payload,
                                        int64_t pay_page_stride, int64_t pay_slot_stride, const void* index_scales,
                                        int64_t sc_page_stride, int64_t sc_slot_stride, int64_t max_slots,
                                        const void* req_to_token, int64_t r2t_stride, const void* seq_lens,
                                        const void* slot_ids, int index_int64, int block_size, float score_factor,
                                        int init_blocks, int local_blocks, int skip_topk, int lse, void* scores,
                                        int score_dtype, int64_t s_head_stride, int64_t s_batch_stride,
                                        int64_t s_block_stride, int max_blocks_hint, xt_stream_t stream) {
  const char* what = "xt_minimax_decode_scores";
  if (batch < 0 || heads < 0) return fail(XT_EINVAL, "%s: negative size", what);
  if (batch == 0 || heads == 0) return ok();
  ScoreArgs a = {};
  a.seq_lens = seq_lens;
  a.slot_ids = slot_ids;
  a.block_size = block_size;
  a.max_slots = max_slots;
  int rc = score_common(what, a, dim, q_dtype, q, index_payload, index_scales, req_to_token, pay_page_stride,
                        pay_slot_stride, sc_page_stride, sc_slot_stride, scores, score_dtype);
  if (rc != XT_OK) return rc;
  a.q_ns = q_batch_stride;
  a.q_hs = q_head_stride;
  a.r2t_stride = r2t_stride;
  a.wide = index_int64;
  a.s_hs = s_head_stride;
  a.s_ns = s_batch_stride;
  a.s_ks = s_block_stride;
  a.batch = batch;
  a.heads = heads;
  a.c = score_factor;
  a.init_blocks = init_blocks;
  a.local_blocks = local_blocks;
  a.skip_topk = skip_topk;
  a.lse = lse;
  // workgroups per request: enough to cover max_blocks_hint blocks with one per wavefront, at most what fills the
  // device about four times over; the kernel strides over any blocks beyond
  const int cus = device_cus();
  int per_req = (max(1, max_blocks_hint) + kScoreWaves - 1) / kScoreWaves;
  per_req = min(per_req, max(1, 4 * cus / batch));
  const dim3 grid((unsigned)per_req, (unsigned)batch, (unsigned)((heads + 31) / 32));
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int T = block_size / 32;
  const bool bf = q_dtype == XT_DTYPE_BF16;
  switch (dim) {
    case 64: rc = bf ? decode_dispatch<4, true>(T, a, grid, st) : decode_dispatch<4, false>(T, a, grid, st); break;
    case 128: rc = bf ? decode_dispatch<8, true>(T, a, grid, st) : decode_dispatch<8, false>(T, a, grid, st); break;
    default: rc = bf ? decode_dispatch<16, true>(T, a, grid, st) : decode_dispatch<16, false>(T, a, grid, st); break;
  }
  if (rc != XT_OK) return fail(rc, "%s: block size %d (32, 64, 128 or 256)", what, block_size);
  return check_launch(what);
}

extern "C" int xt_minimax_prefill_scores(const void* q, int64_t q_token_stride, int64_t q_head_stride, int batch,
                                         int heads, int dim, int q_dtype, int max_q_len, const void* index_payload,
                                         int64_t pay_page_stride, int64_t pay_slot_stride, const void* index_scales,
                                         int64_t sc_page_stride, int64_t sc_slot_stride, int64_t max_slots,
                                         const void* req_to_token, int64_t r2t_stride, const void* cu_seqlens,
                                         const void* seq_lens, const void* prefix_lens, const void* slot_ids,
                                         int index_int64, int block_size, float score_factor, void* scores,
                                         int score_dtype, int64_t s_head_stride, int64_t s_token_stride,
                                         int64_t s_block_stride, xt_stream_t stream) {
  const char* what = "xt_minimax_prefill_scores";
  if (batch < 0 || heads < 0 || max_q_len < 0) return fail(XT_EINVAL, "%s: negative size", what);
  if (batch == 0 || heads == 0 || max_q_len == 0) return ok();
  if (!cu_seqlens || !prefix_lens) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  ScoreArgs a = {};
  a.seq_lens = seq_lens;
  a.slot_ids = slot_ids;
  a.block_size = block_size;
  a.max_slots = max_slots;
  int rc = score_common(what, a, dim, q_dtype, q, index_payload, index_scales, req_to_token, pay_page_stride,
                        pay_slot_stride, sc_page_stride, sc_slot_stride, scores, score_dtype);
  if (rc != XT_OK) return rc;
  a.q_ns = q_token_stride;
  a.q_hs = q_head_stride;
  a.r2t_stride = r2t_stride;
  a.prefix_lens = prefix_lens;
  a.cu_seqlens = cu_seqlens;
  a.wide = index_int64;
  a.s_hs = s_head_stride;
  a.s_ns = s_token_stride;
  a.s_ks = s_block_stride;
  a.batch = batch;
  a.heads = heads;
  a.c = score_factor;
  const int hpw = heads >= 4 ? 4 : heads >= 2 ? 2 : 1;   // heads per workgroup: 256 / hpw rows each
  const int rows = 256 / hpw;
  // block ranges: the request's blocks are at most ceil(r2t_stride / block_size) (its positions index a row of
  // req_to_token); ranges of at least 8 blocks, at most 64 ranges
  const int64_t max_blocks = (r2t_stride + block_size - 1) / block_size;
  const int64_t want_chunks = (max_blocks + 7) / 8;
  a.chunks = want_chunks < 1 ? 1 : want_chunks > 64 ? 64 : (int)want_chunks;
  a.chunk_blocks = max_blocks > 0 ? (int)((max_blocks + a.chunks - 1) / a.chunks) : 0x7FFFFFFF;
  const int64_t tiles = (max_q_len + rows - 1) / rows;
  if (tiles * a.chunks > 0x7FFFFFFF) return fail(XT_EUNSUPPORTED, "%s: %lld query tiles", what, (long long)tiles);
  const dim3 grid((unsigned)(tiles * a.chunks), (unsigned)batch, (unsigned)((heads + hpw - 1) / hpw));
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool bf = q_dtype == XT_DTYPE_BF16;
  switch (dim) {
    case 64: bf ? prefill_dispatch<4, true>(hpw, a, grid, st) : prefill_dispatch<4, false>(hpw, a, grid, st); break;
    case 128: bf ? prefill_dispatch<8, true>(hpw, a, grid, st) : prefill_dispatch<8, false>(hpw, a, grid, st); break;
    default: bf ? prefill_dispatch<16, true>(hpw, a, grid, st) : prefill_dispatch<16, false>(hpw, a, grid, st); break;
  }
  return check_launch(what);
}
