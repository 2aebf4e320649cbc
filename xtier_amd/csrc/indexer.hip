// The step before the sparse attention: the indexer logits that score every key for each query, and the top-k
// selection that turns them into the int32 [rows, topk] position lists the attention kernels read.
//
//   QSA indexer logits (BF16 / FP16 q and k): logits[r, n] = sum_h ReLU(q[r, h] . k[n]) / score_scale, -inf outside
//     the row's [start, end). v_mfma_f32_32x32x16_{bf16,f16}: A = 32 keys x 16 dims, B = 16 dims x (32 / H rows x H
//     heads); ReLU and the head sum on the accumulators (H lanes apart within a row of 16 lanes); the division as a
//     multiplication by 1 / score_scale.
//   DSA logits (FP8 E4M3 q and k, an FP32 scale per key, FP32 head weights): logits[q, n] = sum_h w[q, h] ReLU(q_h .
//     k_n) * k_scale[n], outside [ks, ke) 0 or -inf. v_mfma_f32_32x32x16_f16 on the E4M3 values converted exactly to
//     FP16, with the heads as rows (A = 32 heads x 16 dims of one query, B = 16 dims x 32 keys): a lane then holds 16
//     heads of one key, so the weighted head sum is 16 FMAs in the lane and one exchange with the lane 32 apart. (The
//     FP8 MFMA rounds inside its 16-product sum, to about 2^-16 of the sum of magnitudes; the FP16 one sums the exact
//     products to FP32 accuracy.) Keys come from a flat array or, for decode, from
//     the paged cache (page = block x D E4M3 values, then block FP32 scales) through the block table.
//   Top-k rows: per row the positions of the topk largest finite values, ascending (ties toward the lower position),
//     -1 padded. One workgroup per row: a three-pass radix select over an order-preserving key finds the topk-th
//     largest key T and how many keys equal to T are taken. Rows up to 98304 columns live in registers: the first
//     pass (13 bits) leaves a small candidate bucket whose keys go to LDS for the other two passes, and bitmaps of the
//     taken columns are turned into positions with one block scan. Longer rows are streamed three times (11, 11, 10
//     bits), and one pass in position order writes the positions, each 1024-position chunk placed by a block-wide
//     prefix count.
#include "xt_common.h"
#include "xt_host.h"

#include <algorithm>
#include <atomic>

namespace xt {
namespace {

typedef float float16_t __attribute__((ext_vector_type(16)));
typedef short short8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------------------------------------------
// Block-wide prefix counts (1024 threads = 16 wavefronts).

__device__ inline uint32_t wave_exclusive_count(bool flag, uint32_t& wave_total) {
  const uint64_t bits = __builtin_amdgcn_ballot_w64(flag);
  wave_total = (uint32_t)__builtin_popcountll(bits);
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(bits >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bits, 0u));
}

// Exclusive prefix of `flag` over the workgroup in thread order, and the total; `scratch` holds 16 words. Two barriers.
__device__ inline uint32_t block_exclusive_count(bool flag, uint32_t* scratch, uint32_t& total) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint32_t wt;
  const uint32_t in_wave = wave_exclusive_count(flag, wt);
  if (lane == 0) scratch[wave] = wt;
  __syncthreads();
  uint32_t before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    const uint32_t c = scratch[w];
    before += w < wave ? c : 0u;
    sum += c;
  }
  __syncthreads();   // scratch is reused by the next call
  total = sum;
  return before + in_wave;
}

// ---------------------------------------------------------------------------------------------------------------
// Top-k rows

__device__ inline bool finite_f32(float f) { return (__float_as_uint(f) & 0x7F800000u) != 0x7F800000u; }
// Order-preserving key: a larger float has a larger key, and -0 has the key of +0 (they compare equal, so they tie).
__device__ inline uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return u == 0x80000000u ? 0x80000000u : (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kTopkThreads = 1024;

__global__ __launch_bounds__(kTopkThreads) void topk_rows_kernel(const float* x, int64_t ld, int cols, int topk,
                                                                   int32_t* out, int64_t out_ld) {
  __shared__ uint32_t hist[2048];
  __shared__ uint32_t scratch[16];
  __shared__ uint32_t sel[2];   // the chosen digit's bucket, the rank left inside it
  const int tid = threadIdx.x;
  const float* xr = x + (int64_t)blockIdx.x * ld;
  int32_t* o = out + (int64_t)blockIdx.x * out_ld;

  uint32_t prefix = 0, pmask = 0, remaining = 0, k = 0;
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : pass == 1 ? 10 : 0;
    const uint32_t dmask = pass == 2 ? 0x3FFu : 0x7FFu;
    for (int i = tid; i < 2048; i += kTopkThreads) hist[i] = 0;
    __syncthreads();
    for (int c = tid; c < cols; c += kTopkThreads) {
      const float f = xr[c];
      const uint32_t key = order_key(f);
      if (finite_f32(f) && (key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & dmask], 1u);
    }
    __syncthreads();
    // thread t owns buckets 2047 - 2t and 2046 - 2t (from the top); the exclusive prefix of their counts in thread
    // order is the number of keys in higher buckets
    const uint32_t hi = 2047 - 2 * tid, lo = hi - 1;
    const uint32_t chi = hist[hi], clo = hist[lo];
    // a block prefix sum of the pair counts (counts up to 2^31: the same wave / block structure with sums)
    const int wave = tid >> 6, lane = tid & 63;
    uint32_t v = chi + clo, incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t y = (uint32_t)__shfl_up((int)incl, d);
      if (lane >= d) incl += y;
    }
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    uint32_t above = incl - v, all = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const uint32_t c = scratch[w];
      above += w < wave ? c : 0u;
      all += c;
    }
    if (pass == 0) {
      k = min((uint32_t)topk, all);   // the finite keys bound how many can be taken
      remaining = k;
    }
    if (k != 0) {
      if (above < remaining && remaining <= above + chi) {
        sel[0] = hi;
        sel[1] = remaining - above;
      } else if (above + chi < remaining && remaining <= above + chi + clo) {
        sel[0] = lo;
        sel[1] = remaining - above - chi;
      }
    }
    __syncthreads();
    if (k == 0) break;
    prefix |= sel[0] << shift;
    pmask |= dmask << shift;
    remaining = sel[1];
    __syncthreads();   // sel and scratch are rewritten by the next pass
  }
  // positions in order: keys above T, then the first `remaining` keys equal to T
  uint32_t placed = 0, eq_seen = 0;
  for (int base = 0; k != 0 && base < cols && placed < k; base += kTopkThreads) {
    const int c = base + tid;
    const float f = c < cols ? xr[c] : -__builtin_inff();
    const bool fin = finite_f32(f);
    const uint32_t key = order_key(f);
    const bool eq = fin && key == prefix;
    uint32_t n_eq, n_take;
    const uint32_t eq_before = eq_seen + block_exclusive_count(eq, scratch, n_eq);
    const bool take = fin && (key > prefix || (eq && eq_before < remaining));
    const uint32_t at = placed + block_exclusive_count(take, scratch, n_take);
    if (take) o[at] = c;
    placed += n_take;
    eq_seen += n_eq;
  }
  for (int i = (int)k + tid; i < topk; i += kTopkThreads) o[i] = -1;
}

// Rows of at most kTopkRegCols columns (16-byte aligned rows): the row is read once into registers as order keys (a
// non-finite value as key 0, which no finite value has; the smallest finite key is 0x00800000). Chunk i of thread t
// holds columns 4 (kTopkRegThreads i + t) .. + 3.
//   1. A histogram of the top 13 bits finds the bucket b0 that holds the topk-th largest key (counted as the row
//      arrives when the loads need no branches).
//   2. One pass over the registers classifies every key: a bucket above b0 is taken (bit e of byte
//      kTopkRegThreads i + t of the taken map, so byte j covers columns 4 j .. 4 j + 3), a key in b0 is a candidate,
//      appended with its column to its wavefront's list in LDS.
//   3. Two histograms over the candidates (bits 18..9, then 8..0, both over 1024 buckets) find the topk-th largest
//      key T and how many keys equal to T are taken; the candidates above T join the taken map, those equal to T go
//      to the tie map. When a wavefront's list overflows, the two histograms run over the registers instead and the
//      maps are rewritten against T.
//   4. Thread t turns bytes 24 t .. 24 t + 23 of both maps (columns 96 t .. 96 t + 95) into positions in column
//      order: one block scan places them, and a key equal to T is written only while fewer than `remaining` of them
//      come before it.
// 1024 threads (four wavefronts per SIMD, 96 keys and 128 registers each) measured 67.5 us against 70.7 us for 512
// threads of 192 keys on 352 rows x 95088 columns: the extra wavefronts hide more of the LDS-atomic and branch latency
constexpr int kTopkRegThreads = 1024;
constexpr int kTopkChunks = 24;
constexpr int kTopkRegCols = 4 * kTopkRegThreads * kTopkChunks;   // 98304
// one list of keys and one of columns per wavefront fill the 32 KB histogram
constexpr int kTopkCandPerWave = 8192 / 2 / (kTopkRegThreads / 64);

template <int NW>
__device__ inline uint32_t block_exclusive_sum(uint32_t v, uint32_t* scratch, uint32_t& total) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint32_t incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = (uint32_t)__shfl_up((int)incl, d);
    if (lane >= d) incl += y;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  uint32_t before = incl - v, sum = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const uint32_t c = scratch[w];
    before += w < wave ? c : 0u;
    sum += c;
  }
  __syncthreads();   // scratch is reused by the next call
  total = sum;
  return before;
}

// The bucket of histogram h (NBK buckets) that holds the remaining-th largest key, and how many keys of that bucket
// are then taken. Thread t owns buckets NBK - 1 - NB t down to NBK - NB (t + 1); the exclusive prefix of their counts
// in thread order is the number of keys in higher buckets. With first_topk >= 0, remaining starts as min(first_topk,
// keys counted), returned in k. remaining is 0 afterwards when there is nothing to take (the bucket is then
// meaningless).
template <int NBK>
__device__ inline uint32_t pick_bucket(const uint32_t* h, uint32_t& remaining, uint32_t* scratch, uint32_t* sel,
                                       int first_topk = -1, uint32_t* k = nullptr) {
  constexpr int NB = NBK / kTopkRegThreads, NW = kTopkRegThreads / 64;
  const int top = NBK - 1 - NB * (int)threadIdx.x;
  uint32_t cnt[NB], sum = 0;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    cnt[b] = h[top - b];
    sum += cnt[b];
  }
  uint32_t all;
  uint32_t above = block_exclusive_sum<NW>(sum, scratch, all);
  if (first_topk >= 0) {
    remaining = min((uint32_t)first_topk, all);
    *k = remaining;
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (above < remaining && remaining <= above + cnt[b]) {
      sel[0] = top - b;
      sel[1] = remaining - above;
    }
    above += cnt[b];
  }
  __syncthreads();
  const uint32_t bucket = sel[0];
  remaining = remaining == 0 ? 0u : sel[1];
  __syncthreads();   // sel is rewritten by the next call
  return bucket;
}

// Sets the bit of column `col` in a byte map (byte col / 4, bit col % 4) with a word-wide LDS atomic.
__device__ inline void map_set(uint32_t* map, uint32_t col) {
  const uint32_t byte = col >> 2;
  atomicOr(&map[byte >> 2], 1u << (8u * (byte & 3u) + (col & 3u)));
}

// ALIGNED4: cols % 4 == 0, so every chunk row loads as float4 from an address clamped into the row (columns past the
// end are masked when converted) and the loads have no branches, which lets the histogram of the first chunk rows run
// while the later ones are still in flight. Otherwise the last chunk rows load per element behind uniform branches,
// and the histogram starts after the whole row has arrived.
template <bool ALIGNED4>
__global__ __launch_bounds__(kTopkRegThreads) void topk_rows_reg_kernel(const float* x, int64_t ld, int cols,
                                                                          int topk, int32_t* out, int64_t out_ld) {
  constexpr int NW = kTopkRegThreads / 64;
  constexpr int MAPW = kTopkRegCols / 16;   // words per map
  __shared__ __align__(16) uint32_t hist[8192];   // the 13-bit histogram, then the candidate lists
  __shared__ uint32_t hist2[1024];
  __shared__ __align__(16) uint32_t gtmap[MAPW], eqmap[MAPW];
  __shared__ uint32_t scratch[NW], sel[2], wcount[NW];
  const int tid = threadIdx.x, wave = tid >> 6;
  const float* xr = x + (int64_t)blockIdx.x * ld;
  int32_t* o = out + (int64_t)blockIdx.x * out_ld;
  // 1. the top 13 bits, counted as the row arrives: each chunk row's atomics run while the later chunk rows' loads
  // are still in flight, so the histogram's LDS time hides under the HBM stream
#pragma unroll
  for (int j = 0; j < 2048 / kTopkRegThreads; ++j)
    reinterpret_cast<uint4*>(hist)[tid + kTopkRegThreads * j] = uint4{0, 0, 0, 0};
  __syncthreads();
  // chunk row i is loaded in step i and converted and counted in step i + kTopkAhead, so kTopkAhead chunk rows of
  // loads stay in flight while the histogram's atomics run
  constexpr int kTopkAhead = 2;
  uint32_t key[kTopkChunks][4];
#pragma unroll
  for (int step = 0; step < kTopkChunks + kTopkAhead; ++step) {
    if (step < kTopkChunks) {
      const int i = step, c = 4 * (kTopkRegThreads * i + tid);
      if (ALIGNED4) {
        const float4_t v = *reinterpret_cast<const float4_t*>(xr + min(c, cols - 4));
        key[i][0] = __float_as_uint(v[0]); key[i][1] = __float_as_uint(v[1]);
        key[i][2] = __float_as_uint(v[2]); key[i][3] = __float_as_uint(v[3]);
      } else if (4 * kTopkRegThreads * (i + 1) <= cols) {   // uniform: the whole chunk row is inside the row
        const float4_t v = *reinterpret_cast<const float4_t*>(xr + c);
        key[i][0] = __float_as_uint(v[0]); key[i][1] = __float_as_uint(v[1]);
        key[i][2] = __float_as_uint(v[2]); key[i][3] = __float_as_uint(v[3]);
      } else {   // an address inside the row; columns past the end are masked when converted
#pragma unroll
        for (int e = 0; e < 4; ++e) key[i][e] = __float_as_uint(xr[min(c + e, cols - 1)]);
      }
    }
    if (step >= kTopkAhead) {
      const int i = step - kTopkAhead;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float f = __uint_as_float(key[i][e]);
        key[i][e] = finite_f32(f) && 4 * (kTopkRegThreads * i + tid) + e < cols ? order_key(f) : 0u;
        if (key[i][e] != 0u) atomicAdd(&hist[key[i][e] >> 19], 1u);
      }
    }
  }
  __syncthreads();
  uint32_t remaining = 0, k = 0;
  const uint32_t b0 = pick_bucket<8192>(hist, remaining, scratch, sel, topk, &k);
  if (k == 0) {   // uniform: no finite value
    for (int i = tid; i < topk; i += kTopkRegThreads) o[i] = -1;
    return;
  }

  // 2. classify: buckets above b0 taken, b0 appended to the wavefront's candidate list (the count stays uniform)
  uint32_t* cand_key = hist + wave * kTopkCandPerWave;
  uint32_t* cand_col = hist + (NW + wave) * kTopkCandPerWave;
  uint8_t* gtb = reinterpret_cast<uint8_t*>(gtmap);
  uint32_t wc = 0;
#pragma unroll
  for (int i = 0; i < kTopkChunks; ++i) {
    uint32_t nib = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t d = key[i][e] >> 19;
      nib |= d > b0 ? 1u << e : 0u;
      const bool c = d == b0;
      const uint64_t m = __builtin_amdgcn_ballot_w64(c);
      if (m != 0) {
        const uint32_t pos =
            wc + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (c && pos < (uint32_t)kTopkCandPerWave) {
          cand_key[pos] = key[i][e];
          cand_col[pos] = (uint32_t)(4 * (kTopkRegThreads * i + tid) + e);
        }
        wc += (uint32_t)__builtin_popcountll(m);
      }
    }
    gtb[kTopkRegThreads * i + tid] = (uint8_t)nib;
  }
  for (int j = tid; j < MAPW; j += kTopkRegThreads) eqmap[j] = 0;
  if ((tid & 63) == 0) wcount[wave] = wc;
  __syncthreads();
  bool fits = true;
#pragma unroll
  for (int w = 0; w < NW; ++w) fits = fits && wcount[w] <= (uint32_t)kTopkCandPerWave;

  // 3. bits 18..9 and 8..0 of the keys in b0
  uint32_t t_key;
  if (fits) {   // uniform
    const int n = (int)wc;
    for (int j = tid; j < 1024; j += kTopkRegThreads) hist2[j] = 0;
    __syncthreads();
    for (int j = tid & 63; j < n; j += 64) atomicAdd(&hist2[(cand_key[j] >> 9) & 1023u], 1u);
    __syncthreads();
    const uint32_t b1 = pick_bucket<1024>(hist2, remaining, scratch, sel);
    for (int j = tid; j < 1024; j += kTopkRegThreads) hist2[j] = 0;
    __syncthreads();
    const uint32_t hi1 = (b0 << 10) | b1;
    for (int j = tid & 63; j < n; j += 64)
      if ((cand_key[j] >> 9) == hi1) atomicAdd(&hist2[cand_key[j] & 511u], 1u);
    __syncthreads();
    const uint32_t b2 = pick_bucket<1024>(hist2, remaining, scratch, sel);
    t_key = (hi1 << 9) | b2;
    for (int j = tid & 63; j < n; j += 64) {
      const uint32_t c = cand_key[j];
      if (c > t_key) map_set(gtmap, cand_col[j]);
      else if (c == t_key) map_set(eqmap, cand_col[j]);
    }
  } else {
    for (int j = tid; j < 1024; j += kTopkRegThreads) hist2[j] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kTopkChunks; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((key[i][e] >> 19) == b0) atomicAdd(&hist2[(key[i][e] >> 9) & 1023u], 1u);
    __syncthreads();
    const uint32_t b1 = pick_bucket<1024>(hist2, remaining, scratch, sel);
    for (int j = tid; j < 1024; j += kTopkRegThreads) hist2[j] = 0;
    __syncthreads();
    const uint32_t hi1 = (b0 << 10) | b1;
#pragma unroll
    for (int i = 0; i < kTopkChunks; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((key[i][e] >> 9) == hi1) atomicAdd(&hist2[key[i][e] & 511u], 1u);
    __syncthreads();
    const uint32_t b2 = pick_bucket<1024>(hist2, remaining, scratch, sel);
    t_key = (hi1 << 9) | b2;
    uint8_t* eqb = reinterpret_cast<uint8_t*>(eqmap);
#pragma unroll
    for (int i = 0; i < kTopkChunks; ++i) {
      uint32_t gn = 0, en = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gn |= key[i][e] > t_key ? 1u << e : 0u;
        en |= key[i][e] == t_key ? 1u << e : 0u;
      }
      gtb[kTopkRegThreads * i + tid] = (uint8_t)gn;
      eqb[kTopkRegThreads * i + tid] = (uint8_t)en;
    }
  }
  __syncthreads();

  // 4. positions in column order
  constexpr int TW = MAPW / kTopkRegThreads;   // 6 words of each map per thread
  uint32_t gw[TW], ew[TW], ng = 0, ne = 0;
#pragma unroll
  for (int j = 0; j < TW / 2; ++j) {
    const uint2 g = reinterpret_cast<const uint2*>(gtmap)[TW / 2 * tid + j];
    const uint2 q = reinterpret_cast<const uint2*>(eqmap)[TW / 2 * tid + j];
    gw[2 * j] = g.x; gw[2 * j + 1] = g.y;
    ew[2 * j] = q.x; ew[2 * j + 1] = q.y;
  }
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    ng += (uint32_t)__builtin_popcount(gw[j]);
    ne += (uint32_t)__builtin_popcount(ew[j]);
  }
  uint32_t tot;
  uint32_t gt_b = block_exclusive_sum<NW>(ng, scratch, tot);
  uint32_t eq_b = block_exclusive_sum<NW>(ne, scratch, tot);
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    uint32_t m = gw[j] | ew[j];
    while (m != 0u) {
      const uint32_t b = (uint32_t)__builtin_ctz(m);
      m &= m - 1u;
      const int col = 4 * (4 * (TW * tid + j) + (int)(b >> 3)) + (int)(b & 7u);
      if ((gw[j] >> b) & 1u) {
        o[gt_b + min(eq_b, remaining)] = col;
        ++gt_b;
      } else {
        if (eq_b < remaining) o[gt_b + eq_b] = col;
        ++eq_b;
      }
    }
  }
  for (int i = (int)k + tid; i < topk; i += kTopkRegThreads) o[i] = -1;
}

// ---------------------------------------------------------------------------------------------------------------
// QSA indexer logits

template <bool BF>
__device__ inline float16_t mfma_qk(short8_t a, short8_t b, float16_t c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                  0, 0, 0);
}

struct QsaArgs {
  const uint16_t* q;
  int64_t q_rs, q_hs;
  const uint16_t* k;
  int64_t k_rs;
  const int32_t* starts;
  const int32_t* ends;
  float score_scale;
  float* logits;
  int64_t ld;
  int rows, keys;
  int keys_per_wg;
  int vec_store;             // logits rows are 16-byte aligned: stores of 4 floats
};

constexpr int kQsaWaves = 4;

// Workgroup = (4 wavefronts x 2 column groups of 32 / H rows, keys_per_wg keys): every wavefront sweeps the whole key
// range for its own 2 x 32 / H rows, so the four wavefronts read the same K blocks (from L1 after the first) and each
// K block leaves L2 once per 8 x 32 / H rows. Lane layouts (32x32x16): A = keys, lane (key l % 32, dims
// 16kk + 8 (l / 32) .. +7) read straight from k; B = queries, lane (column j = l % 32: row j / H, head j % H; same
// dims) kept in registers, one set per column group; C = S^T, lane (column j, keys 8 (r / 4) + 4 (l / 32) + r % 4).
constexpr int kQsaGroups = 2;   // column groups per wavefront

template <int H, int NK, bool BF>
__global__ __launch_bounds__(64 * kQsaWaves) void qsa_logits_kernel(const QsaArgs a) {
  constexpr int kRowsG = 32 / H, kRowsW = kQsaGroups * kRowsG;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  const int rw = (blockIdx.x * kQsaWaves + wave) * kRowsW;   // this wavefront's first row
  const int head = j % H;
  int my_row[kQsaGroups], start[kQsaGroups], end[kQsaGroups];
  bool row_ok[kQsaGroups];
  short8_t qb[kQsaGroups][NK];
#pragma unroll
  for (int g = 0; g < kQsaGroups; ++g) {
    my_row[g] = rw + g * kRowsG + j / H;
    row_ok[g] = my_row[g] < a.rows;
    start[g] = row_ok[g] ? a.starts[my_row[g]] : 0;
    end[g] = row_ok[g] ? a.ends[my_row[g]] : 0;
    const uint16_t* qp = a.q + (int64_t)(row_ok[g] ? my_row[g] : 0) * a.q_rs + (int64_t)head * a.q_hs + 8 * h;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const uint4 w = row_ok[g] ? *reinterpret_cast<const uint4*>(qp + 16 * kk) : uint4{0u, 0u, 0u, 0u};
      qb[g][kk] = __builtin_bit_cast(short8_t, w);
    }
  }
  // the wavefront's key range: a 32-key block outside every one of its rows' [start, end) is written as -inf
  // without the product
  int lo = 0x7FFFFFFF, hi = 0;
  for (int r = 0; r < kRowsW; ++r) {
    if (rw + r < a.rows) {
      lo = min(lo, max(0, a.starts[rw + r]));
      hi = max(hi, min(a.keys, a.ends[rw + r]));
    }
  }
  // x / score_scale as x * (1 / score_scale): one more rounding, at most 2^-24 relative
  const float inv = 1.0f / a.score_scale;
  const int k_begin = blockIdx.y * a.keys_per_wg, k_end = min(a.keys, k_begin + a.keys_per_wg);
  if constexpr (H <= 4) {
    // Queries as rows: S = Q . K^T with A = the query columns above, B = K; C lane (key kb + j, column-group rows
    // i = 8 (r / 4) + 4 h + r % 4: row i / H, head i % H). A row's H heads are H consecutive r of one lane, so the
    // head sum stays in the lane, and lane j writes key kb + j of 16 / H rows (each row: 32 consecutive keys across
    // the lanes).
    constexpr int kOut = 16 / H;
    int orow[kQsaGroups][kOut], ost[kQsaGroups][kOut], oen[kQsaGroups][kOut];
    int max_start = 0, min_end = 0x7FFFFFFF;
#pragma unroll
    for (int g = 0; g < kQsaGroups; ++g)
#pragma unroll
      for (int o = 0; o < kOut; ++o) {
        const int r = o * H;
        orow[g][o] = rw + g * kRowsG + (8 * (r >> 2) + 4 * h + (r & 3)) / H;
        const bool ok = orow[g][o] < a.rows;
        ost[g][o] = ok ? a.starts[orow[g][o]] : 0;
        oen[g][o] = ok ? a.ends[orow[g][o]] : 0;
        if (ok) {
          max_start = max(max_start, ost[g][o]);
          min_end = min(min_end, oen[g][o]);
        }
      }
    // over the wavefront: a block inside every row's range needs no per-key test
    for (int d = 1; d < 64; d <<= 1) {
      max_start = max(max_start, __shfl_xor(max_start, d));
      min_end = min(min_end, __shfl_xor(min_end, d));
    }
    for (int kb = k_begin; kb < k_end; kb += 32) {
      const int key = kb + j;
      if (kb + 32 <= lo || kb >= hi) {   // uniform over the wavefront
#pragma unroll
        for (int g = 0; g < kQsaGroups; ++g)
#pragma unroll
          for (int o = 0; o < kOut; ++o)
            if (orow[g][o] < a.rows && key < a.keys) a.logits[(int64_t)orow[g][o] * a.ld + key] = -__builtin_inff();
        continue;
      }
      const bool inside = kb >= max_start && kb + 32 <= min_end;
      const uint16_t* kp = a.k + (int64_t)min(key, a.keys - 1) * a.k_rs + 8 * h;
      short8_t kf[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) kf[kk] = __builtin_bit_cast(short8_t, *reinterpret_cast<const uint4*>(kp + 16 * kk));
#pragma unroll
      for (int g = 0; g < kQsaGroups; ++g) {
        float16_t sc = {};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) sc = mfma_qk<BF>(qb[g][kk], kf[kk], sc);
#pragma unroll
        for (int o = 0; o < kOut; ++o) {
          float x = fmaxf(sc[o * H], 0.0f);
#pragma unroll
          for (int e = 1; e < H; ++e) x += fmaxf(sc[o * H + e], 0.0f);
          const bool in_range = inside || (key >= ost[g][o] && key < oen[g][o]);
          if (orow[g][o] < a.rows && key < a.keys)
            a.logits[(int64_t)orow[g][o] * a.ld + key] = in_range ? x * inv : -__builtin_inff();
        }
      }
    }
    return;
  }
  for (int kb = k_begin; kb < k_end; kb += 32) {
    float v[kQsaGroups][16];
    if (kb + 32 <= lo || kb >= hi) {   // uniform over the wavefront
#pragma unroll
      for (int g = 0; g < kQsaGroups; ++g)
#pragma unroll
        for (int r = 0; r < 16; ++r) v[g][r] = -__builtin_inff();
    } else {
      const int key = min(kb + j, a.keys - 1);
      const uint16_t* kp = a.k + (int64_t)key * a.k_rs + 8 * h;
      short8_t kf[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) kf[kk] = __builtin_bit_cast(short8_t, *reinterpret_cast<const uint4*>(kp + 16 * kk));
#pragma unroll
      for (int g = 0; g < kQsaGroups; ++g) {
        float16_t s = {};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) s = mfma_qk<BF>(kf[kk], qb[g][kk], s);
        // ReLU, then the sum over the H heads of a row (H consecutive lanes), in the order lane ^ 1, ^ 2, ...
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = fmaxf(s[r], 0.0f);
          if constexpr (H >= 2) x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
          if constexpr (H >= 4) x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
          if constexpr (H >= 8) x += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), (4 << 10) | 0x1F));
          if constexpr (H >= 16) x += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), (8 << 10) | 0x1F));
          if constexpr (H >= 32) x += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), (16 << 10) | 0x1F));
          const int kr = kb + 8 * (r >> 2) + 4 * h + (r & 3);
          v[g][r] = (kr >= start[g] && kr < end[g]) ? x * inv : -__builtin_inff();
        }
      }
    }
    // the lane of head 0 of each row writes its 16 keys: 4 runs of 4 consecutive keys
#pragma unroll
    for (int g = 0; g < kQsaGroups; ++g) {
      if (row_ok[g] && head == 0) {
        float* op = a.logits + (int64_t)my_row[g] * a.ld;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int key = kb + 8 * q4 + 4 * h;
          if (key + 4 <= a.keys && a.vec_store) {
            *reinterpret_cast<float4_t*>(op + key) =
                float4_t{v[g][4 * q4], v[g][4 * q4 + 1], v[g][4 * q4 + 2], v[g][4 * q4 + 3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (key + e < a.keys) op[key + e] = v[g][4 * q4 + e];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// DSA logits (FP8)

struct DsaArgs {
  const uint8_t* q;          // [num_q, heads, D] E4M3
  int64_t q_rs, q_hs;
  const uint8_t* k;          // flat: [num_kv, D] E4M3 with k_rs bytes per key; paged: the page buffer
  int64_t k_rs;
  const float* k_scale;      // flat: [num_kv]
  int64_t page_bytes;        // paged: bytes from one page to the next (block x (D + 4))
  int64_t num_pages;         // paged: pages in the cache (table entries past it read as no key)
  int block;                 // paged: keys per page (0: flat keys)
  const int32_t* block_table;
  int64_t bt_stride;
  int bt_width;
  const float* w;            // [num_q, heads]
  int64_t w_rs;
  const int32_t* ks;         // flat: [num_q] (inclusive) start, or NULL
  const int32_t* ke;         // flat: end (exclusive); paged: context length per row
  int clean;
  float* logits;
  int64_t ld;
  int num_q, num_kv, heads;
  int keys_per_wg;
  int out_cols;              // columns written per row (paged: max_seq_len)
};

constexpr int kDsaWaves = 4;

// Workgroup = (4 query rows, one per wavefront, keys_per_wg keys); the wavefronts walk the same 32-key blocks, so a
// block's key bytes are fetched once for the four rows. Per block and 32-head group, S = Q . K^T on 32x32x16 FP16
// MFMAs of the converted E4M3 values (A = Q: lane (head l % 32, dims 16kk + 8 (l / 32) .. +7); B = K^T: lane (key
// l % 32, same dims); C: lane (key column l % 32, heads 8 (r / 4) + 4 (l / 32) + r % 4)).
template <int NK>
__global__ __launch_bounds__(64 * kDsaWaves) void dsa_logits_kernel(const DsaArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  const int qrow = blockIdx.x * kDsaWaves + wave;
  if (qrow >= a.num_q) return;   // no barrier below
  const int groups = a.heads / 32;
  const int k_begin = blockIdx.y * a.keys_per_wg, k_end = min(a.out_cols, k_begin + a.keys_per_wg);
  const bool paged = a.block > 0;
  const int lim_lo = (!paged && a.ks) ? a.ks[qrow] : 0;
  const int lim_hi = paged ? a.ke[qrow] : (a.ke ? a.ke[qrow] : a.num_kv);
  const float fill = a.clean ? -__builtin_inff() : 0.0f;
  for (int kb = k_begin; kb < k_end; kb += 32) {
    const int key = kb + j;
    bool live = key >= lim_lo && key < lim_hi && key < (paged ? a.bt_width * a.block : a.num_kv);
    int32_t page = 0;
    if (paged) {
      // a negative entry reads page 0, as the reference's clamp does (indexer_torch.py:61); an entry past the cache
      // reads as no key
      page = live ? max(a.block_table[(int64_t)qrow * a.bt_stride + key / a.block], 0) : 0;
      live = live && page < a.num_pages;
      page = live ? page : 0;
    }
    float total = 0.0f;
    if (__builtin_amdgcn_ballot_w64(live)) {
      // this lane's key row and scale
      const uint8_t* kp;
      float ksc;
      if (paged) {
        const int kk = live ? key : 0;
        const uint8_t* pg = a.k + (int64_t)page * a.page_bytes;
        kp = pg + (int64_t)(kk % a.block) * (16 * NK);
        ksc = *reinterpret_cast<const float*>(pg + (int64_t)a.block * (16 * NK) + 4 * (kk % a.block));
      } else {
        const int kk = live ? key : 0;
        kp = a.k + (int64_t)kk * a.k_rs;
        ksc = a.k_scale[kk];
      }
      uint64_t kf[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) kf[kk] = *reinterpret_cast<const uint64_t*>(kp + 16 * kk + 8 * h);
      float acc = 0.0f;
      for (int g = 0; g < groups; ++g) {
        const uint8_t* qp = a.q + (int64_t)qrow * a.q_rs + (int64_t)(32 * g + j) * a.q_hs + 8 * h;
        float16_t s = {};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
          s = __builtin_amdgcn_mfma_f32_32x32x16_f16(fp8x8_to_f16(*reinterpret_cast<const uint64_t*>(qp + 16 * kk)),
                                                     fp8x8_to_f16(kf[kk]), s, 0, 0, 0);
        const float* wp = a.w + (int64_t)qrow * a.w_rs + 32 * g + 4 * h;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc += fmaxf(s[r], 0.0f) * wp[8 * (r >> 2) + (r & 3)];
      }
      // the other 16 heads of each group are in the lane 32 apart
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
      total = (__uint_as_float(sw[0]) + __uint_as_float(sw[1])) * ksc;
    }
    if (h == 0 && key < k_end) a.logits[(int64_t)qrow * a.ld + key] = live ? total : fill;
  }
}

// Flat keys, heads x dim within registers (G head groups of 32, G * NK <= 16): the four rows of a workgroup read the
// same keys, so the workgroup stages them once per 128 keys in LDS (E4M3 bytes, double-buffered, one barrier per
// stage), each wavefront keeps its row's query (as FP16) and head weights in registers for the whole key range, and
// converts each 32-key block's K once for all its head groups.
constexpr int kDsaStageKeys = 128;

template <int NK, int G>
__global__ __launch_bounds__(64 * kDsaWaves) void dsa_flat_kernel(const DsaArgs a) {
  // LDS bytes per key: D + 8, so the 32 keys a half-wavefront reads sit on 32 distinct bank pairs ((D + 8) / 4 is
  // twice an odd number)
  constexpr int D = 16 * NK, ROW = D + 8;
  constexpr int PIECES = kDsaStageKeys * D / 16;           // 16-byte pieces per stage
  constexpr int PER_THREAD = PIECES / (64 * kDsaWaves);
  __shared__ __align__(16) uint8_t kt[2][kDsaStageKeys * ROW];   // ROW * 128 is a multiple of 16
  __shared__ float kst[2][kDsaStageKeys];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5, tid = threadIdx.x;
  const int qrow = blockIdx.x * kDsaWaves + wave;
  const bool row_ok = qrow < a.num_q;   // every thread takes every barrier below
  const int k_begin = blockIdx.y * a.keys_per_wg, k_end = min(a.num_kv, k_begin + a.keys_per_wg);
  const int lim_lo = (row_ok && a.ks) ? a.ks[qrow] : 0;
  const int lim_hi = row_ok ? (a.ke ? a.ke[qrow] : a.num_kv) : 0;
  const float fill = a.clean ? -__builtin_inff() : 0.0f;
  // this row's query (A operand: head 32 g + j, dims 16 kk + 8 h .. + 7) and weights (C rows of lane half h)
  half8_t qf[G][NK];
  float wv[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint8_t* qp = a.q + (int64_t)(row_ok ? qrow : 0) * a.q_rs + (int64_t)(32 * g + j) * a.q_hs + 8 * h;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      qf[g][kk] = fp8x8_to_f16(row_ok ? *reinterpret_cast<const uint64_t*>(qp + 16 * kk) : 0ull);
    const float* wp = a.w + (int64_t)(row_ok ? qrow : 0) * a.w_rs + 32 * g + 4 * h;
#pragma unroll
    for (int r = 0; r < 16; ++r) wv[g][r] = row_ok ? wp[8 * (r >> 2) + (r & 3)] : 0.0f;
  }
  uint4 reg[PER_THREAD];
  float sreg = 0.0f;
  auto load_stage = [&](int k0) {   // keys past the end read the last key (never written out)
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int c = tid + 64 * kDsaWaves * i, key = min(k0 + c / (D / 16), a.num_kv - 1);
      reg[i] = *reinterpret_cast<const uint4*>(a.k + (int64_t)key * a.k_rs + 16 * (c % (D / 16)));
    }
    if (tid < kDsaStageKeys) sreg = a.k_scale[min(k0 + tid, a.num_kv - 1)];
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int c = tid + 64 * kDsaWaves * i;
      uint2* dst = reinterpret_cast<uint2*>(&kt[buf][(c / (D / 16)) * ROW + 16 * (c % (D / 16))]);
      dst[0] = uint2{reg[i].x, reg[i].y};   // 8-byte aligned rows: two 8-byte stores
      dst[1] = uint2{reg[i].z, reg[i].w};
    }
    if (tid < kDsaStageKeys) kst[buf][tid] = sreg;
  };
  const int stages = k_end > k_begin ? (k_end - k_begin + kDsaStageKeys - 1) / kDsaStageKeys : 0;
  if (stages > 0) {
    load_stage(k_begin);
    store_stage(0);
  }
  __syncthreads();
  for (int st = 0; st < stages; ++st) {
    const int k0 = k_begin + st * kDsaStageKeys, buf = st & 1;
    if (st + 1 < stages) load_stage(k0 + kDsaStageKeys);   // in flight during this stage's MFMAs
#pragma unroll 1
    for (int t = 0; t < kDsaStageKeys / 32; ++t) {
      const uint8_t* kr = &kt[buf][(32 * t + j) * ROW + 8 * h];
      half8_t kv[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) kv[kk] = fp8x8_to_f16(*reinterpret_cast<const uint64_t*>(kr + 16 * kk));
      float acc = 0.0f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float16_t sc = {};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qf[g][kk], kv[kk], sc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc += fmaxf(sc[r], 0.0f) * wv[g][r];
      }
      // the other 16 heads of each group are in the lane 32 apart
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
      const float total = (__uint_as_float(sw[0]) + __uint_as_float(sw[1])) * kst[buf][32 * t + j];
      const int key = k0 + 32 * t + j;
      const bool live = key >= lim_lo && key < lim_hi;
      if (row_ok && h == 0 && key < k_end) a.logits[(int64_t)qrow * a.ld + key] = live ? total : fill;
    }
    if (st + 1 < stages) store_stage(buf ^ 1);   // its readers finished the stage before the last barrier
    __syncthreads();
  }
}

}  // namespace
}  // namespace xt

using namespace xt;

extern "C" int xt_topk_rows(const float* x, int64_t ld, int rows, int cols, int topk, int32_t* out, int64_t out_ld,
                            xt_stream_t stream) {
  const char* what = "xt_topk_rows";
  if (rows < 0 || cols < 0 || topk < 0) return fail(XT_EINVAL, "%s: negative size", what);
  if (rows == 0 || topk == 0) return ok();
  if (!out || (!x && cols > 0)) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (ld < cols || out_ld < topk) return fail(XT_EINVAL, "%s: row strides shorter than the rows", what);
  // the register-resident rows read at column 0 (and at cols - 4 when cols % 4 == 0); empty rows stream, reading
  // nothing, and come out all -1
  const bool in_registers = cols > 0 && cols <= 4 * kTopkRegThreads * kTopkChunks && ld % 4 == 0 && aligned(x, 16);
  if (in_registers && cols % 4 == 0)
    hipLaunchKernelGGL(topk_rows_reg_kernel<true>, dim3((unsigned)rows), dim3(kTopkRegThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), x, ld, cols, topk, out, out_ld);
  else if (in_registers)
    hipLaunchKernelGGL(topk_rows_reg_kernel<false>, dim3((unsigned)rows), dim3(kTopkRegThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), x, ld, cols, topk, out, out_ld);
  else
    hipLaunchKernelGGL(topk_rows_kernel, dim3((unsigned)rows), dim3(kTopkThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), x, ld, cols, topk, out, out_ld);
  return check_launch(what);
}

// Workgroups of one instantiation that fit a CU at once (its register use sets it), read once per process.
template <int H, int NK, bool BF>
static int qsa_per_cu() {
  static std::atomic<int> cached{0};
  int n = cached.load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, qsa_logits_kernel<H, NK, BF>, 64 * kQsaWaves, 0) !=
            hipSuccess || n <= 0)
      n = 1;
    cached.store(n, std::memory_order_relaxed);
  }
  return n;
}

// The grid: row tiles x key chunks, the chunks sized so that the workgroups fit one round on the CUs (a second round
// of a few workgroups would take as long as the first: 558 workgroups at 512 per round measured 116 us).
template <int H, int NK, bool BF>
static void qsa_go(QsaArgs a, int row_tiles, hipStream_t st) {
  const int64_t slots = (int64_t)device_cus() * qsa_per_cu<H, NK, BF>();
  const int64_t chunks = std::max<int64_t>(1, slots / row_tiles);
  a.keys_per_wg = (int)std::max<int64_t>(32, ((a.keys + chunks - 1) / chunks + 31) / 32 * 32);
  const dim3 grid((unsigned)row_tiles, (unsigned)((a.keys + a.keys_per_wg - 1) / a.keys_per_wg));
  hipLaunchKernelGGL((qsa_logits_kernel<H, NK, BF>), grid, dim3(64 * kQsaWaves), 0, st, a);
}

template <int H>
static int qsa_launch(int nk, bool bf, const QsaArgs& a, int row_tiles, hipStream_t st) {
#define XT_QSA(NK)                                                                                                    \
  if (nk == NK) {                                                                                                    \
    if (bf)                                                                                                          \
      qsa_go<H, NK, true>(a, row_tiles, st);                                                                         \
    else                                                                                                             \
      qsa_go<H, NK, false>(a, row_tiles, st);                                                                        \
    return XT_OK;                                                                                                    \
  }
  XT_QSA(4)
  XT_QSA(8)
  XT_QSA(16)
#undef XT_QSA
  return XT_EUNSUPPORTED;
}

extern "C" int xt_qsa_indexer_logits(const void* q, int64_t q_row_stride, int64_t q_head_stride, int rows, int heads,
                                     int dim, const void* k, int64_t k_row_stride, int keys, const int32_t* starts,
                                     const int32_t* ends, float score_scale, int dtype, float* logits, int64_t ld,
                                     xt_stream_t stream) {
  const char* what = "xt_qsa_indexer_logits";
  if (rows < 0 || keys < 0) return fail(XT_EINVAL, "%s: negative size", what);
  if (rows == 0 || keys == 0) return ok();
  if (!q || !k || !starts || !ends || !logits) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (heads != 1 && heads != 2 && heads != 4 && heads != 8 && heads != 16 && heads != 32)
    return fail(XT_EUNSUPPORTED, "%s: %d heads (supported: powers of 2 up to 32)", what, heads);
  if (dim != 64 && dim != 128 && dim != 256) return fail(XT_EUNSUPPORTED, "%s: head size %d (64, 128, 256)", what, dim);
  if (dtype != XT_DTYPE_BF16 && dtype != XT_DTYPE_F16) return fail(XT_EINVAL, "%s: q / k must be BF16 or FP16", what);
  if (!aligned(q, 16) || !aligned(k, 16) || q_row_stride % 8 || q_head_stride % 8 || k_row_stride % 8 ||
      ld < keys || !(score_scale > 0.0f))
    return fail(XT_EINVAL, "%s: rows must be 16-byte aligned, ld >= keys, score_scale > 0", what);
  QsaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_rs = q_row_stride;
  a.q_hs = q_head_stride;
  a.k = static_cast<const uint16_t*>(k);
  a.k_rs = k_row_stride;
  a.starts = starts;
  a.ends = ends;
  a.score_scale = score_scale;
  a.logits = logits;
  a.ld = ld;
  a.rows = rows;
  a.keys = keys;
  a.keys_per_wg = 1024;   // set with the grid in qsa_go
  a.vec_store = (ld % 4 == 0) && aligned(logits, 16);
  const int rows_per_wg = kQsaWaves * kQsaGroups * (32 / heads);
  const int row_tiles = (rows + rows_per_wg - 1) / rows_per_wg;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool bf = dtype == XT_DTYPE_BF16;
  const int nk = dim / 16;
  int e = XT_EUNSUPPORTED;
  switch (heads) {
    case 1: e = qsa_launch<1>(nk, bf, a, row_tiles, st); break;
    case 2: e = qsa_launch<2>(nk, bf, a, row_tiles, st); break;
    case 4: e = qsa_launch<4>(nk, bf, a, row_tiles, st); break;
    case 8: e = qsa_launch<8>(nk, bf, a, row_tiles, st); break;
    case 16: e = qsa_launch<16>(nk, bf, a, row_tiles, st); break;
    case 32: e = qsa_launch<32>(nk, bf, a, row_tiles, st); break;
  }
  if (e != XT_OK) return fail(e, "%s: no kernel for %d heads x %d", what, heads, dim);
  return check_launch(what);
}

static int dsa_common(const char* what, DsaArgs& a, int dim, xt_stream_t stream) {
  if (a.heads % 32 || a.heads <= 0 || a.heads > 128)
    return fail(XT_EUNSUPPORTED, "%s: %d heads (supported: 32, 64, 96, 128)", what, a.heads);
  if (dim != 64 && dim != 128 && dim != 256) return fail(XT_EUNSUPPORTED, "%s: head size %d (64, 128, 256)", what, dim);
  if (!aligned(a.q, 8) || a.q_rs % 8 || a.q_hs % 8 || !aligned(a.w, 4) || a.ld < a.out_cols)
    return fail(XT_EINVAL, "%s: q rows must be 8-byte aligned and ld >= the columns written", what);
  a.keys_per_wg = 4096;
  const dim3 grid((unsigned)((a.num_q + kDsaWaves - 1) / kDsaWaves), (unsigned)((a.out_cols + 4095) / 4096));
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int nk = dim / 16, groups = a.heads / 32;
  if (a.block == 0 && groups * nk <= 16 && aligned(a.k, 16) && a.k_rs % 16 == 0) {
#define XT_DSA_FLAT(NK, G)                                                                                           \
  if (nk == NK && groups == G) {                                                                                     \
    hipLaunchKernelGGL((dsa_flat_kernel<NK, G>), grid, dim3(64 * kDsaWaves), 0, st, a);                             \
    return check_launch(what);                                                                                       \
  }
    XT_DSA_FLAT(4, 1) XT_DSA_FLAT(4, 2) XT_DSA_FLAT(4, 3) XT_DSA_FLAT(4, 4) XT_DSA_FLAT(8, 1) XT_DSA_FLAT(8, 2)
    XT_DSA_FLAT(16, 1)
#undef XT_DSA_FLAT
  }
  switch (dim / 16) {
    case 4: hipLaunchKernelGGL(dsa_logits_kernel<4>, grid, dim3(64 * kDsaWaves), 0, st, a); break;
    case 8: hipLaunchKernelGGL(dsa_logits_kernel<8>, grid, dim3(64 * kDsaWaves), 0, st, a); break;
    default: hipLaunchKernelGGL(dsa_logits_kernel<16>, grid, dim3(64 * kDsaWaves), 0, st, a); break;
  }
  return check_launch(what);
}

extern "C" int xt_dsa_mqa_logits(const void* q, int64_t q_row_stride, int64_t q_head_stride, int num_q, int heads,
                                 int dim, const void* k, int64_t k_row_stride, const float* k_scale, int num_kv,
                                 const float* weights, int64_t w_row_stride, const int32_t* ks, const int32_t* ke,
                                 int clean_logits, float* logits, int64_t ld, xt_stream_t stream) {
  const char* what = "xt_dsa_mqa_logits";
  if (num_q < 0 || num_kv < 0) return fail(XT_EINVAL, "%s: negative size", what);
  if (num_q == 0 || num_kv == 0) return ok();
  if (!q || !k || !k_scale || !weights || !logits) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (!aligned(k, 8) || k_row_stride % 8 || k_row_stride < dim)
    return fail(XT_EINVAL, "%s: key rows must be 8-byte aligned", what);
  DsaArgs a = {};
  a.q = static_cast<const uint8_t*>(q);
  a.q_rs = q_row_stride;
  a.q_hs = q_head_stride;
  a.k = static_cast<const uint8_t*>(k);
  a.k_rs = k_row_stride;
  a.k_scale = k_scale;
  a.block = 0;
  a.w = weights;
  a.w_rs = w_row_stride;
  a.ks = ks;
  a.ke = ke;
  a.clean = clean_logits;
  a.logits = logits;
  a.ld = ld;
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.heads = heads;
  a.out_cols = num_kv;
  return dsa_common(what, a, dim, stream);
}

extern "C" int xt_dsa_paged_mqa_logits(const void* q, int64_t q_row_stride, int64_t q_head_stride, int batch,
                                       int heads, int dim, const void* kvcache, int64_t num_pages, int64_t page_bytes,
                                       int block,
                                       const int32_t* block_table, int64_t bt_stride, int bt_width,
                                       const int32_t* context_lens, const float* weights, int64_t w_row_stride,
                                       int max_seq_len, int clean_logits, float* logits, int64_t ld,
                                       xt_stream_t stream) {
  const char* what = "xt_dsa_paged_mqa_logits";
  if (batch < 0 || max_seq_len < 0) return fail(XT_EINVAL, "%s: negative size", what);
  if (batch == 0 || max_seq_len == 0) return ok();
  if (!q || !kvcache || !block_table || !context_lens || !weights || !logits)
    return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (block <= 0 || num_pages <= 0 || page_bytes < (int64_t)block * (dim + 4) || page_bytes % 8 ||
      !aligned(kvcache, 8) || bt_width <= 0 || bt_stride < bt_width)
    return fail(XT_EINVAL, "%s: pages of %d keys need %d bytes each (8-byte aligned)", what, block, block * (dim + 4));
  DsaArgs a = {};
  a.q = static_cast<const uint8_t*>(q);
  a.q_rs = q_row_stride;
  a.q_hs = q_head_stride;
  a.k = static_cast<const uint8_t*>(kvcache);
  a.page_bytes = page_bytes;
  a.num_pages = num_pages;
  a.block = block;
  a.block_table = block_table;
  a.bt_stride = bt_stride;
  a.bt_width = bt_width;
  a.w = weights;
  a.w_rs = w_row_stride;
  a.ks = nullptr;
  a.ke = context_lens;
  a.clean = clean_logits;
  a.logits = logits;
  a.ld = ld;
  a.num_q = batch;
  a.num_kv = bt_width * block;
  a.heads = heads;
  a.out_cols = max_seq_len;
  return dsa_common(what, a, dim, stream);
}
