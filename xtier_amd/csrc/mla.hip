// Sparse MLA: 128 query heads share one key per token. Two cache formats:
//   NVFP4 latent (kNvfp4): key = [latent (512, NVFP4 with E4M3 block scales and a global scale) | rope (64, BF16)],
//     576 wide, value = the latent; operands FP16 for the latent (the query as q * 2^-e per head, the key tile as
//     e2m1 * e4m3, both exact) and BF16 for the rope (the cache's values and q * 2^-e, exact), the global scale
//     applied to the FP32 latent scores and to the values on the normalized output (with two caches, P carries each
//     key's g relative to the larger of the two);
//   DeepSeek V4 FP8 pages (kFp8V4, sparse_mla.py:38-59): key = [448 E4M3 values x UE8M0 scale per 64 | 64 BF16 rope],
//     512 wide, value = the key; operands BF16 as in the reference, the scale applied to the FP32 scores.
// q.k and p.v on MFMA (v_mfma_f32_16x16x32_f16 / _bf16), online softmax in the exp2 domain, an optional per-head sink
// in the denominator. With key splits, each (row, split) writes its output normalized by its own sum (FP16 for the
// NVFP4 latent, before the global scale: a convex combination of e2m1 * e4m3 values, at most 2688 in magnitude; FP32
// for V4) with its max and sum, and a second, wide launch merges the splits and applies the global scale:
// one merging workgroup per row would read a row's partials at one CU's bandwidth.
//
// Work decomposition: a workgroup = 8 wavefronts x 16 heads = 128 heads of one (query row, key split), so every key is
// read and dequantized once for all heads. Per step of 32 keys the workgroup
//   1. turns the raw key records (loaded one step ahead into registers) into two LDS tiles: K [32 keys][Dk] and
//      V^T [512][32 keys] (16-bit values);
//   2. each wave computes S^T [32 keys x 16 heads] = K . Q^T (Dk/32 MFMAs per 16-key tile, Q^T mostly resident in
//      registers), the softmax, and O^T [512 x 16 heads] += V^T . P^T (32 MFMAs), P^T taken straight from the score
//      registers (the key order T(j) below matches the V^T operand).
//
// Lane layouts (16x16x32 MFMA, hl = lane % 16, j = lane / 16):
//   QK: A = K tile, lane (key hl, dims 32kk + 8j .. +7); B = Q^T, lane (head hl, same dims); C = S^T, lane (head hl,
//       keys 4j .. 4j+3 of the 16-key tile).
//   PV: A = V^T, lane (dim hl of a 16-dim tile, keys T(j) = {4j..4j+3, 16+4j..16+4j+3}); B = P^T, lane (head hl, keys
//       T(j)); C = O^T, lane (head hl, dims 4j .. 4j+3 of the tile).
//
// Numerics: NVFP4: e2m1 * e4m3 is exact in FP16 (at most 6 significant bits), and so is the query scaled by a power of
// two; the rope chunks multiply BF16 values (the cache's rope and q * 2^-e) exactly in the BF16 MFMA; the latent and
// rope parts of a score accumulate apart, and score = (latent . q * g + rope . q) * scale *
// log2(e) * 2^e in FP32 (g of the key's cache); P is FP16 of p (of p * g / max(g0, g1) with two caches), the sum takes
// p, and the normalization multiplies by g (by max(g0, g1)). V4: e4m3 * 2^(e - 127) is exact in BF16 (4 significant
// bits) for scales from 2^-126; a zero scale byte (2^-127) reads as 0; P is BF16. The running maximum is raised lazily
// (P <= 256); sums are FP32.
#include "xt_common.h"
#include "xt_host.h"

#include <algorithm>
#include <atomic>

namespace xt {
namespace {

enum { kNvfp4 = 0, kFp8V4 = 1 };
constexpr int kDl = 512;                 // value width; NVFP4 latent: 256 payload bytes, 32 scale bytes per token
constexpr int kDr = 64;                  // rope width (BF16): 128 bytes per token
constexpr int kV4Nope = 448;             // V4: E4M3 values per token, one UE8M0 scale per 64
constexpr int kV4Row = 576;              // V4: bytes of a token's data row (448 + 128)
template <int F>
constexpr int kDk = F == kNvfp4 ? kDl + kDr : kDl;   // key width
constexpr int kMSteps = 32;              // keys per step
constexpr int kMWaves = 8;
constexpr int kMHeads = 16 * kMWaves;    // heads per workgroup
// Row pitches of the LDS tiles, measured with SQ_LDS_BANK_CONFLICT (gfx950 LDS: 64 banks; b128 reads served 16 lanes
// per cycle, b64 32): a K pitch of 32 mod 64 bytes (1184 / 1056) makes both the QK reads (16 key rows x 4 column
// quarters, b128) and the transposing value reads (16 key rows x 4 dim groups, b64) conflict-free, as a query pitch
// of 96 bytes does for the LDS query reads.
template <int F>
constexpr int kKRow = kDk<F> + 16;       // 16-bit values per K tile row
template <int F>
constexpr int kKTile = kMSteps * kKRow<F> * 2;
template <int F>
constexpr int kQChunks = kDk<F> / 32;    // 32-dim chunks of a query row
template <int F>
constexpr int kQReg = F == kNvfp4 ? 9 : 7;     // chunks kept in registers; the others live in LDS
template <int F>
constexpr int kLatChunks = F == kNvfp4 ? kDl / 32 : kQChunks<F>;   // NVFP4: chunks of the latent (FP16 MFMA); the
                                                                   // rope chunks after them run BF16
constexpr int kQRow = 32;                // 16-bit values per (chunk, head) row of the LDS query block; the four 16-byte
                                         // pieces of row r sit at piece ^ ((r >> 1) & 3), which measures free of bank
                                         // conflicts for the b128 reads of 16 rows x 4 pieces
constexpr int kQAhead = 2;               // chunks of K fragments read ahead of their QK MFMAs
constexpr int kSlotIters = 11;           // slot list entries per thread: (max keys per split + 32) / 512, rounded up
template <int F>
constexpr int kQTile = (kQChunks<F> - kQReg<F>) * kMHeads * kQRow * 2;
constexpr int kRescaleM = 8;
// The phases of the per-wave timeline (xt_mla_timeline), in stamp order.
enum { kMsEntry, kMsSlots, kMsQuery, kMsTile0, kMsLoop, kMsOut, kMsStaged, kMlaStamps = 8 };

struct CacheDev {
  const uint8_t* pay;                // NVFP4: latent payload; V4: the page buffer
  const uint8_t* sf;
  const uint16_t* rope;
  const float* g;
  int64_t slots;
  uint32_t pay_stride, sf_stride, rope_stride;   // NVFP4: bytes from one slot to the next
  uint32_t page_shift;               // V4: log2(tokens per page)
  uint64_t page_bytes;               // V4: bytes from one page to the next (data rows, then 8-byte scale rows)
};

struct MlaArgs {
  const uint16_t* q;
  int64_t q_rs, q_hs;
  CacheDev c[2];
  const int32_t* idx[2];
  int64_t idx_stride[2];
  int topk[2];
  const int32_t* len[2];
  const float* sink;
  float qscale;                      // softmax scale * log2(e)
  uint16_t* out;
  int64_t o_rs, o_hs;
  int out_dtype;
  float* lse;
  int heads, splits, keys_per_split, steps;
  void* part;                        // [rows, splits, heads, 512] FP16 (NVFP4) / FP32 (V4): the split's output
                                     // normalized by its own sum
  float* ml;                         // [rows, splits, heads, 2]: the split's running max (log2 domain) and sum
  uint32_t xcd_units, xcd_extra;
  uint64_t* stamps;                  // per-wave timeline (xt_mla_timeline), NULL: off
  uint32_t stamp_blocks;             // workgroups whose stamps fit the buffer
  int o32;                           // NVFP4: every cache has fewer than 2^24 slots and all its rows within 2^32
                                     // bytes, so record offsets are one 24-bit multiply-add (else 64-bit arithmetic)
};

typedef short short8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// 16x16x32 MFMA on 16-bit operands of the format: FP16 (NVFP4 latent) or BF16 (V4)
template <int F>
__device__ inline float4_t mfma16(short8_t a, short8_t b, float4_t c) {
  if constexpr (F == kNvfp4)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// Slot list entries: >= 0 a slot of cache 0, <= -2 slot (-e - 2) of cache 1, -1 no key.
__device__ inline bool entry_valid(int32_t e) { return e != -1; }

// Dequant mapping: thread t handles keys 4kq .. 4kq+3 (kq = t / 64, the wave) and latent dims 8c .. 8c+7 (c = t % 64),
// so a wave reads one key's record as one contiguous run and writes one 1 KiB K tile row per store (no LDS bank
// conflicts); rope: key t / 8, part t % 8. V4 (same mapping, all 512 dims): dims 8c .. 8c+7 are E4M3 bytes (c < 56)
// or BF16 rope values (c >= 56).
template <int F>
struct Raw;
template <>
struct Raw<kNvfp4> {
  uint32_t pay[4];   // payload bytes 4c .. 4c+3 of keys 4kq + i
  uint32_t sc[4];    // scale byte c / 2 of those keys
  uint4 rope;        // rope values 8p .. 8p+7 of key t / 8 (threads 0-255)
};
template <>
struct Raw<kFp8V4> {
  uint4 d[4];        // keys 4kq + i: E4M3 bytes 8c .. 8c+7 in (x, y) (z, w unused), or rope values 8(c - 56) .. +7
  uint32_t sc[4];    // UE8M0 scale byte c / 8 of those keys (c < 56)
};

// The record of slot list entry e: with one key list the entry is the slot (or -1: slot 0, ignored); with two the
// cache is chosen per key.
template <bool TWO>
__device__ inline const CacheDev& cache_of(const MlaArgs& a, int32_t e, uint32_t& s) {
  if (!TWO) {
    s = e < 0 ? 0u : (uint32_t)e;
    return a.c[0];
  }
  s = e >= 0 ? (uint32_t)e : (e <= -2 ? (uint32_t)(-e - 2) : 0u);
  return a.c[e <= -2 ? 1 : 0];
}

// The slot entries of keys 4kq .. 4kq+3 of a step as one 16-byte LDS read, issued before any K tile write (a write
// the compiler cannot tell apart from the slot list would otherwise order each entry's read after the previous write).
__device__ inline void step_entries(const int32_t* slots, int step, int kq, int32_t (&e)[4]) {
  const int4 v = *reinterpret_cast<const int4*>(slots + step * kMSteps + 4 * kq);
  e[0] = v.x;
  e[1] = v.y;
  e[2] = v.z;
  e[3] = v.w;
}

template <int F, bool TWO>
__device__ inline void load_raw(const MlaArgs& a, const int32_t* slots, int step, Raw<F>& r) {
  const int t = threadIdx.x, kq = t >> 6, c = t & 63;
  int32_t ent[4];
  step_entries(slots, step, kq, ent);
  if constexpr (F == kFp8V4) {
    // token s of a cache: page s >> page_shift, row s & (page size - 1); data row at row * 576, scale row after the
    // page's data rows at row * 8. Lanes c < 56 take E4M3 bytes 8c .. 8c+7 and scale byte c / 8, lanes 56-63 rope
    // bytes 448 + 16 (c - 56) .. +15; every lane makes the same two 8-byte loads and one byte load (bytes it does not
    // use stay inside the token's records), so the wave does not branch.
    const bool nope = c < kV4Nope / 8;
    const uint32_t off = nope ? 8u * c : kV4Nope + 16u * (c - kV4Nope / 8);
    const uint32_t sb = nope ? (uint32_t)c >> 3 : 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t s;
      const CacheDev& cd = cache_of<TWO>(a, ent[i], s);
      const uint32_t ps = 1u << cd.page_shift, rw = s & (ps - 1u);
      const uint8_t* page = cd.pay + (uint64_t)(s >> cd.page_shift) * cd.page_bytes;
      const uint8_t* rp = page + (uint64_t)rw * kV4Row + off;
      const uint2 v0 = *reinterpret_cast<const uint2*>(rp), v1 = *reinterpret_cast<const uint2*>(rp + 8);
      r.d[i] = uint4{v0.x, v0.y, v1.x, v1.y};
      r.sc[i] = page[(uint64_t)ps * kV4Row + (uint64_t)rw * 8 + sb];
    }
    return;
  } else {
  if (a.o32) {   // uniform over the launch; unsigned 32-bit offsets (HIP's __umul24 returns a signed int)
    const uint32_t cu = (uint32_t)c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t s;
      const CacheDev& cd = cache_of<TWO>(a, ent[i], s);
      r.pay[i] = *reinterpret_cast<const uint32_t*>(cd.pay + ((uint32_t)__umul24(s, cd.pay_stride) + 4u * cu));
      r.sc[i] = cd.sf[(uint32_t)__umul24(s, cd.sf_stride) + (cu >> 1)];
    }
    if (t < 256) {
      uint32_t s;
      const CacheDev& cd = cache_of<TWO>(a, slots[step * kMSteps + (t >> 3)], s);
      r.rope = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(cd.rope) +
                                               ((uint32_t)__umul24(s, cd.rope_stride) + 16u * ((uint32_t)t & 7u)));
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t s;
    const CacheDev& cd = cache_of<TWO>(a, ent[i], s);
    r.pay[i] = *reinterpret_cast<const uint32_t*>(cd.pay + (uint64_t)s * cd.pay_stride + 4 * c);
    r.sc[i] = cd.sf[(uint64_t)s * cd.sf_stride + (c >> 1)];
  }
  if (t < 256) {
    uint32_t s;
    const CacheDev& cd = cache_of<TWO>(a, slots[step * kMSteps + (t >> 3)], s);
    r.rope = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(cd.rope) + (uint64_t)s * cd.rope_stride +
                                             16 * (t & 7));
  }
  }
}

// Raw records -> the K tile (the value operand is read from it transposed). An invalid key's value becomes 0 (so
// P * V stays finite whatever slot 0 holds); an NVFP4 key's rope is left as read: its score is masked by a select,
// never multiplied.
template <int F, bool TWO>
__device__ inline void dequant(const MlaArgs& a, const int32_t* slots, int step, const Raw<F>& r, uint16_t* kt) {
  const int t = threadIdx.x, kq = t >> 6, c = t & 63;
  int32_t ent[4];
  step_entries(slots, step, kq, ent);
  if constexpr (F == kFp8V4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = entry_valid(ent[i]);
      // e4m3 * 2^(e - 127): the scaled conversion takes the scale's exponent, exact in BF16; e = 0 reads as 0. Rope
      // lanes (c >= 56) keep their raw BF16 values; both forms are computed and one selected, without a branch.
      const float sc = __uint_as_float(r.sc[i] << 23);
      const bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.d[i].x, sc, false);
      const bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.d[i].x, sc, true);
      const bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.d[i].y, sc, false);
      const bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r.d[i].y, sc, true);
      const bool nope = c < kV4Nope / 8;
      const bool live = ok && (!nope || r.sc[i] != 0u);
      const uint4 w = uint4{
          live ? (nope ? __builtin_bit_cast(uint32_t, p0) : r.d[i].x) : 0u,
          live ? (nope ? __builtin_bit_cast(uint32_t, p1) : r.d[i].y) : 0u,
          live ? (nope ? __builtin_bit_cast(uint32_t, p2) : r.d[i].z) : 0u,
          live ? (nope ? __builtin_bit_cast(uint32_t, p3) : r.d[i].w) : 0u};
      *reinterpret_cast<uint4*>(kt + (4 * kq + i) * kKRow<F> + 8 * c) = w;
    }
    return;
  } else {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const _Float16 h = entry_valid(ent[i]) ? fp8x2_to_f16<false>(r.sc[i]).x : (_Float16)0.0f;
    const half2_t s2 = half2_t{h, h};
    const half2_t p0 = fp4x2_to_f16<0>(r.pay[i]) * s2, p1 = fp4x2_to_f16<1>(r.pay[i]) * s2;
    const half2_t p2 = fp4x2_to_f16<2>(r.pay[i]) * s2, p3 = fp4x2_to_f16<3>(r.pay[i]) * s2;
    *reinterpret_cast<half8_t*>(kt + (4 * kq + i) * kKRow<F> + 8 * c) =
        half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
  }
  if (t < 256)   // the rope stays BF16: its chunks run the BF16 MFMA, with no range or precision loss
    *reinterpret_cast<uint4*>(kt + (t >> 3) * kKRow<F> + kDl + 8 * (t & 7)) = r.rope;
  }
}

// A wave's 16 heads x 512 output dims (accumulator acc[dt][r]: head hl, dim 16 dt + 4 j + r), times inv, as head
// rows of 1 KiB in LDS. The 16-byte pieces of row r sit at piece index ^ r: rows are 1 KiB apart, so unswizzled the 16
// heads of a write would all fall on the same banks; swizzled, each half-wave's write covers 64 distinct banks.
template <bool BF>
__device__ inline void stage_rows(uint16_t* stage, const float4_t (&acc)[32], float inv, int hl, int j) {
#pragma unroll
  for (int dt = 0; dt < 32; ++dt)
    *reinterpret_cast<uint2*>(stage + hl * kDl + 8 * ((2 * dt + (j >> 1)) ^ hl) + 4 * (j & 1)) =
        make_uint2(pack2_16<BF>(acc[dt][0] * inv, acc[dt][1] * inv), pack2_16<BF>(acc[dt][2] * inv, acc[dt][3] * inv));
}


// Element index of a split partial in the accumulators' lane order: (row, split, wave of 16 heads, dim-tile pair k,
// lane) holds 8 values, head 16 wave + lane % 16, dims 32k + 4 (lane / 16) .. +3 then 32k + 16 + 4 (lane / 16) .. +3;
// heads are padded to whole waves.
__device__ inline int64_t part_index(const MlaArgs& a, int64_t row, int split, int wave, int k, int lane) {
  const int waves = (a.heads + 15) >> 4;
  return ((((row * a.splits + split) * waves + wave) * 16 + k) * 64 + lane) * 8;
}

// TL: the per-wave timeline build (xt_mla_timeline), launched only while a stamp buffer is set, so the kernel the
// serving path runs carries none of its instructions or registers.
template <int F, bool TWO, bool TL>
__global__ void __launch_bounds__(512) mla_kernel(const MlaArgs a) {
  constexpr int kQC = kQChunks<F>, kQR = kQReg<F>, kLatC = kLatChunks<F>;
  extern __shared__ __align__(16) uint8_t lds[];
  asm volatile("" ::"s"(a.xcd_units), "s"(a.xcd_extra), "s"(a.splits), "s"(a.keys_per_split), "s"(a.topk[0]),
               "s"(a.topk[1]), "s"(a.idx[0]), "s"(a.idx[1]), "s"(a.idx_stride[0]), "s"(a.idx_stride[1]),
               "s"(a.len[0]), "s"(a.len[1]), "s"(a.q), "s"(a.q_rs), "s"(a.q_hs), "s"(a.heads));
  // XCD-aware numbering as in the decode kernel: a row's splits run on one XCD
  const uint32_t gidx = blockIdx.x;
  // per-wave timeline (diagnostics, off unless xt_mla_timeline set a buffer): the first lane of every wave writes the
  // 100 MHz constant clock at each phase (kMlaStamps per wave); a branch uniform over the launch otherwise
  const bool timeline = TL && gidx < a.stamp_blocks;
  const uint64_t t_entry = timeline ? __builtin_amdgcn_s_memrealtime() : 0;
  const uint32_t xcd = gidx & 7u;
  const uint32_t u = xcd * a.xcd_units + min(xcd, a.xcd_extra) + (gidx >> 3);
  const int split = (int)(u % (uint32_t)a.splits);
  const int64_t row = u / (uint32_t)a.splits;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, hl = lane & 15, j = lane >> 4;
  const int head = 16 * wave + hl;
  const bool head_live = head < a.heads;
  // (the wave's stamp address is formed at each stamp from values the loop keeps anyway: kept live across the main
  // loop it would take registers the loop needs)
  auto stamp = [&](int phase) {
    if (timeline) {
      const uint64_t t = __builtin_amdgcn_s_memrealtime();
      if ((hl | j) == 0) a.stamps[((uint64_t)gidx * kMWaves + wave) * kMlaStamps + phase] = t;
    }
  };
  if (timeline && lane == 0) {   // phases a wave does not reach stay 0
    uint64_t* const my_stamps = a.stamps + ((uint64_t)gidx * kMWaves + wave) * kMlaStamps;
    my_stamps[kMsEntry] = t_entry;
#pragma unroll
    for (int i = 1; i < kMlaStamps; ++i) my_stamps[i] = 0;
  }

  // two K tiles: step n computes on tile n % 2 while the next step's keys are dequantized into the other
  uint16_t* ktiles = reinterpret_cast<uint16_t*>(lds);
  uint16_t* qs = reinterpret_cast<uint16_t*>(lds + 2 * kKTile<F>);
  int32_t* slots = reinterpret_cast<int32_t*>(lds + 2 * kKTile<F> + kQTile<F>);

  // 1. the split's key list: columns [t0, t0 + keys_per_split) of list 0 then list 1, as slot entries in LDS. The
  //    list lengths are uniform scalar loads; every thread's index loads (kSlotIters, 512 apart) issue together and
  //    before the query's loads, so that waiting for them does not wait for those.
  const int t0 = split * a.keys_per_split;
  const int total = (a.steps + 1) * kMSteps;   // one padding step of invalid keys
  const int n0 = a.len[0] ? min(a.len[0][row], a.topk[0]) : a.topk[0];
  const int n1 = a.len[1] ? min(a.len[1][row], a.topk[1]) : a.topk[1];
  int32_t sraw[kSlotIters];
#pragma unroll
  for (int u = 0; u < kSlotIters; ++u) {
    const int i = (int)threadIdx.x + 512 * u;
    const int col = t0 + i;
    const int li = col < a.topk[0] ? 0 : 1;
    const int cc = col - (li ? a.topk[0] : 0);
    sraw[u] = (i < a.keys_per_split && cc < (li ? n1 : n0)) ? a.idx[li][row * a.idx_stride[li] + cc] : -1;
  }

  // the query's B operands: dims 32kk + 8j .. +7 of head `head` (a clamped valid head for padding lanes)
  uint4 qraw[kQC];
  {
    const uint16_t* qp = a.q + row * a.q_rs + (int64_t)min(head, a.heads - 1) * a.q_hs;
#pragma unroll
    for (int kk = 0; kk < kQC; ++kk) qraw[kk] = *reinterpret_cast<const uint4*>(qp + 32 * kk + 8 * j);
  }
#pragma unroll
  for (int u = 0; u < kSlotIters; ++u) {
    const int i = (int)threadIdx.x + 512 * u;
    const int li = t0 + i < a.topk[0] ? 0 : 1;
    const int32_t sv = sraw[u];
    const int32_t e = (sv >= 0 && sv < a.c[li].slots) ? (li ? -sv - 2 : sv) : -1;
    if (i < total) slots[i] = e;
  }
  __syncthreads();
  stamp(kMsSlots);

  // B operands of q.k, chunks 0..kQR-1 in registers, the rest in LDS: NVFP4, FP16 of q * 2^-e, exact, with 2^e per
  // head from its largest magnitude (pow2_query_scale), and scale * log2(e) * 2^e applied to the FP32 scores; V4, q
  // as given (BF16), the scale applied to the FP32 scores
  float smul = a.qscale;
  float qdown = 1.0f;
  if constexpr (F == kNvfp4) {
    float qmax = 0.0f;
#pragma unroll
    for (int kk = 0; kk < kQC; ++kk) {
      const uint32_t ws[4] = {qraw[kk].x, qraw[kk].y, qraw[kk].z, qraw[kk].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        qmax = fmaxf(qmax, fmaxf(__builtin_fabsf(bf16_bits_to_f32(ws[e] & 0xFFFFu)),
                                 __builtin_fabsf(bf16_bits_to_f32(ws[e] >> 16))));
    }
    const float2_t p2 = pow2_query_scale(max4_lanes16(qmax));   // the head's maximum over its four lanes
    qdown = p2[0];
    smul = a.qscale * p2[1];
  }
  short8_t qb[kQR];
#pragma unroll
  for (int kk = 0; kk < kQC; ++kk) {
    short8_t h;
    if (F == kNvfp4 && kk >= kLatC) {   // rope chunks: BF16 of q * 2^-e, exact (a power of two), for the BF16 MFMA
      const uint32_t ws[4] = {qraw[kk].x, qraw[kk].y, qraw[kk].z, qraw[kk].w};
      uint32_t b[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        b[e] = head_live ? ((__float_as_uint(bf16_bits_to_f32(ws[e] & 0xFFFFu) * qdown) >> 16) |
                            (__float_as_uint(bf16_bits_to_f32(ws[e] >> 16) * qdown) & 0xFFFF0000u))
                         : 0u;
      h = __builtin_bit_cast(short8_t, uint4{b[0], b[1], b[2], b[3]});
    } else if constexpr (F == kNvfp4) {
      const uint32_t ws[4] = {qraw[kk].x, qraw[kk].y, qraw[kk].z, qraw[kk].w};
      half8_t hh;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hh[2 * e] = head_live ? (_Float16)(bf16_bits_to_f32(ws[e] & 0xFFFFu) * qdown) : (_Float16)0.0f;
        hh[2 * e + 1] = head_live ? (_Float16)(bf16_bits_to_f32(ws[e] >> 16) * qdown) : (_Float16)0.0f;
      }
      h = __builtin_bit_cast(short8_t, hh);
    } else {
      h = __builtin_bit_cast(short8_t, head_live ? qraw[kk] : uint4{0u, 0u, 0u, 0u});
    }
    if (kk < kQR)
      qb[kk < kQR ? kk : 0] = h;
    else
      *reinterpret_cast<short8_t*>(qs + ((kk - kQR) * kMHeads + 16 * wave + hl) * kQRow + 8 * (j ^ ((hl >> 1) & 3))) = h;
  }
  // NVFP4 global scales (V4 has none): g0 / g1 scale the latent scores; with two caches P carries g / max(g0, g1)
  // (at most 1, so P <= 256 stays in FP16's range whatever the scales) and the normalization multiplies by the max.
  // (1 / max is uniform: readfirstlane keeps it in a scalar register, and P's select reuses the scores' g0 / g1).
  float g0 = 1.0f, g1 = 1.0f, ginv = 1.0f;
  if constexpr (F == kNvfp4) {
    g0 = *a.c[0].g;
    g1 = TWO ? *a.c[1].g : g0;
    const float gm = fmaxf(g0, g1);
    if (TWO && gm > 0.0f) ginv = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(1.0f / gm)));
  }

  float m = -__builtin_inff(), l = 0.0f;
  float4_t acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};

  Raw<F> raw;
  stamp(kMsQuery);
  load_raw<F, TWO>(a, slots, 0, raw);
  dequant<F, TWO>(a, slots, 0, raw, ktiles);
  if (a.steps > 1) load_raw<F, TWO>(a, slots, 1, raw);
  __syncthreads();
  stamp(kMsTile0);
  for (int step = 0; step < a.steps; ++step) {
    const uint16_t* kt = ktiles + (step & 1) * (kKTile<F> / 2);
    // the next step's keys into the other tile (its readers finished before the previous barrier; after the last step
    // it is the padding step, all zeros, never read), then the raw records of the step after, if there is one (a
    // branch uniform over the launch: on the last two steps it skips loads whose records were already read, which the
    // epilogue would otherwise wait for before reusing their registers; the padding step's dequant ignores them)
    dequant<F, TWO>(a, slots, step + 1, raw, ktiles + ((step + 1) & 1) * (kKTile<F> / 2));
    if (step + 2 < a.steps) load_raw<F, TWO>(a, slots, step + 2, raw);
    const uint32_t valid = (uint32_t)__builtin_amdgcn_ballot_w64(lane < kMSteps &&
                                                                  entry_valid(slots[step * kMSteps + (lane & 31)]));
    // S^T for the two 16-key tiles, one MFMA chain each. The K fragments (and LDS-resident query chunks) of chunk
    // kk + kQAhead are read while the MFMAs of chunk kk run; scheduling barriers keep that order, so an MFMA does not
    // wait for a read issued just before it.
    // this lane's keys T(j) as bits 0..7: keys 4j .. 4j+3, then 16+4j .. 16+4j+3
    const uint32_t vmask = ((valid >> (4 * j)) & 0xFu) | (((valid >> (16 + 4 * j)) & 0xFu) << 4);
    // NVFP4: the global scale of each of those keys (of its cache; two caches may differ). Chunks below kLatC are the
    // latent's: once they are summed, the accumulators are multiplied by the key's global scale, and the rope chunks
    // (no global scale) add onto them.
    uint32_t l1 = 0u;   // bit e: key e of T(j) is cache 1's
    if constexpr (F == kNvfp4 && TWO) {
      const uint32_t b =
          (uint32_t)__builtin_amdgcn_ballot_w64(lane < kMSteps && slots[step * kMSteps + (lane & 31)] <= -2);
      l1 = ((b >> (4 * j)) & 0xFu) | (((b >> (16 + 4 * j)) & 0xFu) << 4);
    }
    float4_t s[2] = {float4_t{0.f, 0.f, 0.f, 0.f}, float4_t{0.f, 0.f, 0.f, 0.f}};
    short8_t kf[kQC][2], qf[kQC];
    auto read_chunk = [&](int kk) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        kf[kk][tt] = *reinterpret_cast<const short8_t*>(kt + (16 * tt + hl) * kKRow<F> + 8 * j + 32 * kk);
      qf[kk] = kk < kQR ? qb[kk < kQR ? kk : 0]
                        : *reinterpret_cast<const short8_t*>(qs + ((kk - kQR) * kMHeads + 16 * wave + hl) * kQRow +
                                                             8 * (j ^ ((hl >> 1) & 3)));
    };
#pragma unroll
    for (int kk = 0; kk < kQAhead; ++kk) read_chunk(kk);
#pragma unroll
    for (int kk = 0; kk < kQC; ++kk) {
      if (kk + kQAhead < kQC) read_chunk(kk + kQAhead);
      __builtin_amdgcn_sched_barrier(0);
      if (kk == kLatC) {
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e >> 2][e & 3] *= ((l1 >> e) & 1u) ? g1 : g0;
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        s[tt] = kk >= kLatC ? mfma16<kFp8V4>(kf[kk][tt], qf[kk], s[tt]) : mfma16<F>(kf[kk][tt], qf[kk], s[tt]);
      __builtin_amdgcn_sched_barrier(0);
    }
    float sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sv[e] = ((vmask >> e) & 1u) ? s[e >> 2][e & 3] * smul : -__builtin_inff();
    // online softmax of head hl over keys T(j), lazy rescale
    float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
    mt = max4_lanes16(mt);
    if (__builtin_amdgcn_ballot_w64(mt > m + kRescaleM)) {
      const float m_new = (mt > m + kRescaleM) ? mt : m;
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 32; ++i) acc[i] *= alpha;
      m = m_new;
    }
    const float m_use = (m == -__builtin_inff()) ? 0.0f : m;
    short8_t pb;
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = __builtin_amdgcn_exp2f(sv[e] - m_use);
      psum += p;
      if constexpr (F == kNvfp4)
        pb[e] = __builtin_bit_cast(short, (_Float16)(TWO ? p * ginv * (((l1 >> e) & 1u) ? g1 : g0) : p));
      else
        pb[e] = __builtin_bit_cast(short, (__bf16)p);
    }
    l += psum;
    // O^T += V^T . P^T over the 32 dim tiles, V^T read from the K tile with transposing reads: in each 16-lane group
    // lane L addresses key 4j + L/4, dims 16 dt + 4 (L % 4) .. +3, and lane i receives dim 16 dt + i of keys 4j .. 4j+3
    // (then 16 + 4j .. from 16 rows further)
    typedef short short4_t __attribute__((ext_vector_type(4)));
    const uint16_t* vr = kt + (4 * j + (hl >> 2)) * kKRow<F> + 4 * (hl & 3);
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) {
      const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) short4_t*)(vr + 16 * dt));
      const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) short4_t*)(vr + 16 * kKRow<F> + 16 * dt));
      const short8_t av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      acc[dt] = mfma16<F>(av, pb, acc[dt]);
    }
    __syncthreads();
  }
  stamp(kMsLoop);
  // the 4 lanes of a head hold disjoint key subsets of l
  const float l_tot = sum4_lanes16(l);

  if (a.splits == 1) {
    // the wave's 16 heads x 512 dims, normalized, staged in LDS as head rows of 1 KiB (the key and query tiles are
    // free: every wave passed the last step's barrier), then written back a head row per store instruction (64
    // lanes x 16 bytes, the pieces of head row r at piece index ^ r); from the accumulators' lane order each store
    // would scatter 4-byte pieces over 16 rows
    if (16 * wave >= a.heads) return;   // no live head in this wave
    const float m_use = (m == -__builtin_inff()) ? 0.0f : m;
    float total = l_tot;
    if (a.sink) total += __builtin_amdgcn_exp2f(a.sink[min(head, a.heads - 1)] * kLog2e - m_use);
    const float inv = l_tot > 0.0f ? (TWO ? fmaxf(g0, g1) : g0) / total : 0.0f;
    uint16_t* stage = reinterpret_cast<uint16_t*>(lds) + wave * 16 * kDl;
    if (a.out_dtype == XT_DTYPE_BF16)
      stage_rows<true>(stage, acc, inv, hl, j);
    else
      stage_rows<false>(stage, acc, inv, hl, j);
    if (head_live && a.lse && j == 0)
      a.lse[row * a.heads + head] = l_tot > 0.0f ? (m + __builtin_log2f(l_tot)) * kLn2 : -__builtin_inff();
    stamp(kMsStaged);
    // (the stage is this wave's own: its LDS writes complete before its reads, no barrier)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint4 x = *reinterpret_cast<const uint4*>(stage + r * kDl + 8 * lane);
      if (16 * wave + r < a.heads)
        *reinterpret_cast<uint4*>(a.out + row * a.o_rs + (int64_t)(16 * wave + r) * a.o_hs + 8 * (lane ^ r)) = x;
    }
    stamp(kMsOut);
    return;
  }
  // 2. the split's output normalized by its own sum (NVFP4: FP16, a convex combination of e2m1 * e4m3 values, so at
  //    most 2688 in magnitude whatever g; V4: FP32) plus its max and sum; a second launch merges the splits. The partials are stored in the accumulators'
  //    lane order (part_index), so every store of a wave writes one contiguous run.
  if (16 * wave >= a.heads) return;   // a wave without live heads has no partials (heads pad to whole waves only)
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;   // NVFP4: without g (the merge applies it)
  const int64_t pbase = part_index(a, row, split, wave, 0, lane);
  if constexpr (F == kNvfp4) {
    uint16_t* pp = static_cast<uint16_t*>(a.part) + pbase;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float4_t x = acc[2 * k] * inv, y = acc[2 * k + 1] * inv;
      *reinterpret_cast<uint4*>(pp + k * 512) =
          uint4{f32_to_f16_bits(x[0]) | (f32_to_f16_bits(x[1]) << 16), f32_to_f16_bits(x[2]) | (f32_to_f16_bits(x[3]) << 16),
                f32_to_f16_bits(y[0]) | (f32_to_f16_bits(y[1]) << 16), f32_to_f16_bits(y[2]) | (f32_to_f16_bits(y[3]) << 16)};
    }
  } else {
    float* pp = static_cast<float*>(a.part) + pbase;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      reinterpret_cast<float4_t*>(pp + k * 512)[0] = acc[2 * k] * inv;
      reinterpret_cast<float4_t*>(pp + k * 512)[1] = acc[2 * k + 1] * inv;
    }
  }
  if (head_live && j == 0)
    *reinterpret_cast<float2*>(a.ml + (((int64_t)row * a.splits + split) * a.heads + head) * 2) = float2{m, l_tot};
  stamp(kMsOut);
}

// Split merge: thread = (row, wave w, dim-tile pair k, lane) of the partials' lane order: head 16w + lane % 16, dims
// 32k + 4 (lane / 16) .. +3 and 32k + 16 + 4 (lane / 16) .. +3. out = sum_s w_s o_s with w_s = 2^(m_s - max m) l_s /
// (sum_s 2^(m_s - max m) l_s + sink term). The splits are taken four at a time with all their loads issued together and
// a running maximum across groups, so the usual four splits cost one round trip; a wave's loads of one split are one
// contiguous run. A workgroup (256 threads: row, w, four consecutive k) holds 16 heads x 128 dims of output; it
// stages them in LDS and writes each head's 256 bytes as 16 consecutive 16-byte pieces (written straight from the
// lane order, every store instruction would scatter 64 pieces of 4 bytes over 16 head rows). In the stage the pieces
// of head row h sit at piece index ^ h, which spreads the 16 heads of an LDS write over distinct banks.
template <int F>
__global__ void __launch_bounds__(256) mla_merge_kernel(const MlaArgs a, int rows) {
  __shared__ __align__(16) uint16_t tile[16][128];
  const int lane = (int)(threadIdx.x & 63), kl = (int)(threadIdx.x >> 6);
  const int64_t rw = blockIdx.x >> 2;         // row * waves + w
  const int k0 = 4 * (int)(blockIdx.x & 3), k = k0 + kl;
  const int waves = (a.heads + 15) >> 4;
  if (rw >= (int64_t)rows * waves) return;    // uniform over the workgroup
  const int row = (int)(rw / waves), w = (int)(rw % waves);
  const int hl = lane & 15, head = 16 * w + hl, d0 = 32 * k + 4 * (lane >> 4);
  const bool live = head < a.heads;
  const int hc = live ? head : a.heads - 1;   // padding heads read a live head's partials and write nothing
  float m_run = -__builtin_inff(), l_run = 0.0f;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < a.splits; s0 += 4) {
    float2 ml[4];
    float x[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {   // past the last split: the last one again, weight 0 below
      const int sp = min(s0 + i, a.splits - 1);
      ml[i] = *reinterpret_cast<const float2*>(a.ml + (((int64_t)row * a.splits + sp) * a.heads + hc) * 2);
      const int64_t pi = part_index(a, row, sp, w, k, lane);
      if constexpr (F == kNvfp4) {
        const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.part) + pi);
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const half2_t h = __builtin_bit_cast(half2_t, u[e]);
          x[i][2 * e] = (float)h.x;
          x[i][2 * e + 1] = (float)h.y;
        }
      } else {
        const float4_t* v = reinterpret_cast<const float4_t*>(static_cast<const float*>(a.part) + pi);
        const float4_t v0 = v[0], v1 = v[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[i][e] = v0[e];
          x[i][4 + e] = v1[e];
        }
      }
    }
    float mc = m_run;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (s0 + i >= a.splits) ml[i].x = -__builtin_inff();
      mc = fmaxf(mc, ml[i].x);
    }
    const float mu = (mc == -__builtin_inff()) ? 0.0f : mc;
    const float alpha = __builtin_amdgcn_exp2f(m_run - mu);
    l_run *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= alpha;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float wt = __builtin_amdgcn_exp2f(ml[i].x - mu) * ml[i].y;
      l_run += wt;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += wt * x[i][e];
    }
    m_run = mc;
  }
  const float mu = (m_run == -__builtin_inff()) ? 0.0f : m_run;
  float total = l_run;
  if (a.sink) total += __builtin_amdgcn_exp2f(a.sink[hc] * kLog2e - mu);
  // NVFP4: the partials are without g; it is max(g0, g1) (c[1] is c[0] with one cache), as in the one-split output
  const float gout = F == kNvfp4 ? fmaxf(*a.c[0].g, *a.c[1].g) : 1.0f;
  const float inv = l_run > 0.0f ? gout / total : 0.0f;
  uint32_t pk[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    pk[e] = a.out_dtype == XT_DTYPE_BF16 ? pack2_16<true>(o[2 * e] * inv, o[2 * e + 1] * inv)
                                         : pack2_16<false>(o[2 * e] * inv, o[2 * e + 1] * inv);
  const int c0 = d0 - 32 * k0;   // this thread's dims within the workgroup's 128: c0 .. c0+3 and c0+16 .. c0+19
  *reinterpret_cast<uint2*>(&tile[hl][8 * ((c0 >> 3) ^ hl) + (c0 & 7)]) = make_uint2(pk[0], pk[1]);
  *reinterpret_cast<uint2*>(&tile[hl][8 * (((c0 + 16) >> 3) ^ hl) + (c0 & 7)]) = make_uint2(pk[2], pk[3]);
  if (live && a.lse && d0 == 0)
    a.lse[(int64_t)row * a.heads + head] = l_run > 0.0f ? (mu + __builtin_log2f(l_run)) * kLn2 : -__builtin_inff();
  __syncthreads();
  // thread u: head 16 w + u / 16, dims 32 k0 + 8 (u % 16) .. +7
  const int sh = (int)threadIdx.x >> 4, sc = (int)threadIdx.x & 15;
  if (16 * w + sh < a.heads)
    *reinterpret_cast<uint4*>(a.out + (int64_t)row * a.o_rs + (int64_t)(16 * w + sh) * a.o_hs + 32 * k0 + 8 * (sc ^ sh)) =
        *reinterpret_cast<const uint4*>(&tile[sh][8 * sc]);
}

int check_cache(const char* what, const xt_mla_cache* c, int64_t* pay_stride, int64_t* sf_stride,
                int64_t* rope_stride) {
  if (!c->pay || !c->scales || !c->rope || !c->g) return fail(XT_EINVAL, "%s: a cache pointer is null", what);
  if (c->slots <= 0 || c->slots > 0x3FFFFFFFLL)
    return fail(XT_EINVAL, "%s: cache slots %lld outside 1..2^30-1", what, (long long)c->slots);
  *pay_stride = c->pay_stride ? c->pay_stride : kDl / 2;
  *sf_stride = c->sf_stride ? c->sf_stride : kDl / 16;
  *rope_stride = c->rope_stride ? c->rope_stride : kDr * 2;
  if (*pay_stride < kDl / 2 || *pay_stride % 4 || *sf_stride < kDl / 16 || *rope_stride < kDr * 2 ||
      *rope_stride % 16 || !aligned(c->pay, 4) || !aligned(c->rope, 16) || *pay_stride > 0xFFFFFFFFLL ||
      *sf_stride > 0xFFFFFFFFLL || *rope_stride > 0xFFFFFFFFLL)
    return fail(XT_EINVAL, "%s: cache strides %lld / %lld / %lld bytes or alignment do not fit the latent rows", what,
                (long long)*pay_stride, (long long)*sf_stride, (long long)*rope_stride);
  return XT_OK;
}

int check_pages(const char* what, const xt_mla_fp8_cache* c, CacheDev* cd) {
  if (!c->pages) return fail(XT_EINVAL, "%s: the page buffer is null", what);
  if (c->page_size <= 0 || (c->page_size & (c->page_size - 1)) || c->page_size > 4096)
    return fail(XT_EUNSUPPORTED, "%s: page size %d (supported: powers of 2 up to 4096)", what, c->page_size);
  const int64_t min_bytes = (int64_t)c->page_size * (kV4Row + 8);
  if (c->num_pages <= 0 || c->page_stride < min_bytes || c->page_stride % 16 || !aligned(c->pages, 16))
    return fail(XT_EINVAL, "%s: %lld pages with a %lld-byte stride do not hold %d tokens of 584 bytes (16-byte "
                "aligned)", what, (long long)c->num_pages, (long long)c->page_stride, c->page_size);
  if (c->num_pages * c->page_size > 0x3FFFFFFFLL)
    return fail(XT_EINVAL, "%s: %lld tokens exceed 2^30-1", what, (long long)(c->num_pages * c->page_size));
  *cd = CacheDev{c->pages, nullptr, nullptr, nullptr, c->num_pages * c->page_size, 0u, 0u, 0u,
                 (uint32_t)__builtin_ctz((unsigned)c->page_size), (uint64_t)c->page_stride};
  return XT_OK;
}

size_t mla_workspace_bytes(int rows, int heads, int splits, size_t part_elem) {
  if (rows < 0 || heads <= 0 || splits <= 0) return 0;
  if (splits == 1) return 256;
  const size_t padded = (size_t)((heads + 15) / 16) * 16;   // partials in whole waves of 16 heads
  return kCounterBytes + (size_t)rows * splits * (padded * kDl * part_elem + heads * 2 * sizeof(float));
}

// The per-wave timeline buffer of the MLA launches (xt_mla_timeline); NULL: off.
std::atomic<uint64_t*> g_mla_timeline{nullptr};
std::atomic<size_t> g_mla_timeline_bytes{0};

// Everything but the caches: checks, key lists, split sizing, workspace carving and the launches.
template <int F>
int mla_launch(const char* what, MlaArgs& a, bool extra, const void* q, int64_t q_row_stride, int64_t q_head_stride,
               int heads, const xt_mla_keys* keys, const xt_mla_keys* extra_keys, const float* sink, float scale,
               void* out, int64_t out_row_stride, int64_t out_head_stride, int out_dtype, float* lse, int rows,
               int splits, void* workspace, size_t workspace_bytes, xt_stream_t stream) {
  const size_t part_elem = F == kNvfp4 ? 2 : 4;
  const size_t need = mla_workspace_bytes(rows, heads, splits, part_elem);
  if (workspace_bytes < need)
    return fail(XT_EWORKSPACE, "%s: workspace %zu bytes < %zu needed", what, workspace_bytes, need);
  if (!aligned(workspace, 256)) return fail(XT_EINVAL, "%s: workspace must be 256-byte aligned", what);
  a.q = static_cast<const uint16_t*>(q);
  a.q_rs = q_row_stride;
  a.q_hs = q_head_stride;
  a.idx[0] = keys->indices;
  a.idx_stride[0] = keys->stride;
  a.topk[0] = keys->topk;
  a.len[0] = keys->lengths;
  a.idx[1] = extra ? extra_keys->indices : keys->indices;
  a.idx_stride[1] = extra ? extra_keys->stride : keys->stride;
  a.topk[1] = extra ? extra_keys->topk : 0;
  a.len[1] = extra ? extra_keys->lengths : nullptr;
  a.sink = sink;
  a.qscale = scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.o_rs = out_row_stride;
  a.o_hs = out_head_stride;
  a.out_dtype = out_dtype;
  a.lse = lse;
  a.heads = heads;
  a.splits = splits;
  const int total_keys = a.topk[0] + a.topk[1];
  a.keys_per_split = (((total_keys + splits - 1) / splits + kMSteps - 1) / kMSteps) * kMSteps;
  a.steps = a.keys_per_split / kMSteps;
  if (a.keys_per_split == 0) {
    a.keys_per_split = kMSteps;   // no keys: one all-invalid step writes the zero rows
    a.steps = 1;
  }
  const size_t lds_bytes = (size_t)2 * kKTile<F> + kQTile<F> + (size_t)(a.steps + 1) * kMSteps * 4;
  if (lds_bytes > 160 * 1024 - 256 || (a.steps + 1) * kMSteps > 512 * kSlotIters)
    return fail(XT_EUNSUPPORTED, "%s: %d keys per split need %zu bytes of LDS; use more splits", what,
                a.keys_per_split, lds_bytes);
  char* ws = static_cast<char*>(workspace);
  a.part = ws + kCounterBytes;
  a.ml = reinterpret_cast<float*>(ws + kCounterBytes +
                                  (size_t)rows * splits * ((heads + 15) / 16) * 16 * kDl * part_elem);
  const int64_t n_units = (int64_t)rows * splits;
  if (n_units > 0x7FFFFFFFLL) return fail(XT_EUNSUPPORTED, "%s: %lld workgroups", what, (long long)n_units);
  a.xcd_units = (uint32_t)(n_units / 8);
  a.xcd_extra = (uint32_t)(n_units % 8);
  a.stamps = g_mla_timeline.load();
  a.stamp_blocks = a.stamps ? (uint32_t)std::min<int64_t>(
                                  n_units, (int64_t)(g_mla_timeline_bytes.load() / ((size_t)kMWaves * kMlaStamps * 8)))
                            : 0u;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)n_units), block(64 * kMWaves);
  const bool tl = a.stamps != nullptr;
  const void* fn = extra ? (tl ? reinterpret_cast<const void*>(&mla_kernel<F, true, true>)
                               : reinterpret_cast<const void*>(&mla_kernel<F, true, false>))
                         : (tl ? reinterpret_cast<const void*>(&mla_kernel<F, false, true>)
                               : reinterpret_cast<const void*>(&mla_kernel<F, false, false>));
  if (int e = allow_lds(fn, lds_bytes, what)) return e;
  if (extra && tl)
    hipLaunchKernelGGL((mla_kernel<F, true, true>), grid, block, lds_bytes, st, a);
  else if (extra)
    hipLaunchKernelGGL((mla_kernel<F, true, false>), grid, block, lds_bytes, st, a);
  else if (tl)
    hipLaunchKernelGGL((mla_kernel<F, false, true>), grid, block, lds_bytes, st, a);
  else
    hipLaunchKernelGGL((mla_kernel<F, false, false>), grid, block, lds_bytes, st, a);
  if (splits > 1) {
    const int64_t threads = (int64_t)rows * ((heads + 15) / 16) * 16 * 64;   // (row, wave, dim-tile pair, lane)
    hipLaunchKernelGGL(mla_merge_kernel<F>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), a, rows);
  }
  return check_launch(what);
}

// Checks shared by both entry points; returns XT_OK with *done set when there is nothing to launch.
int mla_common_checks(const char* what, const void* q, int64_t q_row_stride, int64_t q_head_stride, int heads,
                      const void* cache, const xt_mla_keys* keys, const xt_mla_keys* extra_keys, void* out,
                      int64_t out_row_stride, int64_t out_head_stride, int out_dtype, int rows, int splits,
                      void* workspace, bool* done) {
  *done = false;
  if (heads <= 0 || heads > kMHeads) return fail(XT_EUNSUPPORTED, "%s: %d heads (supported: 1..%d)", what, heads,
                                                 kMHeads);
  if (rows < 0 || splits < 1 || splits > 64) return fail(XT_EINVAL, "%s: bad rows %d / splits %d", what, rows, splits);
  if (out_dtype != XT_DTYPE_BF16 && out_dtype != XT_DTYPE_F16)
    return fail(XT_EINVAL, "%s: output dtype must be BF16 or FP16", what);
  if (!cache || !keys) return fail(XT_EINVAL, "%s: the key cache and key list are required", what);
  if (rows == 0) {
    *done = true;
    return ok();
  }
  if (!q || !out || !workspace || !keys->indices) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (!aligned(q, 16) || q_row_stride % 8 || q_head_stride % 8 || !aligned(out, 16) || out_row_stride % 8 ||
      out_head_stride % 8)
    return fail(XT_EINVAL, "%s: q and out rows must be 16-byte aligned (strides in elements: multiples of 8)", what);
  if (keys->topk < 0 || (extra_keys && extra_keys->topk < 0)) return fail(XT_EINVAL, "%s: negative topk", what);
  return XT_OK;
}

}  // namespace
}  // namespace xt

using namespace xt;

// Workspace: [kCounterBytes, unused here: the counter region of the decode entry points][partial outputs [rows,
// splits, heads, 512] FP16 (NVFP4) or FP32 (V4)][partial max and sum [rows, splits, heads, 2] FP32]

extern "C" int xt_mla_timeline(uint64_t* stamps, size_t bytes) {
  if (stamps && (!aligned(stamps, 8) || bytes < 64))
    return fail(XT_EINVAL, "xt_mla_timeline: the stamp buffer must be 8-byte aligned and hold one wave's 8 stamps");
  g_mla_timeline_bytes.store(stamps ? bytes : 0);
  g_mla_timeline.store(stamps);
  return ok();
}

extern "C" size_t xt_sparse_mla_workspace_bytes(int rows, int heads, int splits) {
  return mla_workspace_bytes(rows, heads, splits, 2);
}

extern "C" size_t xt_sparse_mla_fp8_workspace_bytes(int rows, int heads, int splits) {
  return mla_workspace_bytes(rows, heads, splits, 4);
}

extern "C" int xt_sparse_mla_max_split_keys(int fp8) {
  const size_t fixed = fp8 ? 2 * (size_t)kKTile<kFp8V4> + kQTile<kFp8V4> : 2 * (size_t)kKTile<kNvfp4> + kQTile<kNvfp4>;
  return (int)(((160 * 1024 - 256 - fixed) / (kMSteps * 4) - 1) * kMSteps);   // one padding step in the slot list
}

extern "C" int xt_sparse_mla_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride, int heads,
                                   int latent_dim, int rope_dim, const xt_mla_cache* cache, const xt_mla_keys* keys,
                                   const xt_mla_cache* extra_cache, const xt_mla_keys* extra_keys, const float* sink,
                                   float scale, void* out, int64_t out_row_stride, int64_t out_head_stride,
                                   int out_dtype, float* lse, int rows, int splits, void* workspace,
                                   size_t workspace_bytes, xt_stream_t stream) {
  const char* what = "xt_sparse_mla_nvfp4";
  if (latent_dim != kDl || rope_dim != kDr)
    return fail(XT_EUNSUPPORTED, "%s: latent %d + rope %d (supported: %d + %d)", what, latent_dim, rope_dim, kDl, kDr);
  bool done;
  int st = mla_common_checks(what, q, q_row_stride, q_head_stride, heads, cache, keys, extra_keys, out,
                             out_row_stride, out_head_stride, out_dtype, rows, splits, workspace, &done);
  if (st != XT_OK || done) return st;
  const bool extra = extra_cache && extra_keys && extra_keys->indices && extra_keys->topk > 0;
  MlaArgs a;
  int64_t ps, ss, rs;
  st = check_cache(what, cache, &ps, &ss, &rs);
  if (st != XT_OK) return st;
  a.c[0] = CacheDev{cache->pay, cache->scales, static_cast<const uint16_t*>(cache->rope), cache->g, cache->slots,
                    (uint32_t)ps, (uint32_t)ss, (uint32_t)rs, 0u, 0u};
  if (extra) {
    st = check_cache(what, extra_cache, &ps, &ss, &rs);
    if (st != XT_OK) return st;
    a.c[1] = CacheDev{extra_cache->pay, extra_cache->scales, static_cast<const uint16_t*>(extra_cache->rope),
                      extra_cache->g, extra_cache->slots, (uint32_t)ps, (uint32_t)ss, (uint32_t)rs, 0u, 0u};
  } else {
    a.c[1] = a.c[0];
  }
  auto fits32 = [](const CacheDev& c) {
    return c.slots < (1 << 24) && (uint64_t)c.slots * c.pay_stride <= 0xFFFFFFFFull &&
           (uint64_t)c.slots * c.sf_stride <= 0xFFFFFFFFull && (uint64_t)c.slots * c.rope_stride <= 0xFFFFFFFFull;
  };
  a.o32 = fits32(a.c[0]) && fits32(a.c[1]);
  return mla_launch<kNvfp4>(what, a, extra, q, q_row_stride, q_head_stride, heads, keys, extra_keys, sink, scale, out,
                            out_row_stride, out_head_stride, out_dtype, lse, rows, splits, workspace,
                            workspace_bytes, stream);
}

extern "C" int xt_sparse_mla_fp8(const void* q, int64_t q_row_stride, int64_t q_head_stride, int heads,
                                 const xt_mla_fp8_cache* cache, const xt_mla_keys* keys,
                                 const xt_mla_fp8_cache* extra_cache, const xt_mla_keys* extra_keys, const float* sink,
                                 float scale, void* out, int64_t out_row_stride, int64_t out_head_stride,
                                 int out_dtype, float* lse, int rows, int splits, void* workspace,
                                 size_t workspace_bytes, xt_stream_t stream) {
  const char* what = "xt_sparse_mla_fp8";
  bool done;
  int st = mla_common_checks(what, q, q_row_stride, q_head_stride, heads, cache, keys, extra_keys, out,
                             out_row_stride, out_head_stride, out_dtype, rows, splits, workspace, &done);
  if (st != XT_OK || done) return st;
  const bool extra = extra_cache && extra_keys && extra_keys->indices && extra_keys->topk > 0;
  MlaArgs a;
  a.o32 = 0;
  st = check_pages(what, cache, &a.c[0]);
  if (st != XT_OK) return st;
  if (extra) {
    st = check_pages(what, extra_cache, &a.c[1]);
    if (st != XT_OK) return st;
  } else {
    a.c[1] = a.c[0];
  }
  return mla_launch<kFp8V4>(what, a, extra, q, q_row_stride, q_head_stride, heads, keys, extra_keys, sink, scale, out,
                            out_row_stride, out_head_stride, out_dtype, lse, rows, splits, workspace,
                            workspace_bytes, stream);
}
