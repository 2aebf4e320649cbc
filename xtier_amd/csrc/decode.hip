// Fused sparse GQA attention over the NVFP4 paged pool: gather through the page table, dequantize in registers, QK
// and PV on MFMA (v_mfma_f32_16x16x32_f16), online softmax in the exp2 domain, in one launch. With one key split per
// row a workgroup writes its heads' outputs directly; with several, each workgroup writes one partial result per
// (row, key split, head), and the last workgroup of a (row, KV head group) to finish merges them.
//
// Work decomposition: a workgroup = W wavefronts = HPW consecutive KV heads x W / HPW key slices of one (query row,
// key split). HPW = 4 when the KV heads are a multiple of 4 and that alone fills every CU, else 2 when a multiple of 2
// fills them, else 1 (more workgroups).
// W = 8 while the workgroups fit one round on the CUs (decode batches), else 4, compiled for two workgroups per CU
// (prefill chunks, one row per query). Each wave owns one (row, KV head, split, slice) and walks its keys in steps of
// 32; with 2 KV heads and 8 waves per workgroup at head size 128 and GQA groups up to 8 (the batch-32 decode), each
// wave instead owns both heads of the pair (paired waves, steps of 16 keys: one contiguous run of the pair's payload
// per key and wave, every MFMA column a query head). The workgroup computes the split's pool slots once into LDS and
// merges the slices of each head through LDS
// behind one barrier. Workgroups are numbered so that all units of a row run on the same XCD (round-robin dispatch
// puts workgroup g on XCD g % 8): their K/V lines, which hold several heads, and their partials share one L2.
//
// Memory pipeline: per step a wave issues 6 loads (K and V payload as row pieces, K and V scales as dwords) and keeps
// P steps in flight in a register ring. V is transposed for the PV operand through a padded LDS tile; the K scales
// reach their lanes with ds_bpermute.
//
// Numerics: e2m1 * e4m3 is exact in FP16 (at most 6 significant bits, magnitudes 2^-10 .. 2688), so K and V enter
// the MFMA exactly without their global scales; the query enters as FP16 of q * scale * log2(e); the K global scale
// multiplies the FP32 scores and the V global scale the merged output. P is FP16 for the PV product, sums are FP32.
// The running maximum is raised only when a score exceeds it by more than 2^8 (lazy rescale), so P <= 256.
//
// Lane layouts (16x16x32 MFMA: A[i][k] = lane i + 16*(k/8), element k%8; B[k][j] = lane j + 16*(k/8), element k%8;
// C[i][j] = lane j + 16*(i/4), element i%4). With hl = lane % 16, j = lane / 16 and head size D (64, 128, 256):
//   QK: C = S^T [16 keys x 16 heads]; A = K tile, lane (key hl, payload bytes (D/8) j .. of the head row); MFMA kk
//       (0 .. D/32 - 1) contracts dword kk of those bytes, d = (D/4) j + 8kk + e; B = Q^T in the same d order. Lane
//       (hl, j) ends up with the scores of head hl for keys T(j) = {4j..4j+3, 16+4j..16+4j+3} of the step.
//   PV: C = O^T [16 rows x 16 heads] per tile t of 16 payload dwords, row c = payload dword 16t + c of the head row;
//       MFMA i (0..7) takes nibble i of every dword, d = 8 (16t + c) + i. A = V^T, lane (dword hl, keys T(j)); B = P^T,
//       lane (head hl, keys T(j)) in the same order. Lane (hl, j) ends up with O^T of head hl for
//       d = 128t + 32j .. 128t + 32j + 31 (D = 64: one tile, lanes j >= 2 empty).
#include "xt_common.h"
#include "xt_host.h"

#include <atomic>
#include <mutex>
#include <type_traits>

namespace xt {
namespace {

constexpr int kStep = 32;          // keys per step
constexpr int kWaves = 8;          // wavefronts per workgroup while one round of workgroups covers the launch
constexpr int kSlotBatch = 4;      // keys per thread whose index / table loads are in flight together
constexpr float kRescale = 8.0f;   // log2 of the largest P before the running maximum is raised
constexpr size_t kMaxLds = 160 * 1024 - 256;   // dynamic LDS per workgroup (the rest: static LDS)

// How a head row of size D (64, 128 or 256) maps onto the lanes and LDS. In the QK layout four lanes (j = 0..3) share
// a key, lane j holding payload bytes kLaneBytes * j .. of it, i.e. dims d = (D / 4) j + 8 kk + e for its kNK dwords
// kk; the scales of those dims are kLaneBytes / 8 consecutive bytes. O^T has one row per payload dword (D / 8 rows) in
// kNT tiles of 16 (D = 64: one tile, rows 8..15 empty).
template <int D>
struct Geo {
  static constexpr int kPay = D / 2;                   // payload bytes of a head row
  static constexpr int kSf = D / 16;                   // scale bytes of a head row
  static constexpr int kLaneBytes = D / 8;             // payload bytes per lane and key in the QK layout
  static constexpr int kNK = D / 32;                   // QK MFMAs per 16-key tile (payload dwords per lane)
  static constexpr int kNT = D >= 128 ? D / 128 : 1;   // 16-row tiles of O^T
  static constexpr int kScaleWords = D >= 256 ? 2 : 1; // K (and V) scale dwords per lane and step
  static constexpr int kVRow = kPay + 16;              // LDS bytes per key in the V transpose tile (80 at D = 128:
                                                       // no bank conflicts)
  static constexpr int kWaveLds = kStep * kVRow + kStep * kSf;   // V tile + V scale tile per wave
  static constexpr int kPartBytes = 2 * D + 16;        // bytes per partial (split, head): D FP16 outputs normalized
                                                       // by the split's sum, then FP32 max, sum and pad
  static constexpr int kMergeRow = 32 * kNT + 4;       // floats per lane in the slice merge: accumulators, max, sum, pad
  static constexpr int kPrefetch = D >= 256 ? 1 : 2;   // steps of loads in flight per wave (D = 256: registers;
                                                       // batch-32 decode: 2 steps 19.1 us, 4 steps 20.1 us)
  template <int W>
  static constexpr int kMergeLds = W * 64 * kMergeRow * 4;   // one merge region per wave
};

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_rs, q_hs;
  const uint8_t* k_pay;
  const uint8_t* v_pay;
  const uint8_t* k_sf;
  const uint8_t* v_sf;
  const float* gk;                   // device global scales; NULL: gk_val / gv_val
  const float* gv;
  float gk_val, gv_val;
  int64_t pool_slots;                // slots addressable as slot * stride (after the page-row remap below)
  int64_t pay_stride, sf_stride;     // bytes from one slot to the next in the payload / scale buffers
  int64_t pay_head_stride, sf_head_stride;   // bytes from one KV head to the next within a slot's row
  int remap_shift;                   // head-major pages: slot s -> (s >> remap_shift) * remap_mul + low bits (0: s)
  int64_t remap_mul;
  int kv_heads, q_heads, group, kv_groups;
  const int32_t* table;
  int64_t table_stride;
  int page_size;
  int page_shift;                    // log2(page_size) for a power of 2, else -1
  const int64_t* row_req;
  const int32_t* indices;
  int64_t idx_stride;
  int64_t idx_head_stride;           // elements between the index lists of consecutive KV heads (0: one shared list)
  int block_shift;                   // an index names 2^block_shift consecutive positions (0: one token)
  int lookup_mask;                   // positions resolve through the table entry of (pos & ~lookup_mask): the block's
                                     // first position (block decode) or every position (0)
  const int32_t* idx_rows;           // per row, the index row to read (NULL: the row itself)
  int max_len;                       // sequence lengths are clamped to this
  int topk;                          // keys per row (index entries << block_shift)
  const int32_t* counts;
  const int32_t* seq_lens;
  const int32_t* query_pos;
  float qscale;                      // softmax scale * log2(e)
  int rows, splits, keys_per_split;  // keys_per_split: a multiple of kStep
  int slot_lds_bytes;                // LDS bytes of the slot list (padded to whole prefetch groups per slice)
  uint16_t* out;
  int64_t o_rs, o_hs;
  int out_dtype;
  float* lse;
  float* part;                       // [rows, splits, q_heads] records of 2 D + 16 bytes: D FP16 outputs normalized by
                                     // the split's sum, max (log2), sum, pad (the workspace holds D + 4 floats each)
  int32_t* counters;                 // [rows * kv_groups] arrivals per (row, KV group); zero between launches
  int64_t n_units;                   // rows * kv_groups * splits workgroups, one per unit
  uint32_t xcd_units;                // n_units / 8
  uint32_t xcd_extra;                // n_units % 8
  uint64_t* stamps;                  // per-wave timeline (xt_decode_timeline), NULL: off
  uint32_t stamp_blocks;             // workgroups whose stamps fit the buffer
};

// The phases of the per-wave timeline, in stamp order.
enum { kStEntry, kStSlots, kStStep0, kStLoop, kStSliceMerge, kStPartials, kStArrived, kStSplitMerge, kStamps };

template <int D>
struct Step {
  uint32_t kw[2][Geo<D>::kNK];     // K payload bytes kLaneBytes * j .. of key 16 * tt + hl
  uint32_t vw[2][Geo<D>::kNK];     // V payload, same keys and bytes
  uint32_t ks[Geo<D>::kScaleWords];   // K scale dwords of key scale_key(lane), from dword scale_word(lane)
  uint32_t vs[Geo<D>::kScaleWords];   // V scale dwords, same
};

// The key whose scale dwords a lane loads: lanes 2k, 2k + 1 share key k (D >= 128); D = 64 has one dword per key, held
// by lane k (lanes 32..63 repeat lanes 0..31).
template <int D>
__device__ inline int scale_key(int lane) { return D == 64 ? (lane & 31) : (lane >> 1); }
// The first of the lane's kScaleWords dwords within the key's scale row.
template <int D>
__device__ inline int scale_word(int lane) { return D == 64 ? 0 : (lane & 1) * Geo<D>::kScaleWords; }

template <int N>
__device__ inline void load_words(const uint8_t* p, uint32_t (&w)[N]) {
  if constexpr (N == 2) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    w[0] = x.x;
    w[1] = x.y;
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const uint4 x = *reinterpret_cast<const uint4*>(p + 4 * i);
      w[i] = x.x;
      w[i + 1] = x.y;
      w[i + 2] = x.z;
      w[i + 3] = x.w;
    }
  }
}

template <int N>
__device__ inline void store_words(uint8_t* p, const uint32_t (&w)[N]) {
  if constexpr (N == 2) {
    *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4)
      *reinterpret_cast<uint4*>(p + 4 * i) = make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]);
  }
}

__device__ inline int key_of(int j, int e) { return (e < 4) ? (4 * j + e) : (16 + 4 * j + (e - 4)); }

__device__ inline half8_t dequant_k(uint32_t w, half2_t sc) {
  const half2_t p0 = fp4x2_to_f16<0>(w) * sc;
  const half2_t p1 = fp4x2_to_f16<1>(w) * sc;
  const half2_t p2 = fp4x2_to_f16<2>(w) * sc;
  const half2_t p3 = fp4x2_to_f16<3>(w) * sc;
  return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

struct WaveCtx {
  const uint8_t* kp;    // this head's payload column (uniform over the wave)
  const uint8_t* vp;
  const uint8_t* ksf;   // this head's scale column
  const uint8_t* vsf;
  const uint8_t* kp2;   // paired waves: the second head's payload and K scale columns
  const uint8_t* vp2;
  const uint8_t* ksf2;
  uint32_t vs_off;      // paired waves: this lane's V scale dword within the first head's scale column
  int64_t row_bytes, row_scales;
  const int32_t* slots;  // this wave's slot list in LDS (-1: invalid)
  int lane, hl, j;
};

// The byte offset of a slot's row plus a lane offset. O32: every slot is below 2^24 and every row offset below 2^32
// (checked on the host), so one 24-bit multiply-add gives it and the load takes the uniform column address plus a
// 32-bit offset; otherwise 64-bit arithmetic.
template <bool O32>
__device__ inline const uint8_t* row_at(const uint8_t* col, int32_t slot, int64_t stride, uint32_t lane_off) {
  const uint32_t s = slot < 0 ? 0u : (uint32_t)slot;
  if constexpr (O32) return col + ((uint32_t)__umul24(s, (uint32_t)stride) + lane_off);   // __umul24 is signed
  else return col + (int64_t)s * stride + lane_off;
}

// PS (D = 128 only): the K and V scales of a head are 16 contiguous bytes (the interleaved pool): one load serves
// both, the even lane of each pair taking the K half and the odd lane the V half; compute_step swaps the halves within
// the pair.
template <int D, bool PS, bool O32>
__device__ inline void load_step(const WaveCtx& w, int step, Step<D>& d) {
  using G = Geo<D>;
  const int base = step * kStep;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int32_t s = w.slots[base + 16 * tt + w.hl];
    load_words(row_at<O32>(w.kp, s, w.row_bytes, G::kLaneBytes * w.j), d.kw[tt]);
    load_words(row_at<O32>(w.vp, s, w.row_bytes, G::kLaneBytes * w.j), d.vw[tt]);
  }
  const int32_t s = w.slots[base + scale_key<D>(w.lane)];
  if constexpr (PS) {
    const uint2 x = *reinterpret_cast<const uint2*>(row_at<O32>(w.ksf, s, w.row_scales, 8 * (w.lane & 1)));
    d.ks[0] = x.x;
    d.vs[0] = x.y;
  } else {
    const uint32_t off = 4 * scale_word<D>(w.lane);
#pragma unroll
    for (int i = 0; i < G::kScaleWords; ++i) {
      d.ks[i] = *reinterpret_cast<const uint32_t*>(row_at<O32>(w.ksf, s, w.row_scales, off + 4 * i));
      d.vs[i] = *reinterpret_cast<const uint32_t*>(row_at<O32>(w.vsf, s, w.row_scales, off + 4 * i));
    }
  }
}

// Paired waves (head size 128, GQA group <= 8): one wave covers the two KV heads of a pair in steps of 16 keys, the
// group of head h in MFMA columns 8h .. 8h + 7, so every column is a query head. QK contracts the 256 dims of both
// heads (MFMAs 0-3 head 0's, 4-7 head 1's) against a block-diagonal Q^T (head 0's columns zero in head 1's dims and
// the other way round); PV contracts 32 (head, key) pairs, rows 0-15 of the V tile head 0's keys and 16-31 head 1's,
// against a block-diagonal P^T. A key's payload of the two heads is one 256-byte run of the interleaved pool (one
// 128-byte line per K or V on SGLang's split pool), read by one wave.
constexpr int kPairStep = 16;      // keys per step of a paired wave
struct PairStep {
  uint32_t kw[2][4];   // K payload bytes 16 j .. 16 j + 15 of key hl, head h of the pair
  uint32_t vw[2][4];   // V payload, same
  uint32_t ks[2];      // K scale dword j / 2 of key hl, head h: the scale bytes 2 j, 2 j + 1 of this lane's dims
  uint32_t vs;         // V scale dword j % 2 of key hl, head j / 2
};

template <bool O32>
__device__ inline void load_step_pair(const WaveCtx& w, int step, PairStep& d) {
  const int32_t s = w.slots[step * kPairStep + w.hl];
  const uint32_t po = 16u * (uint32_t)w.j;
  load_words(row_at<O32>(w.kp, s, w.row_bytes, po), d.kw[0]);
  load_words(row_at<O32>(w.kp2, s, w.row_bytes, po), d.kw[1]);
  load_words(row_at<O32>(w.vp, s, w.row_bytes, po), d.vw[0]);
  load_words(row_at<O32>(w.vp2, s, w.row_bytes, po), d.vw[1]);
  const uint32_t so = 4u * (uint32_t)(w.j >> 1);
  d.ks[0] = *reinterpret_cast<const uint32_t*>(row_at<O32>(w.ksf, s, w.row_scales, so));
  d.ks[1] = *reinterpret_cast<const uint32_t*>(row_at<O32>(w.ksf2, s, w.row_scales, so));
  d.vs = *reinterpret_cast<const uint32_t*>(row_at<O32>(w.vsf, s, w.row_scales, w.vs_off));
}

// Bit 7 of byte b set where byte b of x is an E4M3 NaN (0x7F / 0xFF).
__device__ inline uint32_t e4m3_nan_bytes(uint32_t x) { return ((x & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u; }
// 16-bit mask of the keys (lanes hl, hl + 16, hl + 32, hl + 48 -> bit hl) where the predicate holds in any lane.
__device__ inline uint32_t key_mask16(bool pred) {
  const uint64_t b = __builtin_amdgcn_ballot_w64(pred);
  return (uint32_t)((b | (b >> 16) | (b >> 32) | (b >> 48)) & 0xFFFFu);
}

template <int D>
struct SoftmaxState {
  float m;            // reference maximum of head hl (log2 domain), identical on the 4 lanes of the head
  float l;            // this lane's share of the sum of 2^(s - m)
  float4_t acc[Geo<D>::kNT][8];   // O^T of head hl: tile t, dims d = 8 (16 t + 4 j + r) + i in acc[t][i][r]
};

template <int D>
__device__ inline void pv_step(int hl, int j, const half8_t& pb, const uint8_t* vtile, SoftmaxState<D>& st);

template <int D, bool PS>
__device__ inline void compute_step(const WaveCtx& w, int step, const Step<D>& d, const half8_t (&qb)[Geo<D>::kNK],
                                    float smul, uint8_t* vtile, SoftmaxState<D>& st) {
  using G = Geo<D>;
  const int lane = w.lane, hl = w.hl, j = w.j;
  // validity of the step's 32 keys (bit t: key t), uniform over the wave
  const uint32_t valid =
      (uint32_t)__builtin_amdgcn_ballot_w64(lane < kStep && w.slots[step * kStep + (lane & 31)] >= 0);
  const bool my_scale_valid = (valid >> scale_key<D>(lane)) & 1u;
  uint32_t ks[G::kScaleWords], vs[G::kScaleWords];
#pragma unroll
  for (int i = 0; i < G::kScaleWords; ++i) {
    ks[i] = d.ks[i];
    vs[i] = d.vs[i];
  }
  if constexpr (PS) {   // even lane: K words 0, 1; odd lane: V words 0, 1 (quad_perm [1, 0, 3, 2] swaps the pair)
    const uint32_t o0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)d.ks[0], 0xB1, 0xF, 0xF, false);
    const uint32_t o1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)d.vs[0], 0xB1, 0xF, 0xF, false);
    const bool odd = lane & 1;
    ks[0] = odd ? o1 : d.ks[0];
    vs[0] = odd ? d.vs[0] : o0;
  }
#pragma unroll
  for (int i = 0; i < G::kScaleWords; ++i)   // invalid keys: V scale 0, so V = 0 whatever slot 0 holds
    vs[i] = my_scale_valid ? vs[i] : 0u;

  // V: stage payload and scales in LDS, transposed reads below
  uint8_t* vscale = vtile + kStep * G::kVRow;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) store_words(vtile + (16 * tt + hl) * G::kVRow + G::kLaneBytes * j, d.vw[tt]);
  if constexpr (D == 64) {
    if (lane < 32) *reinterpret_cast<uint32_t*>(vscale + lane * 4) = vs[0];
  } else {
#pragma unroll
    for (int i = 0; i < G::kScaleWords; ++i)
      *reinterpret_cast<uint32_t*>(vscale + scale_key<D>(lane) * G::kSf + 4 * (scale_word<D>(lane) + i)) = vs[i];
  }

  // QK: lane (hl, j) of tile tt needs the scale bytes of its dims, kLaneBytes / 8 bytes from byte (D / 64) j of key
  // 16 tt + hl, taken from the lane that loaded them
  float4_t s[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int key = 16 * tt + hl;
    uint32_t chunk;
    if constexpr (D == 64) {
      chunk = (uint32_t)__shfl((int)ks[0], key) >> (8 * j);
    } else if constexpr (D == 128) {
      chunk = (uint32_t)__shfl((int)ks[0], 2 * key + (j >> 1)) >> (16 * (j & 1));
    } else {
      const uint32_t a0 = (uint32_t)__shfl((int)ks[0], 2 * key + (j >> 1));
      const uint32_t a1 = (uint32_t)__shfl((int)ks[1], 2 * key + (j >> 1));
      chunk = (j & 1) ? a1 : a0;
    }
    const half2_t c01 = fp8x2_to_f16<false>(chunk);
    const half2_t c23 = D == 256 ? fp8x2_to_f16<true>(chunk) : c01;
    s[tt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < G::kNK; ++kk) {
      const int bi = kk >> 1;   // scale block of dword kk within the lane's bytes
      const _Float16 sc = bi == 0 ? c01.x : bi == 1 ? c01.y : bi == 2 ? c23.x : c23.y;
      s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(dequant_k(d.kw[tt][kk], half2_t{sc, sc}), qb[kk], s[tt], 0, 0,
                                                     0);
    }
  }
  // online softmax of head hl over keys T(j), lazy rescale. The scores' multiplier smul (this lane's head's: K global
  // scale, softmax scale, log2(e) and the query's power of two) is positive, so a masked score (-inf) gives P = 0.
  // Only a step with invalid keys (a slice's tail, causal limits) masks scores, a branch uniform over the wave.
  // The maximum reads the products (ordinary VALU results), never the MFMA accumulators themselves: inline asm gets
  // no MFMA read-after-write wait states from the compiler.
  const bool full = valid == 0xFFFFFFFFu;
  float sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sv[e] = s[e >> 2][e & 3] * smul;
  if (!full) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sv[e] = ((valid >> key_of(j, e)) & 1u) ? sv[e] : -__builtin_inff();
  }
  float mt = max3_raw(max3_raw(sv[0], sv[1], sv[2]), max3_raw(sv[3], sv[4], sv[5]), max2_raw(sv[6], sv[7]));
  mt = max4_lanes16(mt);
  if (__builtin_amdgcn_ballot_w64(mt > st.m + kRescale)) {   // rare after the first steps
    const float m_new = (mt > st.m + kRescale) ? mt : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= alpha;
#pragma unroll
    for (int t = 0; t < G::kNT; ++t)
#pragma unroll
      for (int i = 0; i < 8; ++i) st.acc[t][i] *= alpha;
    st.m = m_new;
  }
  const float m_use = (st.m == -__builtin_inff()) ? 0.0f : st.m;
  float p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(sv[e] - m_use);
  st.l += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  const half8_t pb = half8_t{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
                             (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
  pv_step<D>(hl, j, pb, vtile, st);
}

// O^T += V^T . P^T over the V tile of the step: rows key_of(j, e) (a 32-key step's keys; paired waves: head 0's 16
// keys, then head 1's), payload at vtile, scale bytes after kStep rows.
template <int D>
__device__ inline void pv_step(int hl, int j, const half8_t& pb, const uint8_t* vtile, SoftmaxState<D>& st) {
  using G = Geo<D>;
  const uint8_t* vscale = vtile + kStep * G::kVRow;
  // V^T operands of tile t: payload dword c = 16 t + hl of keys T(j), and the scale byte of block c / 2 of those keys
  asm volatile("" ::: "memory");
#pragma unroll
  for (int t = 0; t < G::kNT; ++t) {
    const int c = 16 * t + hl;
    const bool row_ok = c < D / 8;   // D = 64: O^T rows 8..15 are empty
    const int cr = row_ok ? c : 0;
    uint32_t vw[8], vb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = key_of(j, e);
      vw[e] = row_ok ? *reinterpret_cast<const uint32_t*>(vtile + key * G::kVRow + 4 * cr) : 0u;
      vb[e] = row_ok ? vscale[key * G::kSf + (cr >> 1)] : 0u;
    }
    half8_t av[8];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const uint32_t w0 = vw[e], w1 = vw[e + 1];
      const uint32_t lo = (w0 & 0x0F0F0F0Fu) | ((w1 & 0x0F0F0F0Fu) << 4);   // byte b: nibble 2b of keys e, e+1
      const uint32_t hi = ((w0 >> 4) & 0x0F0F0F0Fu) | (w1 & 0xF0F0F0F0u);   // byte b: nibble 2b+1
      const half2_t sp = fp8x2_to_f16<false>(vb[e] | (vb[e + 1] << 8));
      half2_t x;
      x = fp4x2_to_f16<0>(lo) * sp; av[0][e] = x.x; av[0][e + 1] = x.y;
      x = fp4x2_to_f16<0>(hi) * sp; av[1][e] = x.x; av[1][e + 1] = x.y;
      x = fp4x2_to_f16<1>(lo) * sp; av[2][e] = x.x; av[2][e + 1] = x.y;
      x = fp4x2_to_f16<1>(hi) * sp; av[3][e] = x.x; av[3][e + 1] = x.y;
      x = fp4x2_to_f16<2>(lo) * sp; av[4][e] = x.x; av[4][e + 1] = x.y;
      x = fp4x2_to_f16<2>(hi) * sp; av[5][e] = x.x; av[5][e + 1] = x.y;
      x = fp4x2_to_f16<3>(lo) * sp; av[6][e] = x.x; av[6][e + 1] = x.y;
      x = fp4x2_to_f16<3>(hi) * sp; av[7][e] = x.x; av[7][e + 1] = x.y;
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], pb, st.acc[t][i], 0, 0, 0);
  }
}

// One 16-key step of a paired wave (head size 128). Lane (hl, j) loaded key hl's pieces of both heads; it ends up with
// the scores of column hl (head hl / 8 of the pair) for keys 4 j .. 4 j + 3. qb[kk]: the block-diagonal Q^T, zero
// where the column's head does not own MFMA kk's dims.
// A NaN scale byte of a valid key must reach only its own head's outputs, as separate heads would: the zero blocks of
// Q^T and P^T multiply the other head's values, and 0 * NaN is NaN. A step holding one (a ballot, uniform over the
// wave) therefore takes the NaN bytes out of the operands and puts NaN where separate heads would have it: into the
// scores of the (key, head) pairs of a K scale, into the outputs of the (head, 16-dim block) pairs of a V scale.
__device__ inline void compute_step_pair(const WaveCtx& w, int step, const PairStep& d, const half8_t (&qb)[8],
                                         float smul, uint8_t* vtile, SoftmaxState<128>& st) {
  using G = Geo<128>;
  const int lane = w.lane, hl = w.hl, j = w.j;
  const uint32_t valid = key_mask16(lane < kPairStep && w.slots[step * kPairStep + hl] >= 0);
  const bool key_ok = (valid >> hl) & 1u;
  uint32_t ks0 = d.ks[0], ks1 = d.ks[1];
  uint32_t vs = key_ok ? d.vs : 0u;   // invalid keys: V scale 0, so V = 0 whatever slot 0 holds
  uint32_t nan_k0 = 0u, nan_k1 = 0u;  // per head: keys with a NaN K scale byte
  uint32_t nan_vb = 0u;               // blocks (bit b: dims 16 b ..) of column hl's head with a NaN V scale byte
  bool nan_v = false;
  if (__builtin_amdgcn_ballot_w64(key_ok && (e4m3_nan_bytes(ks0) | e4m3_nan_bytes(ks1) | e4m3_nan_bytes(vs)))) {
    const uint32_t n0 = e4m3_nan_bytes(ks0), n1 = e4m3_nan_bytes(ks1), nv = e4m3_nan_bytes(vs);
    nan_k0 = key_mask16(key_ok && n0);
    nan_k1 = key_mask16(key_ok && n1);
    // lane (key, j) holds V scale bytes 4 (j % 2) .. + 3 of head j / 2, i.e. blocks 4 (j % 2) + b
    uint32_t m0 = 0u, m1 = 0u;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint64_t bal = __builtin_amdgcn_ballot_w64((nv >> (8 * b + 7)) & 1u);
      m0 |= (((bal & 0xFFFFull) != 0) << b) | ((((bal >> 16) & 0xFFFFull) != 0) << (4 + b));
      m1 |= ((((bal >> 32) & 0xFFFFull) != 0) << b) | ((((bal >> 48) & 0xFFFFull) != 0) << (4 + b));
    }
    nan_vb = hl < 8 ? m0 : m1;
    nan_v = (m0 | m1) != 0u;
    ks0 &= ~((n0 >> 7) * 0xFFu);   // NaN bytes -> 0 (bit 7 of a byte times 0xFF: that byte all ones)
    ks1 &= ~((n1 >> 7) * 0xFFu);
    vs &= ~((nv >> 7) * 0xFFu);
  }

  // V: payload rows 16 h + key, then the scale rows in the same order
  store_words(vtile + hl * G::kVRow + 16 * j, d.vw[0]);
  store_words(vtile + (16 + hl) * G::kVRow + 16 * j, d.vw[1]);
  *reinterpret_cast<uint32_t*>(vtile + kStep * G::kVRow + (16 * (j >> 1) + hl) * G::kSf + 4 * (j & 1)) = vs;

  // QK: dword kk of the lane's 16 payload bytes holds dims 32 j + 8 kk .., scale byte 2 j + kk / 2 of the head row
  float4_t s = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const half2_t c01 = fp8x2_to_f16<false>((h ? ks1 : ks0) >> (16 * (j & 1)));
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const _Float16 sc = kk < 2 ? c01.x : c01.y;
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(dequant_k(d.kw[h][kk], half2_t{sc, sc}), qb[4 * h + kk], s, 0, 0, 0);
    }
  }
  float sv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) sv[e] = s[e] * smul;
  if (valid != 0xFFFFu) {
#pragma unroll
    for (int e = 0; e < 4; ++e) sv[e] = ((valid >> (4 * j + e)) & 1u) ? sv[e] : -__builtin_inff();
  }
  if (nan_k0 | nan_k1) {
    const uint32_t nk = hl < 8 ? nan_k0 : nan_k1;
#pragma unroll
    for (int e = 0; e < 4; ++e) sv[e] = ((nk >> (4 * j + e)) & 1u) ? __builtin_nanf("") : sv[e];
  }
  float mt = max2_raw(max2_raw(sv[0], sv[1]), max2_raw(sv[2], sv[3]));
  mt = max4_lanes16(mt);
  if (__builtin_amdgcn_ballot_w64(mt > st.m + kRescale)) {   // rare after the first steps
    const float m_new = (mt > st.m + kRescale) ? mt : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[0][i] *= alpha;
    st.m = m_new;
  }
  const float m_use = (st.m == -__builtin_inff()) ? 0.0f : st.m;
  float p[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) p[e] = __builtin_amdgcn_exp2f(sv[e] - m_use);
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
  const _Float16 z = (_Float16)0.0f;
  const half8_t pb = hl < 8 ? half8_t{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3], z, z, z, z}
                            : half8_t{z, z, z, z, (_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
  pv_step<128>(hl, j, pb, vtile, st);
  if (nan_v) {   // acc[0][i][r] holds dims 8 (4 j + r) + i: block (4 j + r) / 2
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if ((nan_vb >> ((4 * j + r) >> 1)) & 1u)
#pragma unroll
        for (int i = 0; i < 8; ++i) st.acc[0][i][r] = __builtin_nanf("");
  }
}

__device__ inline void store_out(const DecodeArgs& a, int row, int head, int d0, const float* v, int n) {
  uint16_t* o = a.out + (int64_t)row * a.o_rs + (int64_t)head * a.o_hs + d0;
  for (int e = 0; e < n; e += 2) {
    *reinterpret_cast<uint32_t*>(o + e) =
        a.out_dtype == XT_DTYPE_BF16 ? pack2_16<true>(v[e], v[e + 1]) : pack2_16<false>(v[e], v[e + 1]);
  }
}

// D: head size; HPW: KV heads per workgroup (4, 2 or 1); the workgroup's W / HPW key slices of each head merge through
// LDS. Two waves per SIMD (one 8-wave or two 4-wave workgroups per CU); three for the 4-wave workgroups of 4 KV heads
// (prefill chunks: one slice per head, no LDS merge region, so three workgroups fit a CU's LDS; 168 VGPRs, the few
// values spilled are held across the main loop only: the batch-4096 prefill chunk 622 -> 599 us). Head size 256
// stays at two: its accumulators alone would spill ~100 registers at 168.
template <int D, int P, int HPW, bool PS, int W, bool O32, bool PR>
__global__ void __launch_bounds__(64 * W, (W == 4 && HPW == 4 && D <= 128) ? 3 : 2)
    decode_split_kernel(const DecodeArgs a) {
  using G = Geo<D>;
  static_assert(!PR || (D == 128 && HPW % 2 == 0), "paired waves: head size 128, whole pairs of KV heads");
  constexpr int kWaveHeads = PR ? 2 : 1;            // KV heads per wave
  constexpr int kHeadSets = HPW / kWaveHeads;       // distinct wave head sets per workgroup
  constexpr int kSlices = W / kHeadSets;
  constexpr int kThreads = 64 * W;
  constexpr int KS = PR ? kPairStep : kStep;        // keys per step
  extern __shared__ __align__(16) uint8_t lds[];
  // XCD-aware numbering: workgroup g runs on XCD g % 8 (round-robin dispatch); XCD x takes the contiguous unit range
  // starting at x * (n / 8) + min(x, n % 8), so a row's units (its heads and splits) share one L2. A bijection on
  // [0, n): no padding workgroups and no early exit, so the argument loads below issue together.
  // The arguments of the prologue and the slot phase are read by an empty asm first: their scalar loads then issue
  // together behind one wait, instead of one round trip each where the compiler would place them next to their uses.
  asm volatile("" ::"s"(a.xcd_units), "s"(a.xcd_extra), "s"(a.splits), "s"(a.kv_groups), "s"(a.kv_heads),
               "s"(a.group), "s"(a.keys_per_split), "s"(a.topk), "s"(a.q), "s"(a.q_rs), "s"(a.q_hs), "s"(a.indices),
               "s"(a.idx_stride), "s"(a.counts), "s"(a.seq_lens), "s"(a.query_pos), "s"(a.row_req), "s"(a.table),
               "s"(a.table_stride), "s"(a.page_shift), "s"(a.page_size), "s"(a.pool_slots), "s"(a.idx_head_stride),
               "s"(a.block_shift), "s"(a.max_len), "s"(a.remap_shift), "s"(a.remap_mul));
  const uint32_t g = blockIdx.x;
  // per-wave timeline (diagnostics, off unless xt_decode_timeline set a buffer): the first lane of every wave writes
  // the 100 MHz constant clock at each phase; a branch uniform over the launch otherwise
  const bool timeline = a.stamps != nullptr && g < a.stamp_blocks;
  const uint64_t t_entry = timeline ? __builtin_amdgcn_s_memrealtime() : 0;
  const uint32_t xcd = g & 7u;
  const uint32_t u = xcd * a.xcd_units + min(xcd, a.xcd_extra) + (g >> 3);
  const uint32_t splits_u = (uint32_t)a.splits, groups_u = (uint32_t)a.kv_groups;
  const int split = (int)(u % splits_u);
  const int kvg = (int)((u / splits_u) % groups_u);
  const int row = (int)(u / splits_u / groups_u);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  uint64_t* const my_stamps = timeline ? a.stamps + ((uint64_t)g * W + wave) * kStamps : nullptr;
  auto stamp = [&](int phase) {
    if (timeline) {
      const uint64_t t = __builtin_amdgcn_s_memrealtime();
      if (lane == 0) my_stamps[phase] = t;
    }
  };
  if (timeline && lane == 0) {   // phases a wave does not reach stay 0
    my_stamps[kStEntry] = t_entry;
#pragma unroll
    for (int i = 1; i < kStamps; ++i) my_stamps[i] = 0;
  }
  const int kvh = kvg * HPW + kWaveHeads * (wave % kHeadSets);   // the wave's (first) KV head
  const int slice = wave / kHeadSets;
  const bool active = kvh < a.kv_heads;

  int32_t* slots = reinterpret_cast<int32_t*>(lds);
  uint8_t* vtile = lds + a.slot_lds_bytes + wave * G::kWaveLds;

  // the query's raw words first (loads complete in order); every lane reads a valid address and heads outside the
  // group are zeroed at conversion, so the loads carry no branch
  const int hl = lane & 15, j = lane >> 4;
  // column hl: a query head of the wave's KV head, or (paired waves) of KV head hl / 8 of its pair
  const int col_kvh = PR ? kvh + (hl >> 3) : kvh;
  const int col_qh = PR ? (hl & 7) : hl;
  const bool q_valid = col_kvh < a.kv_heads && col_qh < a.group;
  uint4 qraw[G::kNK];
  {
    const int head = min(col_kvh, a.kv_heads - 1) * a.group + min(col_qh, a.group - 1);
    const uint16_t* qp = a.q + (int64_t)row * a.q_rs + (int64_t)head * a.q_hs;
#pragma unroll
    for (int kk = 0; kk < G::kNK; ++kk) qraw[kk] = *reinterpret_cast<const uint4*>(qp + (D / 4) * j + 8 * kk);
  }

  // 1. the split's pool slots (-1: invalid key), shared by the workgroup's waves; each slice owns a whole number of
  // prefetch groups, padded with invalid keys that compute to no-ops (P = 0, V = 0, maximum unchanged). The first
  // kSlotBatch * kThreads index loads go out before the row's count, length and table row are read (they need only launch
  // constants), so the chain to the first K/V load is two dependent loads: index, then table.
  const int t0 = split * a.keys_per_split;
  const int kmax = max(0, min(a.keys_per_split, a.topk - t0));
  const int64_t irow = a.idx_rows ? uniform_load(a.idx_rows + row) : row;
  const int32_t* ip = a.indices + irow * a.idx_stride + (int64_t)kvg * a.idx_head_stride;
  const int bmask = (1 << a.block_shift) - 1;
  // Lanes whose key is past the split read a valid stand-in address (the row's length) instead of sitting in a
  // per-lane branch (its select would wait for the load right after it, serializing the batch); batches with no key
  // of the split issue no loads at all (a branch uniform over the workgroup). The loaded words stay raw until every
  // batch is issued.
  const int32_t* len_p = a.seq_lens + row;
  int32_t ev[kSlotBatch];
#pragma unroll
  for (int b = 0; b < kSlotBatch; ++b) {
    const int i = b * kThreads + (int)threadIdx.x, k = t0 + i;
    ev[b] = -1;
    if (b == 0 || b * kThreads < kmax) ev[b] = *((i < kmax) ? ip + (k >> a.block_shift) : len_p);
  }
  // the row's count, length, causal limit and table row, and the global scales: scalar loads from addresses valid
  // whether or not the optional arrays are given (a missing one reads the row's length and is ignored), so none waits
  // in a branch. The scales are read here, not next to their first use: a vector load issued after the K/V loads
  // would make the first softmax step wait for all of them.
  const int32_t* req_p = a.row_req ? reinterpret_cast<const int32_t*>(a.row_req + row) : len_p;
  int32_t len_v = uniform_load(len_p);
  int32_t cnt_v = uniform_load(a.counts ? a.counts + row : len_p);
  int32_t qpos_v = uniform_load(a.query_pos ? a.query_pos + row : len_p);
  int32_t req_lo = uniform_load(req_p), req_hi = uniform_load(a.row_req ? req_p + 1 : len_p);
  float gk_v = a.gk ? uniform_load_f32(a.gk) : a.gk_val;
  float gv_v = a.gv ? uniform_load_f32(a.gv) : a.gv_val;
  // every use below follows this asm, so the seven loads issue together behind one wait
  asm volatile("" : "+s"(len_v), "+s"(cnt_v), "+s"(qpos_v), "+s"(req_lo), "+s"(req_hi), "+s"(gk_v), "+s"(gv_v));
  const int count = a.counts ? min(cnt_v, a.topk) : a.topk;
  const int n = max(0, min(t0 + a.keys_per_split, count) - t0);
  const int slice_steps = (((n + KS - 1) / KS + kSlices * P - 1) / (kSlices * P)) * P;
  {
    const int32_t seqlen = min(len_v, a.max_len);
    const int32_t qpos = a.query_pos ? qpos_v : 0x7FFFFFFF;
    const int64_t trow = a.row_req ? (int64_t)(((uint64_t)(uint32_t)req_hi << 32) | (uint32_t)req_lo) : row;
    const int32_t* tp = a.table + trow * a.table_stride;
    const int total = kSlices * slice_steps * KS;
    int32_t pos[kSlotBatch];
#pragma unroll
    for (int b = 0; b < kSlotBatch; ++b) {
      const int i = b * kThreads + (int)threadIdx.x, k = t0 + i;
      const int32_t e = (i < kmax) ? ev[b] : -1;
      pos[b] = e < 0 ? -1 : (e << a.block_shift) + (k & bmask);
    }
    for (int i0 = 0;;) {
      // validity and table offsets of all kSlotBatch keys first, then their table loads back to back (a use of an
      // index between two table loads would wait for the earlier table load too)
      bool ok[kSlotBatch];
      int32_t toff[kSlotBatch], ent[kSlotBatch];
#pragma unroll
      for (int b = 0; b < kSlotBatch; ++b) {
        const int i = i0 + b * kThreads + (int)threadIdx.x;
        ok[b] = i < n && pos[b] >= 0 && pos[b] < seqlen && pos[b] <= qpos;
        const int32_t tpos = pos[b] & ~a.lookup_mask;   // block decode: a block's slots follow its first position's
        toff[b] = a.page_shift >= 0 ? (tpos >> a.page_shift) : tpos / a.page_size;
      }
#pragma unroll
      for (int b = 0; b < kSlotBatch; ++b) {   // (a lane with ok[b] false reads the stand-in; its entry is unused)
        ent[b] = -1;
        if (b == 0 || i0 + b * kThreads < n) ent[b] = *(ok[b] ? tp + toff[b] : len_p);
      }
#pragma unroll
      for (int b = 0; b < kSlotBatch; ++b) {
        const int i = i0 + b * kThreads + (int)threadIdx.x;
        int32_t slot = -1;
        if (ok[b] && ent[b] >= 0) {
          const int64_t sl = (int64_t)ent[b] * a.page_size + (pos[b] - toff[b] * a.page_size);
          const int64_t v = (sl >> a.remap_shift) * a.remap_mul + (sl & ((1 << a.remap_shift) - 1));
          if (v < a.pool_slots) slot = (int32_t)v;
        }
        if (i < total) slots[i] = slot;
      }
      i0 += kSlotBatch * kThreads;
      if (i0 >= total) break;
#pragma unroll
      for (int b = 0; b < kSlotBatch; ++b) {   // splits longer than kSlotBatch * kThreads keys
        const int i = i0 + b * kThreads + (int)threadIdx.x, k = t0 + i;
        const int32_t e0 = *((i < kmax) ? ip + (k >> a.block_shift) : len_p);
        const int32_t e = (i < kmax) ? e0 : -1;
        pos[b] = e < 0 ? -1 : (e << a.block_shift) + (k & bmask);
      }
    }
  }
  // With one wave per slice and 64-key slices (the batch decode's paired waves, the one-KV-head shapes), thread 64 w + l
  // wrote key 64 w + l, so every wave reads only the slots its own lanes wrote: LDS keeps a wave's accesses in order,
  // and the wave goes on to its first K/V loads without waiting for the other waves' table loads. (A condition
  // uniform over the workgroup.)
  if (kHeadSets == 1 && slice_steps * KS == 64) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  } else {
    __syncthreads();
  }
  stamp(kStSlots);

  SoftmaxState<D> st;
  st.m = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int t = 0; t < G::kNT; ++t)
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[t][i] = float4_t{0.f, 0.f, 0.f, 0.f};

  if (active && slice_steps > 0) {
    WaveCtx w;
    w.row_bytes = a.pay_stride;
    w.row_scales = a.sf_stride;
    w.kp = a.k_pay + (int64_t)kvh * a.pay_head_stride;
    w.vp = a.v_pay + (int64_t)kvh * a.pay_head_stride;
    w.ksf = a.k_sf + (int64_t)kvh * a.sf_head_stride;
    w.vsf = a.v_sf + (int64_t)kvh * a.sf_head_stride;
    w.kp2 = w.kp + a.pay_head_stride;
    w.vp2 = w.vp + a.pay_head_stride;
    w.ksf2 = w.ksf + a.sf_head_stride;
    w.vs_off = 4u * (uint32_t)(j & 1) + (uint32_t)(j >> 1) * (uint32_t)a.sf_head_stride;
    w.slots = slots + slice * slice_steps * KS;
    w.lane = lane;
    w.hl = hl;
    w.j = j;
    using StepT = typename std::conditional<PR, PairStep, Step<D>>::type;
    StepT buf[P];
    auto load = [&](int step, StepT& d) {
      if constexpr (PR) load_step_pair<O32>(w, step, d);
      else load_step<D, PS, O32>(w, step, d);
    };
#pragma unroll
    for (int p = 0; p < P; ++p) load(p, buf[p]);
    // the query's operands, prepared while the first steps' loads are in flight. B operand of the QK MFMAs: FP16 of
    // q * 2^-e, exact, with 2^e per head from its largest magnitude
    // (pow2_query_scale); heads beyond the group are zero. The FP32 scores are multiplied by smul = |gk| * scale *
    // log2(e) * 2^e, this lane's head's. A negative K global scale moves its sign into the query, and a magnitude below
    // FLT_MIN (zero included) is raised to it, so the softmax works with smul > 0 for a positive softmax scale (a NaN
    // stays NaN); at that size the scaled scores round to 0 either way.
    const float gk_abs = __builtin_fabsf(gk_v);
    const float gk = gk_abs < 1.17549435e-38f ? 1.17549435e-38f : gk_abs;
    float qmax = 0.0f;
#pragma unroll
    for (int kk = 0; kk < G::kNK; ++kk) {
      const uint32_t ws[4] = {qraw[kk].x, qraw[kk].y, qraw[kk].z, qraw[kk].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        qmax = fmaxf(qmax, fmaxf(__builtin_fabsf(bf16_bits_to_f32(ws[e] & 0xFFFFu)),
                                 __builtin_fabsf(bf16_bits_to_f32(ws[e] >> 16))));
    }
    const float2_t p2 = pow2_query_scale(max4_lanes16(qmax));   // the head's maximum over its four lanes
    const float qs = gk_v < 0.0f ? -p2[0] : p2[0];
    const float smul = gk * a.qscale * p2[1];
    // paired waves: MFMA kk < 4 contracts head 0's dims, kk >= 4 head 1's; a column's operand is zero in the other
    // head's dims (block-diagonal Q^T)
    constexpr int kQB = PR ? 2 * G::kNK : G::kNK;
    half8_t qb[kQB];
#pragma unroll
    for (int kk = 0; kk < G::kNK; ++kk) {
      const uint32_t ws[4] = {q_valid ? qraw[kk].x : 0u, q_valid ? qraw[kk].y : 0u, q_valid ? qraw[kk].z : 0u,
                              q_valid ? qraw[kk].w : 0u};
      half8_t h;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[2 * e] = (_Float16)(bf16_bits_to_f32(ws[e] & 0xFFFFu) * qs);
        h[2 * e + 1] = (_Float16)(bf16_bits_to_f32(ws[e] >> 16) * qs);
      }
      if constexpr (PR) {
        const half8_t zero = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        qb[kk] = hl < 8 ? h : zero;
        qb[(G::kNK + kk) % kQB] = hl < 8 ? zero : h;
      } else {
        qb[kk] = h;
      }
    }
    auto compute = [&](int step, const StepT& d) {
      if constexpr (PR) compute_step_pair(w, step, d, qb, smul, vtile, st);
      else compute_step<D, PS>(w, step, d, qb, smul, vtile, st);
      if (step == 0) stamp(kStStep0);
    };
    int s0 = 0;
    for (; s0 + P < slice_steps; s0 += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        compute(s0 + p, buf[p]);
        load(s0 + p + P, buf[p]);
      }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) compute(s0 + p, buf[p]);
  }
  stamp(kStLoop);
  // the 4 lanes of a head hold disjoint key subsets of l
  float l_tot = sum4_lanes16(st.l);

  // One slice per head and one key split (4 KV heads per 4-wave workgroup: prefill chunks): the wave's state is its
  // head's result; it normalizes and writes it from registers (acc[t][0..7][r] are dims 128 t + 32 j + 8 r .. + 7),
  // with no LDS merge, and the launch reserves no merge region.
  if constexpr (kSlices == 1) {
    if (a.splits == 1) {
      if (active && q_valid && (D != 64 || j < 2)) {
        const float inv = l_tot > 0.0f ? gv_v / l_tot : 0.0f;
        const int head = col_kvh * a.group + col_qh;
#pragma unroll
        for (int t = 0; t < G::kNT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = st.acc[t][i][r] * inv;
            store_out(a, row, head, 128 * t + 32 * j + 8 * r, v, 8);
          }
        if (a.lse && j == 0)
          a.lse[(int64_t)row * a.q_heads + head] =
              l_tot > 0.0f ? (st.m + __builtin_log2f(l_tot)) * kLn2 : -__builtin_inff();
      }
      stamp(kStPartials);
      return;
    }
  }

  // 2. the slices merge through LDS behind one barrier: every wave leaves its (O^T in dim order, max, sum) per lane
  // in its own region (after the slot list and V tiles, so no wave still reading those is disturbed); then each
  // thread merges 4 dims of one (KV head, lane) over the slices and normalizes (one split) or writes the partial
  float* mrg = reinterpret_cast<float*>(lds + a.slot_lds_bytes + W * G::kWaveLds);
  {
    float4_t* mine = reinterpret_cast<float4_t*>(mrg + (wave * 64 + lane) * G::kMergeRow);
#pragma unroll
    for (int t = 0; t < G::kNT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {   // dims 8 (16 t + 4 j + r) .. + 7
        mine[8 * t + 2 * r] = float4_t{st.acc[t][0][r], st.acc[t][1][r], st.acc[t][2][r], st.acc[t][3][r]};
        mine[8 * t + 2 * r + 1] = float4_t{st.acc[t][4][r], st.acc[t][5][r], st.acc[t][6][r], st.acc[t][7][r]};
      }
    mine[8 * G::kNT] = float4_t{st.m, l_tot, 0.0f, 0.0f};
  }
  __syncthreads();
  stamp(kStSliceMerge);
  uint8_t* row_part = reinterpret_cast<uint8_t*>(a.part) + (int64_t)row * a.splits * a.q_heads * G::kPartBytes;
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      row_part, (short)0, a.splits > 1 ? (int)((int64_t)a.splits * a.q_heads * G::kPartBytes) : 0, 0x00020000);
  const float gv = gv_v;
  constexpr int kParts = 8 * G::kNT;   // 4-dim pieces per lane
  constexpr int kUnits = (kHeadSets * 64 * kParts + kThreads - 1) / kThreads;   // pieces per thread
  // the KV head and query head of column uh of the wave head set hw (paired waves: head uh / 8 of the pair)
  auto unit_kvh = [&](int hw, int uh) { return kvg * HPW + kWaveHeads * hw + (PR ? (uh >> 3) : 0); };
  auto unit_qh = [&](int uh) { return PR ? (uh & 7) : uh; };
  // with key splits and at most two pieces per thread, each thread keeps its pieces' merged (output, max, sum) for
  // the split merge below (with more, the registers would spill: the merge reloads its own split too)
  constexpr bool kKeep = kUnits <= 2;
  float4_t keep_o[kUnits];
  float keep_m[kUnits], keep_l[kUnits];
#pragma unroll
  for (int k = 0; k < kUnits; ++k) {
    const int u = (int)threadIdx.x + k * kThreads;
    keep_m[k] = -__builtin_inff();
    keep_l[k] = 0.0f;
    keep_o[k] = float4_t{0.f, 0.f, 0.f, 0.f};
    if (u >= kHeadSets * 64 * kParts) continue;
    const int part = u % kParts, ln = (u / kParts) & 63, hw = u / (kParts * 64);   // piece part of lane ln, head set hw
    const int uh = ln & 15, uj = ln >> 4;
    const int ukvh = unit_kvh(hw, uh), uqh = unit_qh(uh);
    if (ukvh >= a.kv_heads || uqh >= a.group || (D == 64 && uj >= 2)) continue;
    float ms[kSlices], ls[kSlices];
    float4_t xs[kSlices];
    float mx = -__builtin_inff();
#pragma unroll
    for (int sl = 0; sl < kSlices; ++sl) {
      const float4_t* src =
          reinterpret_cast<const float4_t*>(mrg + ((sl * kHeadSets + hw) * 64 + ln) * G::kMergeRow);
      xs[sl] = src[part];
      const float4_t ml = src[8 * G::kNT];
      ms[sl] = ml[0];
      ls[sl] = ml[1];
      mx = fmaxf(mx, ms[sl]);
    }
    const float mu = (mx == -__builtin_inff()) ? 0.0f : mx;
    float4_t o = float4_t{0.f, 0.f, 0.f, 0.f};
    float l = 0.0f;
#pragma unroll
    for (int sl = 0; sl < kSlices; ++sl) {
      const float wgt = __builtin_amdgcn_exp2f(ms[sl] - mu);
      o += wgt * xs[sl];
      l += wgt * ls[sl];
    }
    const int head = ukvh * a.group + uqh, d0 = 128 * (part >> 3) + 32 * uj + 4 * (part & 7);
    if (a.splits == 1) {   // no partials: normalize and write
      const float inv = l > 0.0f ? gv / l : 0.0f;
      const float v[4] = {o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv};
      store_out(a, row, head, d0, v, 4);
      if (a.lse && d0 == 0)
        a.lse[(int64_t)row * a.q_heads + head] = l > 0.0f ? (mx + __builtin_log2f(l)) * kLn2 : -__builtin_inff();
    } else {               // 3. partials of this row, written through: the output normalized by the split's own
                           //    sum (a convex combination of e2m1 * e4m3 values, at most 2688 in magnitude) as FP16
      const int at = (split * a.q_heads + head) * G::kPartBytes;
      const float inv_l = l > 0.0f ? 1.0f / l : 0.0f;
      const float4_t on = o * inv_l;
      store_partial_h4(pr, at + d0 * 2, on);
      if (d0 == 0) store_partial(pr, at + 2 * D, float4_t{mx, l, 0.0f, 0.0f});
      if constexpr (kKeep) {   // rounded as the others' are read back, so the merge does not depend on who merges
        keep_m[k] = mx;
        keep_l[k] = l;
        const half2_t h0 = __builtin_convertvector(float2_t{on[0], on[1]}, half2_t);
        const half2_t h1 = __builtin_convertvector(float2_t{on[2], on[3]}, half2_t);
        keep_o[k] = float4_t{(float)h0[0], (float)h0[1], (float)h1[0], (float)h1[1]};
      }
    }
  }
  stamp(kStPartials);
  if (a.splits == 1) return;
  // the last workgroup of (row, KV group) to arrive merges the partials (the split arrival of xt_common.h): each
  // thread merges the same pieces it wrote, in split order whichever workgroup arrives last (so the result does not
  // depend on the order of arrival), its own split's from registers and the others' loaded, four splits at a time
  // with their loads issued together (its own split and splits past the last read nothing: an offset past the buffer
  // reads zeros)
  __shared__ int s_last;
  int32_t* counter = a.counters + (int64_t)row * a.kv_groups + kvg;
  const bool last = arrive_last(counter, a.splits, &s_last);
  stamp(kStArrived);
  if (!last) return;
  int heads_k[kUnits], d0s[kUnits];
  bool live_k[kUnits];
#pragma unroll
  for (int k = 0; k < kUnits; ++k) {
    const int u = (int)threadIdx.x + k * kThreads;
    const int part = u % kParts, ln = (u / kParts) & 63, hw = u / (kParts * 64);
    const int uh = ln & 15, uj = ln >> 4;
    const int ukvh = unit_kvh(hw, uh), uqh = unit_qh(uh);
    live_k[k] = u < kHeadSets * 64 * kParts && ukvh < a.kv_heads && uqh < a.group && !(D == 64 && uj >= 2);
    heads_k[k] = min(ukvh, a.kv_heads - 1) * a.group + min(uqh, a.group - 1);
    d0s[k] = 128 * (part >> 3) + 32 * uj + 4 * (part & 7);
  }
  // up to two pieces at a time: their loads of four splits (16 x 16 bytes) go out together
  constexpr int kBatch = kUnits < 2 ? kUnits : 2;
#pragma unroll
  for (int kb = 0; kb < kUnits; kb += kBatch) {
    float m_run[kBatch], l_run[kBatch];
    float4_t o[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      m_run[b] = -__builtin_inff();
      l_run[b] = 0.0f;
      o[b] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
    for (int s0 = 0; s0 < a.splits; s0 += 4) {
      float4_t ml[kBatch][4], x[kBatch][4];
#pragma unroll
      for (int b = 0; b < kBatch; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool other = live_k[kb + b] && s0 + i < a.splits && (!kKeep || s0 + i != split);
          const int at = other ? ((s0 + i) * a.q_heads + heads_k[kb + b]) * G::kPartBytes : 0x7FFF0000;
          ml[b][i] = load_partial(pr, at + 2 * D);
          x[b][i] = load_partial_h4(pr, at + d0s[kb + b] * 2);
        }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        float mc = m_run[b];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (kKeep && s0 + i == split) {
            ml[b][i][0] = keep_m[kb + b];
            ml[b][i][1] = keep_l[kb + b];
            x[b][i] = keep_o[kb + b];
          } else if (s0 + i >= a.splits) {
            ml[b][i][0] = -__builtin_inff();
          }
          mc = fmaxf(mc, ml[b][i][0]);
        }
        const float mu = (mc == -__builtin_inff()) ? 0.0f : mc;
        const float alpha = __builtin_amdgcn_exp2f(m_run[b] - mu);
        l_run[b] *= alpha;
        o[b] *= alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) {   // the partials are normalized: weight 2^(m - mu) * l
          const float wl = __builtin_amdgcn_exp2f(ml[b][i][0] - mu) * ml[b][i][1];
          l_run[b] += wl;
          o[b] += wl * x[b][i];
        }
        m_run[b] = mc;
      }
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int k = kb + b;
      if (!live_k[k]) continue;
      const float inv = l_run[b] > 0.0f ? gv / l_run[b] : 0.0f;
      const float v[4] = {o[b][0] * inv, o[b][1] * inv, o[b][2] * inv, o[b][3] * inv};
      store_out(a, row, heads_k[k], d0s[k], v, 4);
      if (a.lse && d0s[k] == 0)
        a.lse[(int64_t)row * a.q_heads + heads_k[k]] =
            l_run[b] > 0.0f ? (m_run[b] + __builtin_log2f(l_run[b])) * kLn2 : -__builtin_inff();
    }
  }
  reset_counter(counter);
  stamp(kStSplitMerge);
}

}  // namespace
}  // namespace xt

using namespace xt;

// KV heads per workgroup: 4 when that alone fills every CU, else 2 when that does, else 1 (more, smaller workgroups).
// A pair of heads reads each key's K and V payload pieces of both heads together (whole 128-byte lines on SGLang's
// split pool). Measured, batch 32 x 4 KV heads, top-2048: 2 heads x 4 splits 18.7 us (split pool 20.8 us) against
// 1 head x 2 splits 19.1 us (21.8 us).
static int heads_per_workgroup(int rows, int kv_heads, int splits, int cus) {
  if (kv_heads % 4 == 0 && (int64_t)rows * (kv_heads / 4) * splits >= cus) return 4;
  if (kv_heads % 2 == 0 && (int64_t)rows * (kv_heads / 2) * splits >= cus) return 2;
  return 1;
}

// Pool and index addressing beyond the token-major pool with one shared index list per row.
struct Addressing {
  int64_t pay_head_stride, sf_head_stride;   // bytes between KV heads of a slot row
  int remap_shift;                           // head-major pages: slot -> (slot >> shift) * mul + low bits
  int64_t remap_mul;
  int64_t idx_head_stride;                   // per-KV-head index lists (0: shared; forces 1 KV head per workgroup)
  int block_shift;                           // an index entry names 2^block_shift positions
  bool token_lookup;                         // resolve every position through the table (else the block start)
  const int32_t* idx_rows;                   // per-row index row (NULL: the row)
  int max_len;                               // sequence lengths clamped to this
  bool scalar_scales;                        // gk / gv NULL: the scores and outputs use gk_val / gv_val
  float gk_val, gv_val;
};

static int decode_impl(const char* what, const void* q, int64_t q_row_stride, int64_t q_head_stride,
                       const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales, const uint8_t* v_scales,
                       const float* gk, const float* gv, int64_t pool_slots, int64_t pay_stride, int64_t sf_stride,
                       int kv_heads, int q_heads, int dim, const int32_t* table, int64_t table_stride, int page_size,
                       const int64_t* row_req, const int32_t* indices, int64_t idx_stride, int topk,
                       const int32_t* counts, const int32_t* seq_lens, const int32_t* query_pos, float scale,
                       void* out, int64_t out_row_stride, int64_t out_head_stride, int out_dtype, float* lse, int rows,
                       int splits, void* workspace, size_t workspace_bytes, const Addressing& ad,
                       xt_stream_t stream);

// Workspace: [arrival counters, kCounterBytes][partials [rows, splits, q_heads, dim + 4] FP32]

// The per-wave timeline buffer of the decode launches (xt_decode_timeline); NULL: off.
static std::atomic<uint64_t*> g_timeline{nullptr};
static std::atomic<size_t> g_timeline_bytes{0};

extern "C" int xt_decode_timeline(uint64_t* stamps, size_t bytes) {
  if (stamps && (!aligned(stamps, 8) || bytes < 64))
    return fail(XT_EINVAL, "xt_decode_timeline: the stamp buffer must be 8-byte aligned and hold one wave's 8 stamps");
  g_timeline_bytes.store(stamps ? bytes : 0);
  g_timeline.store(stamps);
  return ok();
}

static bool supported_dim(int dim) { return dim == 64 || dim == 128 || dim == 256; }

extern "C" size_t xt_sparse_decode_workspace_bytes(int rows, int q_heads, int dim, int splits) {
  if (rows < 0 || q_heads <= 0 || dim <= 0 || splits <= 0) return 0;
  if (splits == 1) return 256;
  return kCounterBytes + (size_t)rows * splits * q_heads * (size_t)(dim + 4) * sizeof(float);
}

extern "C" int xt_sparse_decode_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                      const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                                      const uint8_t* v_scales, const float* gk, const float* gv, int64_t pool_slots,
                                      int64_t pay_stride, int64_t sf_stride, int64_t pay_head_stride,
                                      int64_t sf_head_stride, int kv_heads, int q_heads, int dim,
                                      const int32_t* table, int64_t table_stride,
                                      int page_size, const int64_t* row_req, const int32_t* indices,
                                      int64_t idx_stride, int topk, const int32_t* counts, const int32_t* seq_lens,
                                      const int32_t* query_pos, float scale, void* out, int64_t out_row_stride,
                                      int64_t out_head_stride, int out_dtype, float* lse, int rows, int splits,
                                      void* workspace, size_t workspace_bytes, xt_stream_t stream) {
  const char* what = "xt_sparse_decode_nvfp4";
  if (!supported_dim(dim)) return fail(XT_EUNSUPPORTED, "%s: head size %d (supported: 64, 128, 256)", what, dim);
  if (kv_heads <= 0) return fail(XT_EINVAL, "%s: kv_heads %d", what, kv_heads);
  if (pay_head_stride == 0) pay_head_stride = dim / 2;
  if (sf_head_stride == 0) sf_head_stride = dim / 16;
  if (pay_stride == 0) pay_stride = (int64_t)kv_heads * pay_head_stride;
  if (sf_stride == 0) sf_stride = (int64_t)kv_heads * sf_head_stride;
  if (pay_head_stride < dim / 2 || sf_head_stride < dim / 16 ||
      pay_stride < (int64_t)(kv_heads - 1) * pay_head_stride + dim / 2 ||
      sf_stride < (int64_t)(kv_heads - 1) * sf_head_stride + dim / 16)
    return fail(XT_EINVAL, "%s: slot strides %lld / %lld and head strides %lld / %lld bytes must hold the heads' "
                "payload / scales", what, (long long)pay_stride, (long long)sf_stride, (long long)pay_head_stride,
                (long long)sf_head_stride);
  if (pool_slots <= 0 || pool_slots > 0x7FFFFFFFLL)
    return fail(XT_EINVAL, "%s: pool_slots %lld outside 1..2^31-1", what, (long long)pool_slots);
  // positions past a table row's pitch are skipped keys, whatever the row's length says (no read past the row)
  const int max_len =
      table_stride > 0 ? (int)std::min<int64_t>(0x7FFFFFFF, table_stride * (int64_t)std::max(page_size, 1)) : 0x7FFFFFFF;
  const Addressing ad{pay_head_stride, sf_head_stride, 0, 1, 0, 0, true, nullptr, max_len, false, 0.0f, 0.0f};
  return decode_impl(what, q, q_row_stride, q_head_stride, k_pay, v_pay, k_scales, v_scales, gk, gv, pool_slots,
                     pay_stride, sf_stride, kv_heads, q_heads, dim, table, table_stride, page_size, row_req, indices,
                     idx_stride, topk, counts, seq_lens, query_pos, scale, out, out_row_stride, out_head_stride,
                     out_dtype, lse, rows, splits, workspace, workspace_bytes, ad, stream);
}

// --- the variant that allocates nothing ------------------------------------------------------------------------------
// Callers that cannot allocate device memory (work under graph capture, tight serving loops, harnesses that forbid
// hipMalloc) run the sparse decode with a workspace that is a fixed array of the library's own device memory: one
// `scratch` array per GPU, loaded with the code object and held until the process ends. The array's name is a host-side
// stand-in; its device address, looked up once per device, is what kernels receive.
constexpr size_t kScratchBytes = 8u << 20;   // arrival counters (64 KB) + split partials
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kScratchDevices = 64;
std::once_flag g_scratch_once[kScratchDevices];
void* g_scratch[kScratchDevices];             // device address of each GPU's array (NULL: lookup failed)
hipError_t g_scratch_error[kScratchDevices];

__global__ void zero_counters(uint32_t* p, int words) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x) p[i] = 0u;
}
}  // namespace

// The current device's scratch address. The first call on a device looks it up with that device current and zeroes
// the counter region with a kernel on `stream` (the decode kernels leave the counters zero after every call, and device
// globals start zeroed, so later calls need no clearing).
static int device_scratch(const char* what, hipStream_t stream, void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices)
    return fail(XT_ELAUNCH, "%s: no current device (or device index >= %d)", what, kScratchDevices);
  std::call_once(g_scratch_once[dev], [&] {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) {
      hipLaunchKernelGGL(zero_counters, dim3(16), dim3(256), 0, stream, static_cast<uint32_t*>(p),
                         (int)(kCounterBytes / 4));
      e = hipGetLastError();
    }
    g_scratch_error[dev] = e;
    g_scratch[dev] = e == hipSuccess ? p : nullptr;
  });
  if (!g_scratch[dev])
    return fail(XT_ELAUNCH, "%s: the device scratch array is not available on device %d: %s", what, dev,
                hipGetErrorString(g_scratch_error[dev]));
  *ptr = g_scratch[dev];
  return XT_OK;
}

extern "C" int xt_sparse_decode_nvfp4_static(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                             const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                                             const uint8_t* v_scales, const float* gk, const float* gv,
                                             int64_t pool_slots, int64_t pay_stride, int64_t sf_stride,
                                             int64_t pay_head_stride, int64_t sf_head_stride, int kv_heads,
                                             int q_heads, int dim, const int32_t* table, int64_t table_stride,
                                             int page_size, const int64_t* row_req, const int32_t* indices,
                                             int64_t idx_stride, int topk, const int32_t* counts,
                                             const int32_t* seq_lens, const int32_t* query_pos, float scale,
                                             void* out, int64_t out_row_stride, int64_t out_head_stride,
                                             int out_dtype, float* lse, int rows, int splits, xt_stream_t stream) {
  const char* what = "xt_sparse_decode_nvfp4_static";
  const size_t need = xt_sparse_decode_workspace_bytes(rows, q_heads, dim, splits);
  if (need > kScratchBytes)
    return fail(XT_EWORKSPACE, "%s: %d rows x %d heads x %d splits need %zu bytes of workspace, more than the %zu of "
                "the static array; use fewer splits or xt_sparse_decode_nvfp4 with a workspace", what, rows, q_heads,
                splits, need, kScratchBytes);
  void* ws = nullptr;
  if (int e = device_scratch(what, reinterpret_cast<hipStream_t>(stream), &ws)) return e;
  return xt_sparse_decode_nvfp4(q, q_row_stride, q_head_stride, k_pay, v_pay, k_scales, v_scales, gk, gv, pool_slots,
                                pay_stride, sf_stride, pay_head_stride, sf_head_stride, kv_heads, q_heads, dim, table,
                                table_stride, page_size, row_req, indices, idx_stride, topk, counts, seq_lens,
                                query_pos, scale, out, out_row_stride, out_head_stride, out_dtype, lse, rows, splits, ws,
                                kScratchBytes, stream);
}

// The head-major page checks shared by the block decode and the block prefill; fills the page-row remap.
static int block_pages(const char* what, int64_t pages, int kv_heads, int dim, int block_size, int64_t page_stride,
                       int64_t head_stride, int64_t row_stride, int64_t sf_page_stride, int64_t sf_head_stride,
                       int64_t sf_row_stride, int topk_blocks, int64_t* mul) {
  if (!supported_dim(dim)) return fail(XT_EUNSUPPORTED, "%s: head size %d (supported: 64, 128, 256)", what, dim);
  if (block_size <= 0 || (block_size & (block_size - 1)) || block_size > 4096)
    return fail(XT_EINVAL, "%s: block_size %d must be a power of 2 up to 4096", what, block_size);
  if (kv_heads <= 0 || pages <= 0 || topk_blocks < 0)
    return fail(XT_EINVAL, "%s: bad kv_heads / pages / topk", what);
  if (row_stride < dim / 2 || sf_row_stride < dim / 16 || row_stride % 16 || sf_row_stride % 4 || head_stride % 16 ||
      sf_head_stride % 4 || page_stride % row_stride || sf_page_stride % sf_row_stride ||
      page_stride / row_stride != sf_page_stride / sf_row_stride || page_stride / row_stride < block_size ||
      head_stride < (int64_t)block_size * row_stride - row_stride + dim / 2 ||
      sf_head_stride < (int64_t)block_size * sf_row_stride - sf_row_stride + dim / 16 ||
      page_stride < (int64_t)(kv_heads - 1) * head_stride + (int64_t)block_size * row_stride)
    return fail(XT_EINVAL, "%s: pool strides (page %lld, head %lld, row %lld; scales %lld, %lld, %lld bytes) do not "
                "describe [pages, kv_heads, %d, dim/2] / [.., dim/16] pages", what, (long long)page_stride,
                (long long)head_stride, (long long)row_stride, (long long)sf_page_stride, (long long)sf_head_stride,
                (long long)sf_row_stride, block_size);
  *mul = page_stride / row_stride;
  if (pages > 0x7FFFFFFFLL / *mul)
    return fail(XT_EUNSUPPORTED, "%s: %lld pages exceed 2^31 rows", what, (long long)pages);
  if ((int64_t)topk_blocks * block_size > 0x7FFFFFFFLL)
    return fail(XT_EUNSUPPORTED, "%s: %d blocks of %d keys", what, topk_blocks, block_size);
  return XT_OK;
}

extern "C" int xt_block_sparse_decode_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                            const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                                            const uint8_t* v_scales, float kv_scale, int64_t pages,
                                            int kv_heads, int q_heads, int dim, int block_size, int64_t page_stride,
                                            int64_t head_stride, int64_t row_stride, int64_t sf_page_stride,
                                            int64_t sf_head_stride, int64_t sf_row_stride,
                                            const int32_t* req_to_token, int64_t req_stride, int max_kv_len,
                                            const int64_t* slot_ids, const int32_t* topk_idx,
                                            int64_t idx_head_stride, int64_t idx_row_stride, int topk_blocks,
                                            const int32_t* seq_lens, float sm_scale, void* out,
                                            int64_t out_row_stride, int64_t out_head_stride, int out_dtype,
                                            float* lse, int rows, int splits, void* workspace,
                                            size_t workspace_bytes, xt_stream_t stream) {
  const char* what = "xt_block_sparse_decode_nvfp4";
  int64_t mul;
  const int st = block_pages(what, pages, kv_heads, dim, block_size, page_stride, head_stride, row_stride,
                             sf_page_stride, sf_head_stride, sf_row_stride, topk_blocks, &mul);
  if (st != XT_OK) return st;
  if (max_kv_len < 0) return fail(XT_EINVAL, "%s: max_kv_len %d", what, max_kv_len);
  if (!slot_ids) return fail(XT_EINVAL, "%s: slot_ids is null", what);
  const int shift = __builtin_ctz((unsigned)block_size);
  const Addressing ad{head_stride, sf_head_stride, shift, mul, idx_head_stride, shift, false, nullptr, max_kv_len, true,
                      kv_scale, kv_scale};
  return decode_impl(what, q, q_row_stride, q_head_stride, k_pay, v_pay, k_scales, v_scales, nullptr, nullptr,
                     pages * mul, row_stride, sf_row_stride, kv_heads, q_heads, dim, req_to_token, req_stride, 1,
                     slot_ids, topk_idx, idx_row_stride, topk_blocks * block_size, nullptr, seq_lens, nullptr,
                     sm_scale, out, out_row_stride, out_head_stride, out_dtype, lse, rows, splits, workspace,
                     workspace_bytes, ad, stream);
}

extern "C" int xt_block_sparse_prefill_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                             const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                                             const uint8_t* v_scales, float kv_scale, int64_t pages,
                                             int kv_heads, int q_heads, int dim, int block_size, int64_t page_stride,
                                             int64_t head_stride, int64_t row_stride, int64_t sf_page_stride,
                                             int64_t sf_head_stride, int64_t sf_row_stride,
                                             const int32_t* req_to_token, int64_t req_stride,
                                             const int64_t* row_req, const int32_t* row_seq_lens,
                                             const int32_t* row_query_pos, const int32_t* topk_idx,
                                             int64_t idx_head_stride, int64_t idx_row_stride, int topk_blocks,
                                             const int32_t* row_idx, float sm_scale, void* out,
                                             int64_t out_row_stride, int64_t out_head_stride, int out_dtype,
                                             float* lse, int rows, int splits, void* workspace,
                                             size_t workspace_bytes, xt_stream_t stream) {
  const char* what = "xt_block_sparse_prefill_nvfp4";
  int64_t mul;
  const int st = block_pages(what, pages, kv_heads, dim, block_size, page_stride, head_stride, row_stride,
                             sf_page_stride, sf_head_stride, sf_row_stride, topk_blocks, &mul);
  if (st != XT_OK) return st;
  if (!row_req || !row_query_pos || !row_idx) return fail(XT_EINVAL, "%s: a per-row array is null", what);
  const int shift = __builtin_ctz((unsigned)block_size);
  const Addressing ad{head_stride, sf_head_stride, shift, mul, idx_head_stride, shift, true, row_idx, 0x7FFFFFFF, true,
                      kv_scale, kv_scale};
  return decode_impl(what, q, q_row_stride, q_head_stride, k_pay, v_pay, k_scales, v_scales, nullptr, nullptr,
                     pages * mul, row_stride, sf_row_stride, kv_heads, q_heads, dim, req_to_token, req_stride, 1,
                     row_req, topk_idx, idx_row_stride, topk_blocks * block_size, nullptr, row_seq_lens,
                     row_query_pos, sm_scale, out, out_row_stride, out_head_stride, out_dtype, lse, rows, splits,
                     workspace, workspace_bytes, ad, stream);
}

// One launch of the decode kernel.
template <int D, int HPW, bool PS, int W, bool O32, bool PR>
static int launch_decode(const DecodeArgs& a, dim3 grid, size_t lds_bytes, hipStream_t stream, const char* what) {
  constexpr int P = Geo<D>::kPrefetch;
  if (int e = allow_lds(reinterpret_cast<const void*>(&decode_split_kernel<D, P, HPW, PS, W, O32, PR>), lds_bytes,
                        what))
    return e;
  hipLaunchKernelGGL((decode_split_kernel<D, P, HPW, PS, W, O32, PR>), grid, dim3(64 * W), lds_bytes, stream, a);
  return check_launch(what);
}

template <int D, int HPW, bool PS, int W, bool PR = false>
static int launch_decode(bool o32, const DecodeArgs& a, dim3 grid, size_t lds_bytes, hipStream_t stream,
                         const char* what) {
  return o32 ? launch_decode<D, HPW, PS, W, true, PR>(a, grid, lds_bytes, stream, what)
             : launch_decode<D, HPW, PS, W, false, PR>(a, grid, lds_bytes, stream, what);
}

template <int D, int W>
static int launch_decode(int hpw, bool ps, bool pr, bool o32, const DecodeArgs& a, dim3 grid, size_t lds_bytes,
                         hipStream_t stream, const char* what) {
  if constexpr (D == 128 && W == kWaves) {   // paired waves: 2 KV heads per workgroup, 8 key slices
    if (pr) return launch_decode<D, 2, false, W, true>(o32, a, grid, lds_bytes, stream, what);
  }
  if constexpr (D == 128) {   // paired K/V scales: the interleaved pool at head size 128
    if (ps) return hpw == 4   ? launch_decode<D, 4, true, W>(o32, a, grid, lds_bytes, stream, what)
                   : hpw == 2 ? launch_decode<D, 2, true, W>(o32, a, grid, lds_bytes, stream, what)
                              : launch_decode<D, 1, true, W>(o32, a, grid, lds_bytes, stream, what);
  }
  return hpw == 4   ? launch_decode<D, 4, false, W>(o32, a, grid, lds_bytes, stream, what)
         : hpw == 2 ? launch_decode<D, 2, false, W>(o32, a, grid, lds_bytes, stream, what)
                    : launch_decode<D, 1, false, W>(o32, a, grid, lds_bytes, stream, what);
}

// LDS bytes of a launch: the slot list, one V tile per wave and, unless each head has one slice and one split (the
// waves then write their heads' outputs from registers), one merge region per wave.
template <int D>
static size_t decode_lds(int slot_bytes, int waves, bool direct) {
  return (size_t)slot_bytes + (size_t)waves * Geo<D>::kWaveLds +
         (direct ? 0 : waves == 4 ? Geo<D>::template kMergeLds<4> : Geo<D>::template kMergeLds<kWaves>);
}

static int prefetch_of(int dim) { return dim == 64 ? Geo<64>::kPrefetch : dim == 128 ? Geo<128>::kPrefetch
                                                                                     : Geo<256>::kPrefetch; }

static int decode_impl(const char* what, const void* q, int64_t q_row_stride, int64_t q_head_stride,
                       const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales, const uint8_t* v_scales,
                       const float* gk, const float* gv, int64_t pool_slots, int64_t pay_stride, int64_t sf_stride,
                       int kv_heads, int q_heads, int dim, const int32_t* table, int64_t table_stride, int page_size,
                       const int64_t* row_req, const int32_t* indices, int64_t idx_stride, int topk,
                       const int32_t* counts, const int32_t* seq_lens, const int32_t* query_pos, float scale,
                       void* out, int64_t out_row_stride, int64_t out_head_stride, int out_dtype, float* lse, int rows,
                       int splits, void* workspace, size_t workspace_bytes, const Addressing& ad,
                       xt_stream_t stream) {
  if (kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads != 0)
    return fail(XT_EINVAL, "%s: q_heads %d must be a positive multiple of kv_heads %d", what, q_heads, kv_heads);
  const int group = q_heads / kv_heads;
  if (group > 16) return fail(XT_EUNSUPPORTED, "%s: GQA group %d (supported: <= 16)", what, group);
  if (rows < 0 || topk < 0 || page_size <= 0) return fail(XT_EINVAL, "%s: bad rows/topk/page_size", what);
  if (splits < 1 || splits > 64) return fail(XT_EINVAL, "%s: splits %d outside 1..64", what, splits);
  if (out_dtype != XT_DTYPE_BF16 && out_dtype != XT_DTYPE_F16)
    return fail(XT_EINVAL, "%s: output dtype must be BF16 or FP16", what);
  if (rows == 0) return ok();
  if (!q || !k_pay || !v_pay || !k_scales || !v_scales || ((!gk || !gv) && !ad.scalar_scales) || !table || !indices ||
      !seq_lens || !out ||
      !workspace)
    return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (!aligned(q, 16) || q_row_stride % 8 || q_head_stride % 8 || !aligned(out, 16) || out_row_stride % 8 ||
      out_head_stride % 8)
    return fail(XT_EINVAL, "%s: q and out rows must be 16-byte aligned (strides in elements: multiples of 8)", what);
  if (pay_stride % 16 || sf_stride % 4 || ad.pay_head_stride % 16 || ad.sf_head_stride % 4)
    return fail(XT_EINVAL, "%s: payload / scale strides must be multiples of 16 / 4 bytes", what);
  if (!aligned(k_pay, 16) || !aligned(v_pay, 16) || !aligned(k_scales, 4) || !aligned(v_scales, 4))
    return fail(XT_EINVAL, "%s: payload must be 16-byte and scales 4-byte aligned", what);
  if (lse && !aligned(lse, 4)) return fail(XT_EINVAL, "%s: lse must be 4-byte aligned", what);
  if (splits > 1 && (int64_t)rows * kv_heads > kCounterSlots)
    return fail(XT_EUNSUPPORTED, "%s: %d rows x %d KV heads with key splits exceed %d arrival counters; use splits 1",
                what, rows, kv_heads, kCounterSlots);
  const size_t need = xt_sparse_decode_workspace_bytes(rows, q_heads, dim, splits);
  if (workspace_bytes < need)
    return fail(XT_EWORKSPACE, "%s: workspace %zu bytes < %zu needed", what, workspace_bytes, need);
  if (!aligned(workspace, 256)) return fail(XT_EINVAL, "%s: workspace must be 256-byte aligned", what);
  const int per_split = (topk + splits - 1) / splits;
  const int kps = ((per_split + kStep - 1) / kStep) * kStep;
  const int cus = device_cus();
  const int hpw = ad.idx_head_stride ? 1 : heads_per_workgroup(rows, kv_heads, splits, cus);
  // Waves per workgroup: 8 when the units fit one round of workgroups, one per CU (decode batches), else 4 (prefill
  // chunks, one row per query; odd batch sizes): two 4-wave workgroups then share a CU, and one's slot list and merge
  // overlap the other's gather, where 8-wave ones would run a second round after the first.
  // Head size 256 always runs 4-wave workgroups: eight waves' merge regions would not fit in LDS.
  const int64_t units = (int64_t)rows * ((kv_heads + hpw - 1) / hpw) * splits;
  const int waves = (units > cus || dim == 256) ? 4 : kWaves;
  // Paired waves (each wave both KV heads of a pair, steps of 16 keys) for workgroups of 2 KV heads at head size 128
  // and GQA groups up to 8 with one index list for all heads: a key's payload of the pair is one contiguous run per
  // wave instead of one piece per wave and head.
  // (Prefill chunks keep one wave per KV head: the paired waves' second query operand costs 16 registers, which
  // spills at their three waves per SIMD; at two waves per SIMD the batch-4096 chunk measured 664 against 598 us.)
  const bool pr = dim == 128 && group <= 8 && !ad.idx_head_stride && hpw == 2 && waves == kWaves;
  const int slices = pr ? waves : waves / hpw;
  const int step_keys = pr ? kPairStep : kStep;
  const int pf = prefetch_of(dim);
  const int slice_steps = ((kps / step_keys + slices * pf - 1) / (slices * pf)) * pf;
  const int slot_bytes = slices * slice_steps * step_keys * (int)sizeof(int32_t);
  const bool direct = slices == 1 && splits == 1;
  const size_t lds_bytes = dim == 64    ? decode_lds<64>(slot_bytes, waves, direct)
                           : dim == 128 ? decode_lds<128>(slot_bytes, waves, direct)
                                        : decode_lds<256>(slot_bytes, waves, direct);
  if (lds_bytes > kMaxLds)
    return fail(XT_EUNSUPPORTED, "%s: %d keys per split needs %zu bytes of LDS; use more splits", what, kps,
                lds_bytes);

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_rs = q_row_stride;
  a.q_hs = q_head_stride;
  a.k_pay = k_pay;
  a.v_pay = v_pay;
  a.k_sf = k_scales;
  a.v_sf = v_scales;
  a.gk = ad.scalar_scales ? nullptr : gk;
  a.gv = ad.scalar_scales ? nullptr : gv;
  a.gk_val = ad.gk_val;
  a.gv_val = ad.gv_val;
  a.pool_slots = pool_slots;
  a.pay_stride = pay_stride;
  a.sf_stride = sf_stride;
  a.pay_head_stride = ad.pay_head_stride;
  a.sf_head_stride = ad.sf_head_stride;
  a.remap_shift = ad.remap_shift;
  a.remap_mul = ad.remap_mul;
  a.idx_head_stride = ad.idx_head_stride;
  a.block_shift = ad.block_shift;
  a.lookup_mask = ad.token_lookup ? 0 : (1 << ad.block_shift) - 1;
  a.idx_rows = ad.idx_rows;
  a.max_len = ad.max_len;
  a.kv_heads = kv_heads;
  a.q_heads = q_heads;
  a.group = group;
  a.kv_groups = (kv_heads + hpw - 1) / hpw;
  a.table = table;
  a.table_stride = table_stride;
  a.page_size = page_size;
  a.page_shift = (page_size & (page_size - 1)) == 0 ? __builtin_ctz((unsigned)page_size) : -1;
  a.row_req = row_req;
  a.indices = indices;
  a.idx_stride = idx_stride;
  a.topk = topk;
  a.counts = counts;
  a.seq_lens = seq_lens;
  a.query_pos = query_pos;
  a.qscale = scale * kLog2e;
  a.rows = rows;
  a.splits = splits;
  a.keys_per_split = kps;
  a.slot_lds_bytes = slot_bytes;
  a.out = static_cast<uint16_t*>(out);
  a.o_rs = out_row_stride;
  a.o_hs = out_head_stride;
  a.out_dtype = out_dtype;
  a.lse = lse;
  a.counters = static_cast<int32_t*>(workspace);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  a.n_units = (int64_t)rows * a.kv_groups * splits;
  a.xcd_units = (uint32_t)(a.n_units / 8);
  a.xcd_extra = (uint32_t)(a.n_units % 8);
  a.stamps = g_timeline.load();
  a.stamp_blocks = a.stamps ? (uint32_t)std::min<int64_t>(a.n_units, (int64_t)(g_timeline_bytes.load() / ((size_t)waves * 64)))
                            : 0u;
  const int64_t launched = a.n_units;
  if (launched > 0x7FFFFFFFLL) return fail(XT_EUNSUPPORTED, "%s: %lld workgroups", what, (long long)launched);

  // K and V scales of a head side by side and 8-byte aligned (head size 128): one load per key serves both
  const bool ps = dim == 128 && v_scales == k_scales + dim / 16 && aligned(k_scales, 8) && sf_stride % 8 == 0 &&
                  ad.sf_head_stride % 8 == 0;
  // 32-bit row offsets: slots below 2^24 (one 24-bit multiply) and every slot's row, plus the lane offsets within it,
  // below 2^32 bytes from the head's column
  const bool o32 = pool_slots <= (1LL << 24) && pay_stride < (1LL << 24) && sf_stride < (1LL << 24) &&
                   (pool_slots - 1) * pay_stride + dim / 2 < (1LL << 32) &&
                   (pool_slots - 1) * sf_stride + dim / 16 < (1LL << 32) &&
                   (!pr || (pool_slots - 1) * sf_stride + ad.sf_head_stride + dim / 16 < (1LL << 32));
  const dim3 grid((unsigned)launched);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dim == 64)
    return waves == 4 ? launch_decode<64, 4>(hpw, ps, false, o32, a, grid, lds_bytes, st, what)
                      : launch_decode<64, kWaves>(hpw, ps, false, o32, a, grid, lds_bytes, st, what);
  if (dim == 256) return launch_decode<256, 4>(hpw, ps, false, o32, a, grid, lds_bytes, st, what);
  return waves == 4 ? launch_decode<128, 4>(hpw, ps, false, o32, a, grid, lds_bytes, st, what)
                    : launch_decode<128, kWaves>(hpw, ps, pr, o32, a, grid, lds_bytes, st, what);
}
