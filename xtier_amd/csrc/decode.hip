// Fused sparse GQA attention over the NVFP4 paged pool: gather through the page table, dequantize in registers, QK
// and PV on MFMA (v_mfma_f32_16x16x32_f16), online softmax in the exp2 domain, in one launch: each workgroup writes one
// partial result per (row, key split, head), and the last workgroup of a row to finish merges the row's partials.
//
// Work decomposition: a workgroup = 8 wavefronts = 4 consecutive KV heads x 2 key halves of one (query row, key
// split); each wave owns one (row, KV head, split, half) and walks its keys in steps of 32. The workgroup computes the
// split's pool slots once into LDS, and merges the two halves of each head through LDS before writing the partial.
// Workgroups are numbered so that all splits of a row run on the same XCD (round-robin dispatch puts workgroup g on
// XCD g % 8): their K/V pages and partials share one L2.
//
// Memory pipeline: per step a wave issues 6 loads (K and V payload as 16-byte row pieces, K and V scales as one dword
// per lane) and keeps P steps in flight in a register ring. V is transposed for the PV operand through a padded LDS
// tile; the K scales reach their lanes with one ds_bpermute per 16-key tile.
//
// Numerics: e2m1 * e4m3 is exact in FP16 (at most 6 significant bits, magnitudes 2^-10 .. 2688), so K and V enter
// the MFMA exactly without their global scales; the query enters as FP16 of q * scale * log2(e); the K global scale
// multiplies the FP32 scores and the V global scale the merged output. P is FP16 for the PV product, sums are FP32.
// The running maximum is raised only when a score exceeds it by more than 2^8 (lazy rescale), so P <= 256.
//
// Lane layouts (16x16x32 MFMA: A[i][k] = lane i + 16*(k/8), element k%8; B[k][j] = lane j + 16*(k/8), element k%8;
// C[i][j] = lane j + 16*(i/4), element i%4). With hl = lane % 16 and j = lane / 16:
//   QK: C = S^T [16 keys x 16 heads]; A = K tile, lane (key hl, payload bytes 16j .. 16j+15 of the head row); MFMA kk
//       (0..3) contracts dword kk of those 16 bytes, d = 32j + 8kk + e; B = Q^T in the same d order. Lane (hl, j)
//       ends up with the scores of head hl for keys T(j) = {4j..4j+3, 16+4j..16+4j+3} of the step.
//   PV: C = O^T [16 rows x 16 heads], row c = payload dword c of the head row; MFMA i (0..7) takes nibble i of every
//       dword, d = 8c + i. A = V^T, lane (dword hl, keys T(j)); B = P^T, lane (head hl, keys T(j)) in the same order.
//       Lane (hl, j) ends up with O^T of head hl for d = 32j .. 32j+31.
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

constexpr int kDim = 128;          // head size: 64 payload bytes, 8 scale bytes per head row
constexpr int kStep = 32;          // keys per step
constexpr int kHeadsPerGroup = 4;  // KV heads per workgroup
constexpr int kHalves = 2;         // key halves per workgroup
constexpr int kWaves = kHeadsPerGroup * kHalves;
constexpr int kVRow = 80;          // LDS bytes per key in the V transpose tile (64 + 16: no bank conflicts)
constexpr int kWaveLds = kStep * kVRow + kStep * 8;   // V tile + V scale tile per wave
constexpr int kPrefetch = 4;       // steps of loads in flight per wave
constexpr float kRescale = 8.0f;   // log2 of the largest P before the running maximum is raised
constexpr int kPartStride = kDim + 4;   // floats per partial (split, head): 128 accumulators, max, sum, 2 pad
constexpr int kMergeLds = kHeadsPerGroup * 64 * 36 * 4;   // a half's (acc, max, sum) per lane for 4 waves

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_rs, q_hs;
  const uint8_t* k_pay;
  const uint8_t* v_pay;
  const uint8_t* k_sf;
  const uint8_t* v_sf;
  const float* gk;
  const float* gv;
  int64_t pool_slots;
  int64_t pay_stride, sf_stride;     // bytes from one slot to the next in the payload / scale buffers
  int kv_heads, q_heads, group, kv_groups;
  const int32_t* table;
  int64_t table_stride;
  int page_size;
  const int64_t* row_req;
  const int32_t* indices;
  int64_t idx_stride;
  int topk;
  const int32_t* counts;
  const int32_t* seq_lens;
  const int32_t* query_pos;
  float qscale;                      // softmax scale * log2(e)
  int rows, splits, keys_per_split;  // keys_per_split: a multiple of kStep
  int slot_lds_bytes;                // LDS bytes of the slot list (padded to whole prefetch groups per half)
  uint16_t* out;
  int64_t o_rs, o_hs;
  int out_dtype;
  float* lse;
  float* part;                       // [rows, splits, q_heads, kPartStride]: accumulators, max (log2), sum
  int32_t* counters;                 // [rows * kv_groups] arrivals per (row, KV group); zero between launches
  int64_t n_units;                   // rows * kv_groups * splits workgroups
  int64_t per_xcd;                   // launched workgroups / 8
  int xcd_map;                       // 1: number units XCD-major (rows >= 8), 0: unit = workgroup
};

struct Step {
  uint4 kw[2];   // K payload bytes 16j..16j+15 of key 16*tt + hl
  uint4 vw[2];   // V payload, same keys and bytes
  uint32_t ks;   // K scale bytes 4*(lane&1) .. +3 of key lane/2
  uint32_t vs;   // V scale bytes, same
};

__device__ inline int key_of(int j, int e) { return (e < 4) ? (4 * j + e) : (16 + 4 * j + (e - 4)); }

__device__ inline half8_t dequant_k(uint32_t w, half2_t sc) {
  const half2_t p0 = fp4x2_to_f16<0>(w) * sc;
  const half2_t p1 = fp4x2_to_f16<1>(w) * sc;
  const half2_t p2 = fp4x2_to_f16<2>(w) * sc;
  const half2_t p3 = fp4x2_to_f16<3>(w) * sc;
  return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

struct WaveCtx {
  const uint8_t* kp;    // this head's payload column
  const uint8_t* vp;
  const uint8_t* ksf;   // this head's scale column
  const uint8_t* vsf;
  int64_t row_bytes, row_scales;
  const int32_t* slots;  // this wave's slot list in LDS (-1: invalid)
  int lane, hl, j;
};

__device__ inline void load_step(const WaveCtx& w, int step, Step& d) {
  const int base = step * kStep;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int32_t s = w.slots[base + 16 * tt + w.hl];
    const int64_t slot = s < 0 ? 0 : s;
    d.kw[tt] = *reinterpret_cast<const uint4*>(w.kp + slot * w.row_bytes + 16 * w.j);
    d.vw[tt] = *reinterpret_cast<const uint4*>(w.vp + slot * w.row_bytes + 16 * w.j);
  }
  const int32_t s = w.slots[base + (w.lane >> 1)];
  const int64_t slot = s < 0 ? 0 : s;
  d.ks = *reinterpret_cast<const uint32_t*>(w.ksf + slot * w.row_scales + 4 * (w.lane & 1));
  d.vs = *reinterpret_cast<const uint32_t*>(w.vsf + slot * w.row_scales + 4 * (w.lane & 1));
}

struct SoftmaxState {
  float m;            // reference maximum of head hl (log2 domain), identical on the 4 lanes of the head
  float l;            // this lane's share of the sum of 2^(s - m)
  float4_t acc[8];    // O^T of head hl, d = 32j + 8r + i in acc[i][r]
};

__device__ inline void compute_step(const WaveCtx& w, int step, const Step& d, const half8_t (&qb)[4], float gk,
                                    uint8_t* vtile, SoftmaxState& st) {
  const int lane = w.lane, hl = w.hl, j = w.j;
  // validity of the step's 32 keys (bit t: key t), uniform over the wave
  const uint32_t valid =
      (uint32_t)__builtin_amdgcn_ballot_w64(lane < kStep && w.slots[step * kStep + (lane & 31)] >= 0);
  const bool my_scale_valid = (valid >> (lane >> 1)) & 1u;
  const uint32_t ks = d.ks;
  const uint32_t vs = my_scale_valid ? d.vs : 0u;   // invalid keys: V scale 0, so V = 0 whatever slot 0 holds

  // V: stage payload and scales in LDS, transposed reads below
  uint8_t* vscale = vtile + kStep * kVRow;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
    *reinterpret_cast<uint4*>(vtile + (16 * tt + hl) * kVRow + 16 * j) = d.vw[tt];
  *reinterpret_cast<uint32_t*>(vscale + (lane >> 1) * 8 + 4 * (lane & 1)) = vs;

  // QK
  float4_t s[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const uint32_t src = (uint32_t)__shfl((int)ks, 2 * (16 * tt + hl) + (j >> 1));
    const half2_t sc2 = fp8x2_to_f16<false>(src >> (16 * (j & 1)));
    const half2_t sc_lo = half2_t{sc2.x, sc2.x}, sc_hi = half2_t{sc2.y, sc2.y};
    const uint32_t kw[4] = {d.kw[tt].x, d.kw[tt].y, d.kw[tt].z, d.kw[tt].w};
    s[tt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(dequant_k(kw[kk], kk < 2 ? sc_lo : sc_hi), qb[kk], s[tt], 0, 0,
                                                     0);
  }
  // online softmax of head hl over keys T(j), lazy rescale
  float sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = s[e >> 2][e & 3] * gk;
    sv[e] = ((valid >> key_of(j, e)) & 1u) ? x : -__builtin_inff();
  }
  float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
  mt = fmaxf(mt, __shfl_xor(mt, 16));
  mt = fmaxf(mt, __shfl_xor(mt, 32));
  if (__builtin_amdgcn_ballot_w64(mt > st.m + kRescale)) {   // rare after the first steps
    const float m_new = (mt > st.m + kRescale) ? mt : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] *= alpha;
    st.m = m_new;
  }
  const float m_use = (st.m == -__builtin_inff()) ? 0.0f : st.m;
  float p[8];
  float psum = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = __builtin_amdgcn_exp2f(sv[e] - m_use);
    psum += p[e];
  }
  st.l += psum;
  const half8_t pb = half8_t{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
                             (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
  // V^T operands: dword hl of keys T(j), and the scale byte of block hl/2 of those keys
  asm volatile("" ::: "memory");
  uint32_t vw[8], vb[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int key = key_of(j, e);
    vw[e] = *reinterpret_cast<const uint32_t*>(vtile + key * kVRow + 4 * hl);
    vb[e] = vscale[key * 8 + (hl >> 1)];
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
  for (int i = 0; i < 8; ++i) st.acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], pb, st.acc[i], 0, 0, 0);
}

// A partial's 16-byte piece, written through to memory (sc1): visible to the merging workgroup on any XCD, whose plain
// loads cannot hit a stale copy (no workgroup reads these addresses before the merge within a launch).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ inline void store_through(__amdgpu_buffer_rsrc_t r, int byte_off, float4_t v) {
  const u32x4_t w = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  __builtin_amdgcn_raw_buffer_store_b128(w, r, byte_off, 0, 16);
}

__device__ inline void store_out(const DecodeArgs& a, int row, int head, int d0, const float* v, int n) {
  uint16_t* o = a.out + (int64_t)row * a.o_rs + (int64_t)head * a.o_hs + d0;
  for (int e = 0; e < n; e += 2) {
    uint32_t packed;
    if (a.out_dtype == XT_DTYPE_BF16)
      packed = f32_to_bf16_bits(v[e]) | (f32_to_bf16_bits(v[e + 1]) << 16);
    else
      packed = f32_to_f16_bits(v[e]) | (f32_to_f16_bits(v[e + 1]) << 16);
    *reinterpret_cast<uint32_t*>(o + e) = packed;
  }
}

template <int P>
__global__ void __launch_bounds__(512) decode_split_kernel(const DecodeArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  // XCD-aware numbering: launched workgroup g runs on XCD g % 8; unit u = (g % 8) * per_xcd + g / 8 keeps a row's
  // consecutive units (its splits) on one XCD.
  const int64_t g = blockIdx.x;
  const int64_t u = a.xcd_map ? (g % 8) * a.per_xcd + g / 8 : g;
  if (u >= a.n_units) return;   // uniform over the workgroup
  const int split = (int)(u % a.splits);
  const int kvg = (int)((u / a.splits) % a.kv_groups);
  const int row = (int)(u / ((int64_t)a.splits * a.kv_groups));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kvh = kvg * kHeadsPerGroup + (wave & (kHeadsPerGroup - 1));
  const int half = wave / kHeadsPerGroup;
  const bool active = kvh < a.kv_heads;

  int32_t* slots = reinterpret_cast<int32_t*>(lds);
  uint8_t* vtile = lds + a.slot_lds_bytes + wave * kWaveLds;

  // the query's raw words first, before any other load (loads complete in order); converted after the slot list
  const int hl = lane & 15, j = lane >> 4;
  const bool q_valid = active && hl < a.group;
  uint4 qraw[4];
  {
    const int head = (active ? kvh : 0) * a.group + (q_valid ? hl : 0);
    const uint16_t* qp = a.q + (int64_t)row * a.q_rs + (int64_t)head * a.q_hs;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      qraw[kk] = q_valid ? *reinterpret_cast<const uint4*>(qp + 32 * j + 8 * kk) : make_uint4(0u, 0u, 0u, 0u);
  }

  // 1. the split's pool slots (-1: invalid key), shared by the workgroup's waves; each half owns a whole number of
  // prefetch groups, padded with invalid keys that compute to no-ops (P = 0, V = 0, maximum unchanged)
  const int count = a.counts ? min(a.counts[row], a.topk) : a.topk;
  const int t0 = split * a.keys_per_split;
  const int n = max(0, min(t0 + a.keys_per_split, count) - t0);
  const int half_steps = (((n + kStep - 1) / kStep + kHalves * P - 1) / (kHalves * P)) * P;
  {
    const int32_t seqlen = a.seq_lens[row];
    const int32_t qpos = a.query_pos ? a.query_pos[row] : 0x7FFFFFFF;
    const int64_t trow = a.row_req ? a.row_req[row] : row;
    const int32_t* tp = a.table + trow * a.table_stride;
    const int32_t* ip = a.indices + (int64_t)row * a.idx_stride + t0;
    for (int i = threadIdx.x; i < kHalves * half_steps * kStep; i += blockDim.x) {
      int32_t slot = -1;
      if (i < n) {
        const int32_t pos = ip[i];
        if (pos >= 0 && pos < seqlen && pos <= qpos) {
          const int64_t sl = (a.page_size == 1) ? (int64_t)tp[pos]
                                                : (int64_t)tp[pos / a.page_size] * a.page_size + pos % a.page_size;
          if (sl >= 0 && sl < a.pool_slots) slot = (int32_t)sl;
        }
      }
      slots[i] = slot;
    }
  }
  __syncthreads();

  // B operand of the QK MFMAs: FP16 of q * scale * log2(e); heads beyond the group are zero
  half8_t qb[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const uint32_t ws[4] = {qraw[kk].x, qraw[kk].y, qraw[kk].z, qraw[kk].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qb[kk][2 * e] = (_Float16)(bf16_bits_to_f32(ws[e] & 0xFFFFu) * a.qscale);
      qb[kk][2 * e + 1] = (_Float16)(bf16_bits_to_f32(ws[e] >> 16) * a.qscale);
    }
  }
  SoftmaxState st;
  st.m = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) st.acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};

  if (active && half_steps > 0) {
    WaveCtx w;
    w.row_bytes = a.pay_stride;
    w.row_scales = a.sf_stride;
    w.kp = a.k_pay + (int64_t)kvh * (kDim / 2);
    w.vp = a.v_pay + (int64_t)kvh * (kDim / 2);
    w.ksf = a.k_sf + (int64_t)kvh * (kDim / 16);
    w.vsf = a.v_sf + (int64_t)kvh * (kDim / 16);
    w.slots = slots + half * half_steps * kStep;
    w.lane = lane;
    w.hl = hl;
    w.j = j;
    Step buf[P];
#pragma unroll
    for (int p = 0; p < P; ++p) load_step(w, p, buf[p]);
    const float gk = *a.gk;
    int s0 = 0;
    for (; s0 + P < half_steps; s0 += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        compute_step(w, s0 + p, buf[p], qb, gk, vtile, st);
        load_step(w, s0 + p + P, buf[p]);
      }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) compute_step(w, s0 + p, buf[p], qb, gk, vtile, st);
  }
  // the 4 lanes of a head hold disjoint key subsets of l
  float l_tot = st.l + __shfl_xor(st.l, 16);
  l_tot += __shfl_xor(l_tot, 32);

  // 2. the second half hands (max, sum, acc) to the first through LDS
  __syncthreads();
  float* mg = reinterpret_cast<float*>(lds) + (wave & (kHeadsPerGroup - 1)) * 64 * 36 + lane * 36;
  if (half == 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) reinterpret_cast<float4_t*>(mg)[i] = st.acc[i];
    mg[32] = st.m;
    mg[33] = l_tot;
  }
  __syncthreads();
  if (half == 0 && active && hl < a.group) {
    const float m1 = mg[32], l1 = mg[33];
    const float mx = fmaxf(st.m, m1);
    const float mu = (mx == -__builtin_inff()) ? 0.0f : mx;
    const float a0 = __builtin_amdgcn_exp2f(st.m - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] = st.acc[i] * a0 + reinterpret_cast<const float4_t*>(mg)[i] * a1;
    l_tot = l_tot * a0 + l1 * a1;
    st.m = mx;
  }
  const int head = kvh * a.group + hl;
  if (a.splits == 1) {   // no partials: normalize and write
    if (half == 1 || !active || hl >= a.group) return;
    const float gv = *a.gv;
    const float inv = l_tot > 0.0f ? gv / l_tot : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = st.acc[i][r] * inv;
      store_out(a, row, head, 32 * j + 8 * r, v, 8);
    }
    if (a.lse && j == 0)
      a.lse[(int64_t)row * a.q_heads + head] =
          l_tot > 0.0f ? (st.m + __builtin_log2f(l_tot)) * kLn2 : -__builtin_inff();
    return;
  }
  // 3. partials of this row, written through; the last workgroup of (row, KV group) to arrive merges them
  float* row_part = a.part + (int64_t)row * a.splits * a.q_heads * kPartStride;
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      row_part, (short)0, (int)((int64_t)a.splits * a.q_heads * kPartStride * 4), 0x00020000);
  if (half == 0 && active && hl < a.group) {
    const int at = ((split * a.q_heads + head) * kPartStride) * 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      store_through(pr, at + (32 * j + 8 * r) * 4, float4_t{st.acc[0][r], st.acc[1][r], st.acc[2][r], st.acc[3][r]});
      store_through(pr, at + (32 * j + 8 * r + 4) * 4,
                    float4_t{st.acc[4][r], st.acc[5][r], st.acc[6][r], st.acc[7][r]});
    }
    if (j == 0) store_through(pr, at + kDim * 4, float4_t{st.m, l_tot, 0.0f, 0.0f});
  }
  __builtin_amdgcn_s_waitcnt(0);   // this thread's stores have reached memory
  __syncthreads();
  __shared__ int32_t s_last;
  int32_t* counter = a.counters + (int64_t)row * a.kv_groups + kvg;
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.splits - 1;
  __syncthreads();
  if (!s_last) return;
  // 512 threads, 8 consecutive outputs each: head h0 + o / 128, d0 = o % 128; loads of 8 splits at a time together
  const int h0 = kvg * kHeadsPerGroup * a.group;
  const int nh = min(kHeadsPerGroup * a.group, a.q_heads - h0);
  const float gv = *a.gv;
  for (int o = threadIdx.x * 8; o < nh * kDim; o += blockDim.x * 8) {
    const int hh = h0 + o / kDim, d0 = o % kDim;
    const float* base = row_part + (int64_t)hh * kPartStride;
    const int64_t sstride = (int64_t)a.q_heads * kPartStride;
    float m_run = -__builtin_inff(), l_run = 0.0f;
    float4_t o0 = float4_t{0.f, 0.f, 0.f, 0.f}, o1 = o0;
    for (int s0 = 0; s0 < a.splits; s0 += 8) {
      float4_t ml[8], x0[8], x1[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {   // past the last split: reload the last one, weight 0 below
        const float* pp = base + min(s0 + i, a.splits - 1) * sstride;
        ml[i] = reinterpret_cast<const float4_t*>(pp + kDim)[0];
        x0[i] = reinterpret_cast<const float4_t*>(pp + d0)[0];
        x1[i] = reinterpret_cast<const float4_t*>(pp + d0)[1];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (s0 + i >= a.splits) ml[i][0] = -__builtin_inff();
      float mc = m_run;
#pragma unroll
      for (int i = 0; i < 8; ++i) mc = fmaxf(mc, ml[i][0]);
      const float mu = (mc == -__builtin_inff()) ? 0.0f : mc;
      const float alpha = __builtin_amdgcn_exp2f(m_run - mu);
      l_run *= alpha;
      o0 *= alpha;
      o1 *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float wgt = __builtin_amdgcn_exp2f(ml[i][0] - mu);
        l_run += wgt * ml[i][1];
        o0 += wgt * x0[i];
        o1 += wgt * x1[i];
      }
      m_run = mc;
    }
    const float inv = l_run > 0.0f ? gv / l_run : 0.0f;
    const float v[8] = {o0[0] * inv, o0[1] * inv, o0[2] * inv, o0[3] * inv,
                        o1[0] * inv, o1[1] * inv, o1[2] * inv, o1[3] * inv};
    store_out(a, row, hh, d0, v, 8);
    if (a.lse && d0 == 0)
      a.lse[(int64_t)row * a.q_heads + hh] =
          l_run > 0.0f ? (m_run + __builtin_log2f(l_run)) * kLn2 : -__builtin_inff();
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace
}  // namespace xt

using namespace xt;

// Workspace: [counters: rows * q_heads int32 (an upper bound of rows * KV groups), padded to 256 B][partials]
static size_t counter_bytes(int rows, int q_heads) { return (((size_t)rows * q_heads * 4 + 255) / 256) * 256; }

extern "C" size_t xt_sparse_decode_workspace_bytes(int rows, int q_heads, int dim, int splits) {
  if (rows < 0 || q_heads <= 0 || dim <= 0 || splits <= 0) return 0;
  if (splits == 1) return 256;
  return counter_bytes(rows, q_heads) + (size_t)rows * splits * q_heads * (size_t)(dim + 4) * sizeof(float);
}

extern "C" int xt_sparse_decode_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                      const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                                      const uint8_t* v_scales, const float* gk, const float* gv, int64_t pool_slots,
                                      int64_t pay_stride, int64_t sf_stride, int kv_heads, int q_heads, int dim,
                                      const int32_t* table, int64_t table_stride,
                                      int page_size, const int64_t* row_req, const int32_t* indices,
                                      int64_t idx_stride, int topk, const int32_t* counts, const int32_t* seq_lens,
                                      const int32_t* query_pos, float scale, void* out, int64_t out_row_stride,
                                      int64_t out_head_stride, int out_dtype, float* lse, int rows, int splits,
                                      void* workspace, size_t workspace_bytes, xt_stream_t stream) {
  const char* what = "xt_sparse_decode_nvfp4";
  if (dim != kDim) return fail(XT_EUNSUPPORTED, "%s: head size %d (supported: %d)", what, dim, kDim);
  if (kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads != 0)
    return fail(XT_EINVAL, "%s: q_heads %d must be a positive multiple of kv_heads %d", what, q_heads, kv_heads);
  const int group = q_heads / kv_heads;
  if (group > 16) return fail(XT_EUNSUPPORTED, "%s: GQA group %d (supported: <= 16)", what, group);
  if (rows < 0 || topk < 0 || page_size <= 0) return fail(XT_EINVAL, "%s: bad rows/topk/page_size", what);
  if (splits < 1 || splits > 64) return fail(XT_EINVAL, "%s: splits %d outside 1..64", what, splits);
  if (out_dtype != XT_DTYPE_BF16 && out_dtype != XT_DTYPE_F16)
    return fail(XT_EINVAL, "%s: output dtype must be BF16 or FP16", what);
  if (rows == 0) return ok();
  if (!q || !k_pay || !v_pay || !k_scales || !v_scales || !gk || !gv || !table || !indices || !seq_lens || !out ||
      !workspace)
    return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (pool_slots <= 0 || pool_slots > 0x7FFFFFFFLL)
    return fail(XT_EINVAL, "%s: pool_slots %lld outside 1..2^31-1", what, (long long)pool_slots);
  if (!aligned(q, 16) || q_row_stride % 8 || q_head_stride % 8 || !aligned(out, 16) || out_row_stride % 8 ||
      out_head_stride % 8)
    return fail(XT_EINVAL, "%s: q and out rows must be 16-byte aligned (strides in elements: multiples of 8)", what);
  if (pay_stride == 0) pay_stride = (int64_t)kv_heads * (dim / 2);
  if (sf_stride == 0) sf_stride = (int64_t)kv_heads * (dim / 16);
  if (pay_stride < (int64_t)kv_heads * (dim / 2) || sf_stride < (int64_t)kv_heads * (dim / 16) || pay_stride % 16 ||
      sf_stride % 4)
    return fail(XT_EINVAL, "%s: slot strides %lld / %lld bytes must hold the heads' payload / scales and be multiples "
                "of 16 / 4", what, (long long)pay_stride, (long long)sf_stride);
  if (!aligned(k_pay, 16) || !aligned(v_pay, 16) || !aligned(k_scales, 4) || !aligned(v_scales, 4))
    return fail(XT_EINVAL, "%s: payload must be 16-byte and scales 4-byte aligned", what);
  if (lse && !aligned(lse, 4)) return fail(XT_EINVAL, "%s: lse must be 4-byte aligned", what);
  const size_t need = xt_sparse_decode_workspace_bytes(rows, q_heads, dim, splits);
  if (workspace_bytes < need)
    return fail(XT_EWORKSPACE, "%s: workspace %zu bytes < %zu needed", what, workspace_bytes, need);
  if (!aligned(workspace, 256)) return fail(XT_EINVAL, "%s: workspace must be 256-byte aligned", what);
  const int per_split = (topk + splits - 1) / splits;
  const int kps = ((per_split + kStep - 1) / kStep) * kStep;
  const int half_steps = ((kps / kStep + kHalves * kPrefetch - 1) / (kHalves * kPrefetch)) * kPrefetch;
  const int slot_bytes = kHalves * half_steps * kStep * (int)sizeof(int32_t);
  size_t lds_bytes = (size_t)slot_bytes + (size_t)kWaves * kWaveLds;
  if (lds_bytes < (size_t)kMergeLds) lds_bytes = kMergeLds;
  if (lds_bytes > 64 * 1024)
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
  a.gk = gk;
  a.gv = gv;
  a.pool_slots = pool_slots;
  a.pay_stride = pay_stride;
  a.sf_stride = sf_stride;
  a.kv_heads = kv_heads;
  a.q_heads = q_heads;
  a.group = group;
  a.kv_groups = (kv_heads + kHeadsPerGroup - 1) / kHeadsPerGroup;
  a.table = table;
  a.table_stride = table_stride;
  a.page_size = page_size;
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
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + counter_bytes(rows, q_heads));
  a.n_units = (int64_t)rows * a.kv_groups * splits;
  // per-XCD ranges of whole rows, so that a row's splits share an XCD (with fewer than 8 rows, plain numbering keeps
  // every XCD busy)
  const int64_t per_row = (int64_t)a.kv_groups * splits;
  a.xcd_map = rows >= 8;
  a.per_xcd = ((rows + 7) / 8) * per_row;
  const int64_t launched = a.xcd_map ? 8 * a.per_xcd : a.n_units;
  if (launched > 0x7FFFFFFFLL) return fail(XT_EUNSUPPORTED, "%s: %lld workgroups", what, (long long)launched);

  hipLaunchKernelGGL(decode_split_kernel<kPrefetch>, dim3((unsigned)launched), dim3(64 * kWaves), lds_bytes,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(what);
}
