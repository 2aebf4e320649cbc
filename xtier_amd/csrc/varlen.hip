// Split-K GQA decode over packed BF16 K/V rows (the varlen attention QSA runs after its gather): row r's one query
// attends to keys [cu_k[r], cu_k[r+1]) of k / v [keys, kv_heads, D]. q.k and p.v on MFMA (v_mfma_f32_16x16x32_bf16),
// scores in FP32 scaled by softmax_scale * log2(e), exp2, P rounded to BF16 for the PV product, FP32 sums and
// accumulators; key splits merged in FP32 by the last workgroup of a (row, KV head) to finish, in the same launch.
//
// Work decomposition: a workgroup = 8 wavefronts = HPW consecutive KV heads x T head tiles (16 query heads each,
// T = ceil(group / 16)) x 8 / (HPW T) key slices of one (row, KV head group, key split). A wave walks its slice in
// steps of 32 keys; the slices of a (KV head, tile) merge through LDS. With HPW = 4 the waves of a slice read the same
// keys' rows of every KV head at once, so the workgroup streams whole key rows ([keys, KV heads, D] packed); one KV
// head per workgroup reads its 2D-byte pieces at the key stride, which streamed at 39 % of HBM peak against 64 % for
// whole rows (batch 32, 4 KV heads, 2048 keys per row, loads alone). Workgroups are numbered so that a row's units run
// on one XCD (workgroup g runs on XCD g % 8).
//
// Lane layouts (16x16x32 MFMA, hl = lane % 16, j = lane / 16):
//   QK: A = K tile, lane (key hl, dims (D/4) j + 8 kk .. +7 for MFMA kk); B = Q^T, lane (head hl, same dims);
//       C = S^T, lane (head hl, keys 4j .. 4j+3 of the 16-key tile).
//   PV: A = V^T, lane (dim hl of a 16-dim tile, keys T(j) = {4j..4j+3, 16+4j..16+4j+3}), read from the wave's LDS copy
//       of the V tile with ds_read_b64_tr_b16; B = P^T, lane (head hl, keys T(j)); C = O^T, lane (head hl, dims
//       4j .. 4j+3 of the tile).
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef short short8_t __attribute__((ext_vector_type(8)));

constexpr int kVStep = 32;           // keys per step
constexpr int kVWaves = 8;
constexpr float kVRescale = 8.0f;    // log2 of the largest P before the running maximum is raised

struct VarlenArgs {
  const uint16_t* q;
  int64_t q_rs, q_hs;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_ns, k_hs, v_ns, v_hs;    // element strides: key, KV head
  const int32_t* cu_q;
  const int32_t* cu_k;
  int heads, kv_heads, group, tiles;
  int hpw, kv_groups;                // KV heads per workgroup, workgroups per (row, split)
  float qscale;                      // softmax scale * log2(e)
  int splits, keys_per_split;        // keys_per_split: a multiple of kVStep
  uint16_t* out;
  int64_t o_rs, o_hs;
  int out_dtype;
  float* part;                       // [rows, splits, heads, D + 4]: accumulators, max (log2), sum
  int32_t* counters;                 // [rows * kv_groups]
  uint32_t xcd_units, xcd_extra;
};

template <int D>
struct VStep {
  uint4 k[2][D / 32];   // K row pieces: key 16 tt + hl, dims (D/4) j .. +D/4-1
  uint4 v[D / 16];      // V row half: key lane / 2, bytes D (lane % 2) .. +D-1
};

__device__ inline int vkey_of(int j, int e) { return (e < 4) ? (4 * j + e) : (16 + 4 * j + (e - 4)); }

template <int D>
__device__ inline void load_vstep(const VarlenArgs& a, const uint16_t* kb, const uint16_t* vb, int first, int last,
                                  int lane, VStep<D>& s) {
  const int hl = lane & 15, j = lane >> 4;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int key = min(first + 16 * tt + hl, last);
    const uint4* p = reinterpret_cast<const uint4*>(kb + key * a.k_ns + (D / 4) * j);
#pragma unroll
    for (int c = 0; c < D / 32; ++c) s.k[tt][c] = p[c];
  }
  const int key = min(first + (lane >> 1), last);
  const uint4* p = reinterpret_cast<const uint4*>(vb + key * a.v_ns + (D / 2) * (lane & 1));
#pragma unroll
  for (int c = 0; c < D / 16; ++c) s.v[c] = p[c];
}

template <int D>
struct VState {
  float m;                  // reference maximum of head hl (log2 domain), the same on the 4 lanes of the head
  float l;                  // this lane's share of the sum of 2^(s - m)
  float4_t acc[D / 16];     // O^T of head hl, dims 16 dt + 4j + r in acc[dt][r]
};

template <int D>
__device__ inline void compute_vstep(const VarlenArgs& a, const VStep<D>& s, int n_valid, const bf16x8_t (&qb)[D / 32],
                                     uint8_t* vt, int lane, VState<D>& st) {
  constexpr int kRow = 2 * D + 16;   // LDS bytes per key of the V tile
  const int hl = lane & 15, j = lane >> 4;
  // V tile into LDS (the wave's own region; LDS operations of a wave complete in order)
#pragma unroll
  for (int c = 0; c < D / 16; ++c)
    *reinterpret_cast<uint4*>(vt + (lane >> 1) * kRow + D * (lane & 1) + 16 * c) = s.v[c];
  float4_t sc[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    sc[tt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < D / 32; ++c)
      sc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, s.k[tt][c]), qb[c], sc[tt], 0, 0,
                                                       0);
  }
  float sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = sc[e >> 2][e & 3] * a.qscale;
    sv[e] = vkey_of(j, e) < n_valid ? x : -__builtin_inff();
  }
  float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
  mt = max4_lanes16(mt);
  if (__builtin_amdgcn_ballot_w64(mt > st.m + kVRescale)) {
    const float m_new = (mt > st.m + kVRescale) ? mt : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.l *= alpha;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) st.acc[dt] *= alpha;
    st.m = m_new;
  }
  const float m_use = (st.m == -__builtin_inff()) ? 0.0f : st.m;
  bf16x8_t pb;
  float psum = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = __builtin_amdgcn_exp2f(sv[e] - m_use);
    psum += p;
    pb[e] = (__bf16)p;
  }
  st.l += psum;
  asm volatile("" ::: "memory");
  // V^T operands: lane l of a 16-lane group addresses key 4j + l/4, dims 16 dt + 4 (l % 4); the transposing read
  // returns dim 16 dt + hl of keys 4j .. 4j+3 (then 16 + 4j .. from the second read)
  const uint8_t* vr = vt + (4 * j + (hl >> 2)) * kRow + 8 * (hl & 3);
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4_t*)(vr + 32 * dt));
    const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4_t*)(vr + 16 * kRow + 32 * dt));
    const short8_t both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    st.acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, both), pb, st.acc[dt], 0, 0, 0);
  }
  asm volatile("" ::: "memory");
}

__device__ inline void store_row(const VarlenArgs& a, int64_t query, int head, int d0, const float* v, int n) {
  uint16_t* o = a.out + query * a.o_rs + (int64_t)head * a.o_hs + d0;
  for (int e = 0; e < n; e += 2) {
    const uint32_t packed = a.out_dtype == XT_DTYPE_BF16
                                ? (f32_to_bf16_bits(v[e]) | (f32_to_bf16_bits(v[e + 1]) << 16))
                                : (f32_to_f16_bits(v[e]) | (f32_to_f16_bits(v[e + 1]) << 16));
    *reinterpret_cast<uint32_t*>(o + e) = packed;
  }
}

template <int D, int P>
__global__ void __launch_bounds__(512) varlen_kernel(const VarlenArgs a) {
  constexpr int kRow = 2 * D + 16;
  constexpr int kWaveTile = kVStep * kRow;
  constexpr int kPart = D + 4;
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t g = blockIdx.x, xcd = g & 7u;
  const uint32_t u = xcd * a.xcd_units + min(xcd, a.xcd_extra) + (g >> 3);
  const uint32_t splits_u = (uint32_t)a.splits, groups_u = (uint32_t)a.kv_groups;
  const int split = (int)(u % splits_u);
  const int kvg = (int)((u / splits_u) % groups_u);
  const int row = (int)(u / splits_u / groups_u);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int hl = lane & 15, j = lane >> 4;
  // wave = (slice * T + tile) * HPW + KV head within the group
  const int hw = wave % a.hpw, tile = (wave / a.hpw) % a.tiles, slice = wave / (a.hpw * a.tiles);
  const int slices = kVWaves / (a.hpw * a.tiles);
  const int kvh = kvg * a.hpw + hw;
  const int gh = 16 * tile + hl;                 // head within the KV head's group
  const bool head_live = gh < a.group;
  const int head = kvh * a.group + min(gh, a.group - 1);

  const int64_t query = a.cu_q[row];
  const int k0 = a.cu_k[row];
  const int count = a.cu_k[row + 1] - k0;
  // Q^T operand (unscaled BF16); heads beyond the group are zero
  bf16x8_t qb[D / 32];
  {
    const uint4* qp = reinterpret_cast<const uint4*>(a.q + query * a.q_rs + (int64_t)head * a.q_hs + (D / 4) * j);
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      const uint4 w = qp[c];
      qb[c] = __builtin_bit_cast(bf16x8_t, head_live ? w : uint4{0u, 0u, 0u, 0u});
    }
  }
  VState<D> st;
  st.m = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) st.acc[dt] = float4_t{0.f, 0.f, 0.f, 0.f};

  // this slice's steps of the split
  const int s0 = split * a.keys_per_split;
  const int n_split = max(0, min(a.keys_per_split, count - s0));
  const int steps = (n_split + kVStep - 1) / kVStep;
  const int per = (steps + slices - 1) / slices;
  const int st_begin = slice * per, st_end = min(steps, st_begin + per);
  if (st_begin < st_end) {
    const uint16_t* kb = a.k + (int64_t)k0 * a.k_ns + (int64_t)kvh * a.k_hs;
    const uint16_t* vb = a.v + (int64_t)k0 * a.v_ns + (int64_t)kvh * a.v_hs;
    const int last = count - 1;   // loads past the keys re-read the last key; its score is masked
    uint8_t* vt = lds + wave * kWaveTile;
    VStep<D> buf[P];
#pragma unroll
    for (int p = 0; p < P; ++p) load_vstep<D>(a, kb, vb, s0 + (st_begin + p) * kVStep, last, lane, buf[p]);
    for (int s = st_begin; s < st_end; s += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        if (s + p < st_end) {
          const int first = s0 + (s + p) * kVStep;
          compute_vstep<D>(a, buf[p], min(kVStep, n_split + s0 - first), qb, vt, lane, st);
          if (s + p + P < st_end) load_vstep<D>(a, kb, vb, first + P * kVStep, last, lane, buf[p]);
        }
      }
    }
  }
  float l_tot = sum4_lanes16(st.l);

  // the slices of a tile merge through LDS (the V tiles' space, free after the first barrier): every wave leaves
  // (O^T, max, sum) per lane, then each thread merges 4 dims of one (tile, head, dim group) over the slices and
  // normalizes the output (one split) or writes its share of the split partial
  constexpr int kLane = D / 4 + 4;   // floats per lane: D/4 accumulators, max, sum, 2 pad
  constexpr int kND = D / 16;
  __syncthreads();
  float* mg = reinterpret_cast<float*>(lds);
  {
    float4_t* p = reinterpret_cast<float4_t*>(mg + (wave * 64 + lane) * kLane);
#pragma unroll
    for (int dt = 0; dt < kND; ++dt) p[dt] = st.acc[dt];
    p[kND] = float4_t{st.m, l_tot, 0.0f, 0.0f};
  }
  __syncthreads();
  float* row_part = a.part + (int64_t)row * a.splits * a.heads * kPart;
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      row_part, (short)0, a.splits > 1 ? (int)((int64_t)a.splits * a.heads * kPart * 4) : 0, 0x00020000);
  // unit u: dims 16 dt + 4 uj .. +3 of head 16 utile + uhl of KV head uhw (uj fastest, so consecutive threads write
  // one head row)
  for (int u = (int)threadIdx.x; u < a.hpw * a.tiles * 64 * kND; u += 64 * kVWaves) {
    const int uj = u & 3, rest = u >> 2;
    const int dt = rest % kND, uhl = (rest / kND) & 15, ut = rest / kND / 16;
    const int utile = ut % a.tiles, uhw = ut / a.tiles;
    const int ugh = 16 * utile + uhl;
    if (ugh >= a.group) continue;
    const int ln = uhl + 16 * uj;
    float mx = -__builtin_inff(), l = 0.0f;
    float4_t o = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int sl = 0; sl < slices; ++sl) {   // online merge: rescale what is held when a larger maximum arrives
      const int sw = (sl * a.tiles + utile) * a.hpw + uhw;   // the wave of slice sl of this (KV head, tile)
      const float4_t* src = reinterpret_cast<const float4_t*>(mg + (sw * 64 + ln) * kLane);
      const float4_t ml = src[kND];
      const float m_new = fmaxf(mx, ml[0]);
      const float mu = (m_new == -__builtin_inff()) ? 0.0f : m_new;
      const float a0 = __builtin_amdgcn_exp2f(mx - mu), a1 = __builtin_amdgcn_exp2f(ml[0] - mu);
      o = o * a0 + src[dt] * a1;
      l = l * a0 + ml[1] * a1;
      mx = m_new;
    }
    const int uhead = (kvg * a.hpw + uhw) * a.group + ugh, d0 = 16 * dt + 4 * uj;
    if (a.splits == 1) {
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
      const float v[4] = {o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv};
      store_row(a, query, uhead, d0, v, 4);
    } else {   // partials of this (row, split), written through; the last workgroup of (row, KV head) merges them
      const int at = ((split * a.heads + uhead) * kPart) * 4;
      store_partial(pr, at + d0 * 4, o);
      if (d0 == 0) store_partial(pr, at + D * 4, float4_t{mx, l, 0.0f, 0.0f});
    }
  }
  if (a.splits == 1) return;
  // the last workgroup of (row, KV head group) to arrive merges the partials (the split arrival of xt_common.h)
  __shared__ int s_last;
  int32_t* counter = a.counters + (int64_t)row * a.kv_groups + kvg;
  if (!arrive_last(counter, a.splits, &s_last)) return;
  // merge: 512 threads over the KV head group's query heads x D outputs, 8 consecutive dims each; the splits are
  // taken 8 at a time with all their loads issued together (one round trip for up to 8 splits) and an online rescale
  // across groups
  const int nthreads = 64 * kVWaves;
  for (int o = threadIdx.x * 8; o < a.hpw * a.group * D; o += nthreads * 8) {
    const int hh = kvg * a.hpw * a.group + o / D, d0 = o % D;
    float m_run = -__builtin_inff(), l_run = 0.0f;
    float4_t o0 = float4_t{0.f, 0.f, 0.f, 0.f}, o1 = o0;
    for (int s0 = 0; s0 < a.splits; s0 += 8) {
      float2 ml[8];
      float4_t x0[8], x1[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {   // past the last split: the last one again, weight 0 below
        const int at = (min(s0 + i, a.splits - 1) * a.heads + hh) * kPart * 4;
        const float4_t m4 = load_partial(pr, at + D * 4);
        ml[i] = make_float2(m4[0], m4[1]);
        x0[i] = load_partial(pr, at + d0 * 4);
        x1[i] = load_partial(pr, at + d0 * 4 + 16);
      }
      float mc = m_run;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (s0 + i >= a.splits) ml[i].x = -__builtin_inff();
        mc = fmaxf(mc, ml[i].x);
      }
      const float mu = (mc == -__builtin_inff()) ? 0.0f : mc;
      const float alpha = __builtin_amdgcn_exp2f(m_run - mu);
      l_run *= alpha;
      o0 *= alpha;
      o1 *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float w = __builtin_amdgcn_exp2f(ml[i].x - mu);
        l_run += w * ml[i].y;
        o0 += w * x0[i];
        o1 += w * x1[i];
      }
      m_run = mc;
    }
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const float v[8] = {o0[0] * inv, o0[1] * inv, o0[2] * inv, o0[3] * inv,
                        o1[0] * inv, o1[1] * inv, o1[2] * inv, o1[3] * inv};
    store_row(a, query, hh, d0, v, 8);
  }
  reset_counter(counter);
}

template <int D>
int launch(const VarlenArgs& a, int64_t units, xt_stream_t stream, const char* what) {
  constexpr int kRow = 2 * D + 16;
  const size_t tiles_bytes = (size_t)kVWaves * kVStep * kRow;
  const size_t merge_bytes = (size_t)kVWaves * 64 * (D / 4 + 4) * 4;
  const size_t lds_bytes = tiles_bytes > merge_bytes ? tiles_bytes : merge_bytes;
  constexpr int P = D >= 256 ? 1 : 2;
  const void* fn = reinterpret_cast<const void*>(&varlen_kernel<D, P>);
  if (int e = allow_lds(fn, lds_bytes, what)) return e;
  hipLaunchKernelGGL((varlen_kernel<D, P>), dim3((unsigned)units), dim3(64 * kVWaves), lds_bytes,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch(what);
}

}  // namespace
}  // namespace xt

using namespace xt;

// Workspace: [arrival counters, kCounterBytes][partials [rows, splits, heads, dim + 4] FP32]

extern "C" size_t xt_varlen_decode_workspace_bytes(int rows, int heads, int dim, int splits) {
  if (rows < 0 || heads <= 0 || dim <= 0 || splits <= 0) return 0;
  if (splits == 1) return 256;
  return kCounterBytes + (size_t)rows * splits * heads * (size_t)(dim + 4) * sizeof(float);
}

extern "C" int xt_varlen_decode_bf16(const void* q, int64_t q_row_stride, int64_t q_head_stride, const void* k,
                                     int64_t k_key_stride, int64_t k_head_stride, const void* v,
                                     int64_t v_key_stride, int64_t v_head_stride, const int32_t* cu_seqlens_q,
                                     const int32_t* cu_seqlens_k, int rows, int heads, int kv_heads, int dim,
                                     int max_seqlen_k, float softmax_scale, void* out, int64_t out_row_stride,
                                     int64_t out_head_stride, int out_dtype, int splits, void* workspace,
                                     size_t workspace_bytes, xt_stream_t stream) {
  const char* what = "xt_varlen_decode_bf16";
  if (dim != 64 && dim != 128 && dim != 256)
    return fail(XT_EUNSUPPORTED, "%s: head size %d (supported: 64, 128, 256)", what, dim);
  if (kv_heads <= 0 || heads <= 0 || heads % kv_heads)
    return fail(XT_EINVAL, "%s: heads %d must be a positive multiple of kv_heads %d", what, heads, kv_heads);
  const int group = heads / kv_heads;
  const int tiles = group <= 16 ? 1 : group <= 32 ? 2 : group <= 64 ? 4 : group <= 128 ? 8 : 0;
  if (!tiles) return fail(XT_EUNSUPPORTED, "%s: GQA group %d (supported: <= 128)", what, group);
  if (rows < 0 || max_seqlen_k < 0) return fail(XT_EINVAL, "%s: bad rows / max_seqlen_k", what);
  if (splits < 1 || splits > 64) return fail(XT_EINVAL, "%s: splits %d outside 1..64", what, splits);
  if (out_dtype != XT_DTYPE_BF16 && out_dtype != XT_DTYPE_F16)
    return fail(XT_EINVAL, "%s: output dtype must be BF16 or FP16", what);
  if (rows == 0) return ok();
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out || !workspace)
    return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16) || q_row_stride % 8 ||
      q_head_stride % 8 || k_key_stride % 8 || k_head_stride % 8 || v_key_stride % 8 || v_head_stride % 8 ||
      out_row_stride % 8 || out_head_stride % 8)
    return fail(XT_EINVAL, "%s: q / k / v / out rows must be 16-byte aligned (strides in elements: multiples of 8)",
                what);
  // KV heads per workgroup: 4 (or 2) whole-row heads when that many workgroups still fill every CU, else 1
  const int cus = device_cus();
  int hpw = 1;
  for (int h : {4, 2})
    if (hpw == 1 && kv_heads % h == 0 && h * tiles <= kVWaves && (int64_t)rows * (kv_heads / h) * splits >= cus) hpw = h;
  if (splits > 1 && (int64_t)rows * (kv_heads / hpw) > kCounterSlots)
    return fail(XT_EUNSUPPORTED, "%s: %d rows x %d KV head groups with key splits exceed %d arrival counters; use "
                "splits 1", what, rows, kv_heads / hpw, kCounterSlots);
  const size_t need = xt_varlen_decode_workspace_bytes(rows, heads, dim, splits);
  if (workspace_bytes < need)
    return fail(XT_EWORKSPACE, "%s: workspace %zu bytes < %zu needed", what, workspace_bytes, need);
  if (!aligned(workspace, 256)) return fail(XT_EINVAL, "%s: workspace must be 256-byte aligned", what);
  VarlenArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_rs = q_row_stride;
  a.q_hs = q_head_stride;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_ns = k_key_stride;
  a.k_hs = k_head_stride;
  a.v_ns = v_key_stride;
  a.v_hs = v_head_stride;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.group = group;
  a.tiles = tiles;
  a.hpw = hpw;
  a.kv_groups = kv_heads / hpw;
  a.qscale = softmax_scale * kLog2e;
  a.splits = splits;
  const int per_split = (max_seqlen_k + splits - 1) / splits;
  a.keys_per_split = ((per_split + kVStep - 1) / kVStep) * kVStep;
  if (a.keys_per_split == 0) a.keys_per_split = kVStep;
  a.out = static_cast<uint16_t*>(out);
  a.o_rs = out_row_stride;
  a.o_hs = out_head_stride;
  a.out_dtype = out_dtype;
  a.counters = static_cast<int32_t*>(workspace);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  const int64_t units = (int64_t)rows * a.kv_groups * splits;
  if (units > 0x7FFFFFFFLL) return fail(XT_EUNSUPPORTED, "%s: %lld workgroups", what, (long long)units);
  a.xcd_units = (uint32_t)(units / 8);
  a.xcd_extra = (uint32_t)(units % 8);
  if (dim == 64) return launch<64>(a, units, stream, what);
  if (dim == 128) return launch<128>(a, units, stream, what);
  return launch<256>(a, units, stream, what);
}
