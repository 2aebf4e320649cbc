// Sparse MLA over an NVFP4 latent cache: 128 query heads share one key per token, [latent (512, NVFP4) | rope (64,
// BF16)] = 576 wide, whose value is the latent. q.k and p.v on MFMA (v_mfma_f32_16x16x32_f16), online softmax in the
// exp2 domain, an optional per-head sink in the denominator. With key splits, each (row, split) writes its output
// normalized by its own sum (FP16) with its max and sum, and a second, wide launch merges the splits: one merging
// workgroup per row would read a row's partials at one CU's bandwidth.
//
// Work decomposition: a workgroup = 8 wavefronts x 16 heads = 128 heads of one (query row, key split), so every key is
// read and dequantized once for all heads. Per step of 32 keys the workgroup
//   1. turns the raw key records (loaded one step ahead into registers) into two LDS tiles: K [32 keys][576] FP16 and
//      V^T [512][32 keys] FP16, the latent as FP16((e2m1 * e4m3) * g) and the rope widened from BF16;
//   2. each wave computes S^T [32 keys x 16 heads] = K . Q^T (18 MFMAs per 16-key tile, Q^T resident in registers
//      as FP16 of q * scale * log2(e)), the softmax, and O^T [512 x 16 heads] += V^T . P^T (32 MFMAs), P^T taken
//      straight from the score registers (the key order T(j) below matches the V^T operand).
//
// Lane layouts (16x16x32 MFMA, hl = lane % 16, j = lane / 16):
//   QK: A = K tile, lane (key hl, dims 32kk + 8j .. +7); B = Q^T, lane (head hl, same dims); C = S^T, lane (head hl,
//       keys 4j .. 4j+3 of the 16-key tile).
//   PV: A = V^T, lane (dim hl of a 16-dim tile, keys T(j) = {4j..4j+3, 16+4j..16+4j+3}); B = P^T, lane (head hl, keys
//       T(j)); C = O^T, lane (head hl, dims 4j .. 4j+3 of the tile).
//
// Numerics: FP16((e2m1 * e4m3) * g) rounds the dequantized latent once (11 significant bits); the rope is exact
// in FP16 within its range. P is FP16 with the lazy rescale of the decode kernel (P <= 256); sums are FP32.
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

constexpr int kDl = 512;                 // latent width (NVFP4): 256 payload bytes, 32 scale bytes per token
constexpr int kDr = 64;                  // rope width (BF16): 128 bytes per token
constexpr int kDk = kDl + kDr;           // key width
constexpr int kMSteps = 32;              // keys per step
constexpr int kMWaves = 8;
constexpr int kMHeads = 16 * kMWaves;    // heads per workgroup
constexpr int kKRow = kDk + 8;           // halves per K tile row (16-byte pad)
constexpr int kVRow = kMSteps + 16;      // halves per V^T tile row (96 bytes); keys stored in the order of the PV
                                         // operand, position 8j + 4b + s holding key 16b + 4j + s, so a lane's eight
                                         // keys are one 16-byte read (at this pitch without LDS bank conflicts)
constexpr int kKTile = kMSteps * kKRow * 2;
constexpr int kVTile = kDl * kVRow * 2;
constexpr int kQChunks = kDk / 32;       // 32-dim chunks of a query row
constexpr int kQReg = 12;                // chunks kept in registers; the others (4 latent + 2 rope) live in LDS
constexpr int kQRow = 32 + 8;            // halves per (chunk, head) row of the LDS query block
constexpr int kQTile = (kQChunks - kQReg) * kMHeads * kQRow * 2;
constexpr int kRescaleM = 8;

struct CacheDev {
  const uint8_t* pay;
  const uint8_t* sf;
  const uint16_t* rope;
  const float* g;
  int64_t slots;
  uint32_t pay_stride, sf_stride, rope_stride;   // bytes from one slot to the next
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
  uint16_t* part;                    // [rows, splits, heads, 512] FP16: the split's output normalized by its own sum
  float* ml;                         // [rows, splits, heads, 2]: the split's running max (log2 domain) and sum
  uint32_t xcd_units, xcd_extra;
};

// Slot list entries: >= 0 a slot of cache 0, <= -2 slot (-e - 2) of cache 1, -1 no key.
__device__ inline bool entry_valid(int32_t e) { return e != -1; }

// Dequant mapping: thread t handles keys 4kq .. 4kq+3 (kq = t % 8) and latent dims 8c .. 8c+7 (c = t / 8), so a
// wave's V^T writes spread over 8 key columns and 8 dim rows (no LDS bank conflicts); rope: key t / 8, part t % 8.
struct Raw {
  uint32_t pay[4];   // payload bytes 4c .. 4c+3 of keys 4kq + i
  uint32_t sc[4];    // scale byte c / 2 of those keys
  uint4 rope;        // rope values 8p .. 8p+7 of key t / 8 (threads 0-255)
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

template <bool TWO>
__device__ inline void load_raw(const MlaArgs& a, const int32_t* slots, int step, Raw& r) {
  const int t = threadIdx.x, kq = t & 7, c = t >> 3;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t s;
    const CacheDev& cd = cache_of<TWO>(a, slots[step * kMSteps + 4 * kq + i], s);
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

// Raw records -> K and V^T tiles. An invalid key's latent becomes 0 (so P * V stays finite whatever slot 0 holds);
// its rope is left as read: its score is masked by a select, never multiplied.
template <bool TWO>
__device__ inline void dequant(const MlaArgs& a, const int32_t* slots, int step, const Raw& r, float g0, float g1,
                               _Float16* kt, _Float16* vt) {
  typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
  const int t = threadIdx.x, kq = t & 7, c = t >> 3;
  half8_t vals[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int32_t e = slots[step * kMSteps + 4 * kq + i];
    const float g = (TWO && e <= -2) ? g1 : g0;
    const float sg = entry_valid(e) ? (float)fp8x2_to_f16<false>(r.sc[i]).x * g : 0.0f;
    const _Float16 h = (_Float16)sg;
    const half2_t s2 = half2_t{h, h};
    const half2_t p0 = fp4x2_to_f16<0>(r.pay[i]) * s2, p1 = fp4x2_to_f16<1>(r.pay[i]) * s2;
    const half2_t p2 = fp4x2_to_f16<2>(r.pay[i]) * s2, p3 = fp4x2_to_f16<3>(r.pay[i]) * s2;
    vals[i] = half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    *reinterpret_cast<half8_t*>(kt + (4 * kq + i) * kKRow + 8 * c) = vals[i];
  }
#pragma unroll
  for (int d = 0; d < 8; ++d)
    *reinterpret_cast<half4_t*>(vt + (8 * c + d) * kVRow + 8 * (kq & 3) + 4 * (kq >> 2)) =
        half4_t{vals[0][d], vals[1][d], vals[2][d], vals[3][d]};
  if (t < 256) {
    const int key = t >> 3, p = t & 7;
    const uint32_t w[4] = {r.rope.x, r.rope.y, r.rope.z, r.rope.w};
    half8_t hv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {   // BF16 -> FP16 is exact in range, so round-toward-zero packing is exact
      const half2_t pr = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(w[e] << 16),
                                                                                __uint_as_float(w[e] & 0xFFFF0000u)));
      hv[2 * e] = pr.x;
      hv[2 * e + 1] = pr.y;
    }
    *reinterpret_cast<half8_t*>(kt + key * kKRow + kDl + 8 * p) = hv;
  }
}

__device__ inline void store_vals(const MlaArgs& a, int64_t row, int head, int d0, const float* v, int n) {
  uint16_t* o = a.out + row * a.o_rs + (int64_t)head * a.o_hs + d0;
  for (int e = 0; e < n; e += 2) {
    uint32_t packed;
    if (a.out_dtype == XT_DTYPE_BF16)
      packed = f32_to_bf16_bits(v[e]) | (f32_to_bf16_bits(v[e + 1]) << 16);
    else
      packed = f32_to_f16_bits(v[e]) | (f32_to_f16_bits(v[e + 1]) << 16);
    *reinterpret_cast<uint32_t*>(o + e) = packed;
  }
}


template <bool TWO>
__global__ void __launch_bounds__(512) mla_kernel(const MlaArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  asm volatile("" ::"s"(a.xcd_units), "s"(a.xcd_extra), "s"(a.splits), "s"(a.keys_per_split), "s"(a.topk[0]),
               "s"(a.topk[1]), "s"(a.idx[0]), "s"(a.idx[1]), "s"(a.idx_stride[0]), "s"(a.idx_stride[1]),
               "s"(a.len[0]), "s"(a.len[1]), "s"(a.q), "s"(a.q_rs), "s"(a.q_hs), "s"(a.heads));
  // XCD-aware numbering as in the decode kernel: a row's splits run on one XCD
  const uint32_t gidx = blockIdx.x;
  const uint32_t xcd = gidx & 7u;
  const uint32_t u = xcd * a.xcd_units + min(xcd, a.xcd_extra) + (gidx >> 3);
  const int split = (int)(u % (uint32_t)a.splits);
  const int64_t row = u / (uint32_t)a.splits;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, hl = lane & 15, j = lane >> 4;
  const int head = 16 * wave + hl;
  const bool head_live = head < a.heads;

  _Float16* kt = reinterpret_cast<_Float16*>(lds);
  _Float16* vt = reinterpret_cast<_Float16*>(lds + kKTile);
  _Float16* qs = reinterpret_cast<_Float16*>(lds + kKTile + kVTile);
  int32_t* slots = reinterpret_cast<int32_t*>(lds + kKTile + kVTile + kQTile);

  // the query's B operands first: dims 32kk + 8j .. +7 of head `head` (a clamped valid head for padding lanes)
  uint4 qraw[kQChunks];
  {
    const uint16_t* qp = a.q + row * a.q_rs + (int64_t)min(head, a.heads - 1) * a.q_hs;
#pragma unroll
    for (int kk = 0; kk < kQChunks; ++kk) qraw[kk] = *reinterpret_cast<const uint4*>(qp + 32 * kk + 8 * j);
  }

  // 1. the split's key list: columns [t0, t0 + keys_per_split) of list 0 then list 1, as slot entries in LDS
  const int t0 = split * a.keys_per_split;
  {
    const int total = a.steps * kMSteps;
    for (int i = threadIdx.x; i < total; i += 512) {
      const int col = t0 + i;
      int32_t e = -1;
      if (i < a.keys_per_split) {
        const int li = col < a.topk[0] ? 0 : 1;
        const int cc = col - (li ? a.topk[0] : 0);
        if (cc < a.topk[li]) {
          const int n = a.len[li] ? min(a.len[li][row], a.topk[li]) : a.topk[li];
          const int32_t s = cc < n ? a.idx[li][row * a.idx_stride[li] + cc] : -1;
          if (s >= 0 && s < a.c[li].slots) e = li ? -s - 2 : s;
        }
      }
      slots[i] = e;
    }
  }
  __syncthreads();

  // B operands of q.k: FP16 of q * scale * log2(e), chunks 0..kQReg-1 in registers, the rest in LDS
  half8_t qb[kQReg];
#pragma unroll
  for (int kk = 0; kk < kQChunks; ++kk) {
    const uint32_t ws[4] = {qraw[kk].x, qraw[kk].y, qraw[kk].z, qraw[kk].w};
    half8_t h;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[2 * e] = head_live ? (_Float16)(bf16_bits_to_f32(ws[e] & 0xFFFFu) * a.qscale) : (_Float16)0.0f;
      h[2 * e + 1] = head_live ? (_Float16)(bf16_bits_to_f32(ws[e] >> 16) * a.qscale) : (_Float16)0.0f;
    }
    if (kk < kQReg)
      qb[kk < kQReg ? kk : 0] = h;
    else
      *reinterpret_cast<half8_t*>(qs + ((kk - kQReg) * kMHeads + 16 * wave + hl) * kQRow + 8 * j) = h;
  }
  const float g0 = *a.c[0].g, g1 = TWO ? *a.c[1].g : g0;

  float m = -__builtin_inff(), l = 0.0f;
  float4_t acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};

  Raw raw;
  load_raw<TWO>(a, slots, 0, raw);
  for (int step = 0; step < a.steps; ++step) {
    dequant<TWO>(a, slots, step, raw, g0, g1, kt, vt);
    __syncthreads();
    if (step + 1 < a.steps) load_raw<TWO>(a, slots, step + 1, raw);
    const uint32_t valid = (uint32_t)__builtin_amdgcn_ballot_w64(lane < kMSteps &&
                                                                  entry_valid(slots[step * kMSteps + (lane & 31)]));
    // S^T for the two 16-key tiles, each as two independent MFMA chains (even / odd dim chunks)
    float4_t s[2], s2[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      s[tt] = float4_t{0.f, 0.f, 0.f, 0.f};
      s2[tt] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int kk = 0; kk < kQChunks; ++kk) {
      const half8_t qv = kk < kQReg ? qb[kk < kQReg ? kk : 0]
                                    : *reinterpret_cast<const half8_t*>(
                                          qs + ((kk - kQReg) * kMHeads + 16 * wave + hl) * kQRow + 8 * j);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const half8_t kv = *reinterpret_cast<const half8_t*>(kt + (16 * tt + hl) * kKRow + 8 * j + 32 * kk);
        if (kk & 1)
          s2[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qv, s2[tt], 0, 0, 0);
        else
          s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qv, s[tt], 0, 0, 0);
      }
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) s[tt] += s2[tt];
    // online softmax of head hl over keys T(j), lazy rescale
    float sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = (e < 4) ? (4 * j + e) : (16 + 4 * j + (e - 4));
      sv[e] = ((valid >> key) & 1u) ? s[e >> 2][e & 3] : -__builtin_inff();
    }
    float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    if (__builtin_amdgcn_ballot_w64(mt > m + kRescaleM)) {
      const float m_new = (mt > m + kRescaleM) ? mt : m;
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 32; ++i) acc[i] *= alpha;
      m = m_new;
    }
    const float m_use = (m == -__builtin_inff()) ? 0.0f : m;
    half8_t pb;
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = __builtin_amdgcn_exp2f(sv[e] - m_use);
      psum += p;
      pb[e] = (_Float16)p;
    }
    l += psum;
    // O^T += V^T . P^T over the 32 dim tiles
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) {
      const half8_t av = *reinterpret_cast<const half8_t*>(vt + (16 * dt + hl) * kVRow + 8 * j);
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb, acc[dt], 0, 0, 0);
    }
    __syncthreads();
  }
  // the 4 lanes of a head hold disjoint key subsets of l
  float l_tot = l + __shfl_xor(l, 16);
  l_tot += __shfl_xor(l_tot, 32);

  if (a.splits == 1) {
    if (!head_live) return;
    const float m_use = (m == -__builtin_inff()) ? 0.0f : m;
    float total = l_tot;
    if (a.sink) total += __builtin_amdgcn_exp2f(a.sink[head] * kLog2e - m_use);
    const float inv = l_tot > 0.0f ? 1.0f / total : 0.0f;
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) {
      const float v[4] = {acc[dt][0] * inv, acc[dt][1] * inv, acc[dt][2] * inv, acc[dt][3] * inv};
      store_vals(a, row, head, 16 * dt + 4 * j, v, 4);
    }
    if (a.lse && j == 0)
      a.lse[row * a.heads + head] = l_tot > 0.0f ? (m + __builtin_log2f(l_tot)) * kLn2 : -__builtin_inff();
    return;
  }
  // 2. the split's output normalized by its own sum (FP16: a convex combination of FP16 latent values) plus its
  //    max and sum; a second launch merges the splits
  if (head_live) {
    const int64_t ph = ((int64_t)row * a.splits + split) * a.heads + head;
    uint16_t* pp = a.part + ph * kDl;
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) {
      const uint2 w = {f32_to_f16_bits(acc[dt][0] * inv) | (f32_to_f16_bits(acc[dt][1] * inv) << 16),
                       f32_to_f16_bits(acc[dt][2] * inv) | (f32_to_f16_bits(acc[dt][3] * inv) << 16)};
      *reinterpret_cast<uint2*>(pp + 16 * dt + 4 * j) = w;
    }
    if (j == 0) *reinterpret_cast<float2*>(a.ml + ph * 2) = float2{m, l_tot};
  }
}

// Split merge: one thread per (row, head, 8 dims); 64 threads cover a head's 512 dims with 16-byte loads.
// out = sum_s w_s o_s with w_s = 2^(m_s - max m) l_s / (sum_s 2^(m_s - max m) l_s + sink term).
__global__ void __launch_bounds__(256) mla_merge_kernel(const MlaArgs a, int rows) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rh = t >> 6;                  // row * heads + head
  if (rh >= (int64_t)rows * a.heads) return;
  const int c = (int)(t & 63);
  const int row = (int)(rh / a.heads), head = (int)(rh % a.heads);
  const int64_t base = (int64_t)row * a.splits * a.heads + head;   // (row, split 0, head)
  float mx = -__builtin_inff();
  for (int sp = 0; sp < a.splits; ++sp) mx = fmaxf(mx, a.ml[(base + (int64_t)sp * a.heads) * 2]);
  const float mu = (mx == -__builtin_inff()) ? 0.0f : mx;
  float l_all = 0.0f;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < a.splits; ++sp) {
    const int64_t ph = base + (int64_t)sp * a.heads;
    const float2 ml = *reinterpret_cast<const float2*>(a.ml + ph * 2);
    const uint4 x = *reinterpret_cast<const uint4*>(a.part + ph * kDl + 8 * c);
    const float w = __builtin_amdgcn_exp2f(ml.x - mu) * ml.y;
    l_all += w;
    const uint32_t u[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const half2_t h = __builtin_bit_cast(half2_t, u[e]);
      o[2 * e] += w * (float)h.x;
      o[2 * e + 1] += w * (float)h.y;
    }
  }
  float total = l_all;
  if (a.sink) total += __builtin_amdgcn_exp2f(a.sink[head] * kLog2e - mu);
  const float inv = l_all > 0.0f ? 1.0f / total : 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] *= inv;
  store_vals(a, row, head, 8 * c, o, 8);
  if (a.lse && c == 0) a.lse[rh] = l_all > 0.0f ? (mu + __builtin_log2f(l_all)) * kLn2 : -__builtin_inff();
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

}  // namespace
}  // namespace xt

using namespace xt;

// Workspace: [kCounterBytes, unused here: the counter region of the decode entry points][partial outputs [rows,
// splits, heads, 512] FP16][partial max and sum [rows, splits, heads, 2] FP32]

extern "C" size_t xt_sparse_mla_workspace_bytes(int rows, int heads, int splits) {
  if (rows < 0 || heads <= 0 || splits <= 0) return 0;
  if (splits == 1) return 256;
  return kCounterBytes + (size_t)rows * splits * heads * (kDl * 2 + 2 * sizeof(float));
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
  if (heads <= 0 || heads > kMHeads) return fail(XT_EUNSUPPORTED, "%s: %d heads (supported: 1..%d)", what, heads,
                                                 kMHeads);
  if (rows < 0 || splits < 1 || splits > 64) return fail(XT_EINVAL, "%s: bad rows %d / splits %d", what, rows, splits);
  if (out_dtype != XT_DTYPE_BF16 && out_dtype != XT_DTYPE_F16)
    return fail(XT_EINVAL, "%s: output dtype must be BF16 or FP16", what);
  if (!cache || !keys) return fail(XT_EINVAL, "%s: the key cache and key list are required", what);
  if (rows == 0) return ok();
  if (!q || !out || !workspace || !keys->indices) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (!aligned(q, 16) || q_row_stride % 8 || q_head_stride % 8 || !aligned(out, 16) || out_row_stride % 8 ||
      out_head_stride % 8)
    return fail(XT_EINVAL, "%s: q and out rows must be 16-byte aligned (strides in elements: multiples of 8)", what);
  if (keys->topk < 0 || (extra_keys && extra_keys->topk < 0)) return fail(XT_EINVAL, "%s: negative topk", what);
  const bool extra = extra_cache && extra_keys && extra_keys->indices && extra_keys->topk > 0;
  MlaArgs a;
  int64_t ps, ss, rs;
  int st = check_cache(what, cache, &ps, &ss, &rs);
  if (st != XT_OK) return st;
  a.c[0] = CacheDev{cache->pay, cache->scales, static_cast<const uint16_t*>(cache->rope), cache->g, cache->slots,
                    (uint32_t)ps, (uint32_t)ss, (uint32_t)rs};
  if (extra) {
    st = check_cache(what, extra_cache, &ps, &ss, &rs);
    if (st != XT_OK) return st;
    a.c[1] = CacheDev{extra_cache->pay, extra_cache->scales, static_cast<const uint16_t*>(extra_cache->rope),
                      extra_cache->g, extra_cache->slots, (uint32_t)ps, (uint32_t)ss, (uint32_t)rs};
  } else {
    a.c[1] = a.c[0];
  }
  const size_t need = xt_sparse_mla_workspace_bytes(rows, heads, splits);
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
  const size_t lds_bytes = (size_t)kKTile + kVTile + kQTile + (size_t)a.steps * kMSteps * 4;
  if (lds_bytes > 160 * 1024 - 256)
    return fail(XT_EUNSUPPORTED, "%s: %d keys per split need %zu bytes of LDS; use more splits", what,
                a.keys_per_split, lds_bytes);
  a.part = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + kCounterBytes);
  a.ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes + (size_t)rows * splits * heads * kDl * 2);
  const int64_t n_units = (int64_t)rows * splits;
  if (n_units > 0x7FFFFFFFLL) return fail(XT_EUNSUPPORTED, "%s: %lld workgroups", what, (long long)n_units);
  a.xcd_units = (uint32_t)(n_units / 8);
  a.xcd_extra = (uint32_t)(n_units % 8);
  // dynamic LDS above 64 KB must be allowed per kernel; raised to the largest size asked for so far
  static size_t lds_allowed[2] = {64 * 1024, 64 * 1024};
  const void* fn = extra ? reinterpret_cast<const void*>(&mla_kernel<true>)
                         : reinterpret_cast<const void*>(&mla_kernel<false>);
  if (lds_bytes > lds_allowed[extra]) {
    const hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
    if (err != hipSuccess)
      return fail(XT_ELAUNCH, "%s: could not allow %zu bytes of LDS: %s", what, lds_bytes, hipGetErrorString(err));
    lds_allowed[extra] = lds_bytes;
  }
  if (extra)
    hipLaunchKernelGGL(mla_kernel<true>, dim3((unsigned)n_units), dim3(64 * kMWaves), lds_bytes,
                       reinterpret_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(mla_kernel<false>, dim3((unsigned)n_units), dim3(64 * kMWaves), lds_bytes,
                       reinterpret_cast<hipStream_t>(stream), a);
  if (splits > 1) {
    const int64_t threads = (int64_t)rows * heads * 64;
    hipLaunchKernelGGL(mla_merge_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), a, rows);
  }
  return check_launch(what);
}
