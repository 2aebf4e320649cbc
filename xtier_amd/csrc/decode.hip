// Fused sparse GQA attention over the NVFP4 paged pool: gather through the page table, dequantize in registers,
// QK and PV on MFMA (v_mfma_f32_16x16x32_f16), online softmax in the exp2 domain, split-K partials, then a combine.
//
// Work unit = one wavefront: (query row, KV head, key split). A workgroup holds 4 units with the KV head fastest, so
// for 4 KV heads the 4 waves of a workgroup read the 4 adjacent 64-byte head rows of the same tokens.
//
// Numerics: e2m1 * e4m3 is exact in FP16 (at most 6 significant bits, magnitudes 2^-10 .. 2688), so K and V enter
// the MFMA exactly without their global scales; the query enters as FP16 of q * scale * log2(e); the K global scale
// multiplies the FP32 scores and the V global scale the final output. P is FP16 for the PV product, all sums FP32.
//
// Lane layouts (16x16x32 MFMA: A[i][k] = lane i + 16*(k/8), element k%8; B[k][j] = lane j + 16*(k/8), element k%8;
// C[i][j] = lane j + 16*(i/4), element i%4). With hl = lane % 16 and j = lane / 16:
//   QK: C = S^T [16 tokens x 16 heads]; A = K tile, lane (token hl, 16 payload bytes j*16..j*16+15 of the head row);
//       MFMA kk (0..3) contracts dword kk of those 16 bytes, i.e. d = 32j + 8kk + e; B = Q^T with the same d order.
//       So lane (hl, j) ends up with the scores of head hl for tokens 4j..4j+3 (tile 0) and 16+4j..16+4j+3 (tile 1).
//   PV: C = O^T [16 rows x 16 heads] where row c is payload dword c of the head row; MFMA i (0..7) takes nibble i of
//       every dword, i.e. d = 8c + i. A = V^T, lane (dword hl, the 8 tokens above); B = P^T, lane (head hl, the same 8
//       tokens in the same order). Lane (hl, j) ends up with O^T for head hl, d = 32j .. 32j+31.
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

constexpr int kDim = 128;            // head size (payload 64 bytes, 8 scale bytes per head row)
constexpr int kStep = 32;            // keys per step
constexpr int kWavesPerBlock = 4;

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
  int kv_heads, q_heads, group;
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
  float* part_acc;                   // [rows, splits, q_heads, kDim]
  float* part_ml;                    // [rows, splits, q_heads, 2]: running max (log2 domain), sum
};

struct StepData {
  uint4 kw[2];        // K payload: 16 bytes of token (16 * tile + hl)
  uint32_t ks[2];     // K scales: the 2 bytes for those 16 payload bytes
  uint32_t vw[8];     // V payload dword hl of tokens T(j)[e]
  uint32_t vs[8];     // V scale byte (block hl / 2) of the same tokens; 0 for invalid tokens
  uint32_t valid;     // bit e: token T(j)[e] is valid
};

// Token (within a step) of the e-th of the 8 tokens a lane of group j holds scores for.
__device__ inline int tok_of(int j, int e) { return (e < 4) ? (4 * j + e) : (16 + 4 * j + (e - 4)); }

__device__ inline void load_step(const DecodeArgs& a, const int32_t* __restrict__ lds_slots, int step, int kvh,
                                 int hl, int j, StepData& d) {
  const int64_t row_bytes = (int64_t)a.kv_heads * (kDim / 2);
  const int64_t row_scales = (int64_t)a.kv_heads * (kDim / 16);
  const uint8_t* kp = a.k_pay + (int64_t)kvh * (kDim / 2);
  const uint8_t* vp = a.v_pay + (int64_t)kvh * (kDim / 2);
  const uint8_t* ksf = a.k_sf + (int64_t)kvh * (kDim / 16);
  const uint8_t* vsf = a.v_sf + (int64_t)kvh * (kDim / 16);
  const int base = step * kStep;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int32_t s = lds_slots[base + 16 * tt + hl];
    const int64_t slot = s < 0 ? 0 : s;
    d.kw[tt] = *reinterpret_cast<const uint4*>(kp + slot * row_bytes + 16 * j);
    d.ks[tt] = *reinterpret_cast<const uint16_t*>(ksf + slot * row_scales + 2 * j);
  }
  d.valid = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int32_t s = lds_slots[base + tok_of(j, e)];
    const int64_t slot = s < 0 ? 0 : s;
    d.vw[e] = *reinterpret_cast<const uint32_t*>(vp + slot * row_bytes + 4 * hl);
    const uint32_t sb = vsf[slot * row_scales + (hl >> 1)];
    d.vs[e] = s < 0 ? 0u : sb;
    d.valid |= (s >= 0 ? 1u : 0u) << e;
  }
}

__device__ inline half8_t dequant_k(uint32_t w, half2_t sc) {
  const half2_t p0 = fp4x2_to_f16<0>(w) * sc;
  const half2_t p1 = fp4x2_to_f16<1>(w) * sc;
  const half2_t p2 = fp4x2_to_f16<2>(w) * sc;
  const half2_t p3 = fp4x2_to_f16<3>(w) * sc;
  return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

__global__ void __launch_bounds__(256) decode_split_kernel(const DecodeArgs a) {
  extern __shared__ int32_t lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hl = lane & 15, j = lane >> 4;
  const int64_t unit = (int64_t)blockIdx.x * kWavesPerBlock + wave;
  const int64_t n_units = (int64_t)a.rows * a.kv_heads * a.splits;
  if (unit >= n_units) return;   // the whole wave leaves; no workgroup barrier is used below
  const int kvh = (int)(unit % a.kv_heads);
  const int split = (int)((unit / a.kv_heads) % a.splits);
  const int row = (int)(unit / ((int64_t)a.kv_heads * a.splits));
  int32_t* slots = lds + wave * (a.keys_per_split + kStep);

  // 1. slots of this unit's keys into LDS (-1: invalid)
  const int count = a.counts ? min(a.counts[row], a.topk) : a.topk;
  const int t0 = split * a.keys_per_split;
  const int t1 = min(t0 + a.keys_per_split, count);
  const int n = max(0, t1 - t0);
  const int32_t seqlen = a.seq_lens[row];
  const int32_t qpos = a.query_pos ? a.query_pos[row] : 0x7FFFFFFF;
  const int64_t trow = a.row_req ? a.row_req[row] : row;
  const int32_t* trow_ptr = a.table + trow * a.table_stride;
  const int steps = (n + kStep - 1) / kStep;
  for (int i = lane; i < steps * kStep; i += 64) {
    int32_t slot = -1;
    if (i < n) {
      const int32_t pos = a.indices[(int64_t)row * a.idx_stride + t0 + i];
      if (pos >= 0 && pos < seqlen && pos <= qpos) {
        int64_t s;
        if (a.page_size == 1)
          s = trow_ptr[pos];
        else
          s = (int64_t)trow_ptr[pos / a.page_size] * a.page_size + pos % a.page_size;
        if (s >= 0 && s < a.pool_slots) slot = (int32_t)s;
      }
    }
    slots[i] = slot;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

  // 2. query: B operand of the 4 QK MFMAs, FP16 of q * scale * log2(e); heads beyond the group are zero
  half8_t qb[4];
  {
    const bool hv = hl < a.group;
    const int head = kvh * a.group + (hv ? hl : 0);
    const uint16_t* qp = a.q + (int64_t)row * a.q_rs + (int64_t)head * a.q_hs;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (hv) w = *reinterpret_cast<const uint4*>(qp + 32 * j + 8 * kk);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qb[kk][2 * e] = (_Float16)(bf16_bits_to_f32(ws[e] & 0xFFFFu) * a.qscale);
        qb[kk][2 * e + 1] = (_Float16)(bf16_bits_to_f32(ws[e] >> 16) * a.qscale);
      }
    }
  }
  const float gk = *a.gk;

  float m_run = -__builtin_inff();
  float l_run = 0.0f;
  float4_t acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};

  StepData cur;
  if (steps > 0) load_step(a, slots, 0, kvh, hl, j, cur);
  for (int st = 0; st < steps; ++st) {
    StepData nxt;
    if (st + 1 < steps) load_step(a, slots, st + 1, kvh, hl, j, nxt);

    // QK: S^T tiles for tokens 0..15 and 16..31 of the step
    float4_t s[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const half2_t sc2 = fp8x2_to_f16<false>(cur.ks[tt]);
      const half2_t sc_lo = half2_t{sc2.x, sc2.x}, sc_hi = half2_t{sc2.y, sc2.y};
      const uint32_t w[4] = {cur.kw[tt].x, cur.kw[tt].y, cur.kw[tt].z, cur.kw[tt].w};
      s[tt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(dequant_k(w[kk], kk < 2 ? sc_lo : sc_hi), qb[kk], s[tt], 0,
                                                       0, 0);
    }
    // online softmax (log2 domain): scores of head hl for tokens T(j)[0..7]
    float sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = s[e >> 2][e & 3] * gk;
      sv[e] = ((cur.valid >> e) & 1u) ? x : -__builtin_inff();
    }
    float mt = sv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mt = fmaxf(mt, sv[e]);
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float p[8];
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = __builtin_amdgcn_exp2f(sv[e] - m_use);
      psum += p[e];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
    const half8_t pb = half8_t{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
                               (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
    // V^T operands: for tokens (e, e+1) build bytes (nibble of token e, same nibble of token e+1)
    half8_t av[8];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const uint32_t w0 = cur.vw[e], w1 = cur.vw[e + 1];
      const uint32_t lo = (w0 & 0x0F0F0F0Fu) | ((w1 & 0x0F0F0F0Fu) << 4);
      const uint32_t hi = ((w0 >> 4) & 0x0F0F0F0Fu) | (w1 & 0xF0F0F0F0u);
      const half2_t sp = fp8x2_to_f16<false>(cur.vs[e] | (cur.vs[e + 1] << 8));
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
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], pb, acc[i], 0, 0, 0);
    cur = nxt;
  }

  // 3. partials: the 4 lanes of a head hold disjoint token subsets of l; acc is already complete per lane
  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot += __shfl_xor(l_tot, 32);
  if (hl < a.group) {
    const int head = kvh * a.group + hl;
    const int64_t at = ((int64_t)row * a.splits + split) * a.q_heads + head;
    float* dst = a.part_acc + at * kDim + 32 * j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      reinterpret_cast<float4_t*>(dst + 8 * r)[0] = float4_t{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
      reinterpret_cast<float4_t*>(dst + 8 * r)[1] = float4_t{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
    }
    if (j == 0) reinterpret_cast<float2_t*>(a.part_ml)[at] = float2_t{m_run, l_tot};
  }
}

// One wave per (row, head): merge the splits in FP32 (weights 2^(m - max m); a row without keys gives 0), apply the
// V global scale, write the output and the natural log-sum-exp.
__global__ void __launch_bounds__(256) decode_combine_kernel(const float* __restrict__ part_acc,
                                                             const float* __restrict__ part_ml, int rows, int q_heads,
                                                             int splits, const float* __restrict__ gv,
                                                             uint16_t* __restrict__ out, int64_t o_rs, int64_t o_hs,
                                                             int out_dtype, float* __restrict__ lse) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (unit >= (int64_t)rows * q_heads) return;
  const int head = (int)(unit % q_heads);
  const int row = (int)(unit / q_heads);
  const float2_t* ml = reinterpret_cast<const float2_t*>(part_ml);
  float top = -__builtin_inff();
  for (int s = 0; s < splits; ++s) top = fmaxf(top, ml[((int64_t)row * splits + s) * q_heads + head].x);
  const float top_use = (top == -__builtin_inff()) ? 0.0f : top;
  float total = 0.0f;
  float2_t o = float2_t{0.f, 0.f};
  for (int s = 0; s < splits; ++s) {
    const int64_t at = ((int64_t)row * splits + s) * q_heads + head;
    const float2_t v = ml[at];
    const float w = __builtin_amdgcn_exp2f(v.x - top_use);
    total += w * v.y;
    const float2_t x = reinterpret_cast<const float2_t*>(part_acc + at * kDim)[lane];
    o += w * x;
  }
  const float g = *gv;
  const float inv = total > 0.0f ? g / total : 0.0f;
  const float a0 = o.x * inv, a1 = o.y * inv;
  uint32_t packed;
  if (out_dtype == XT_DTYPE_BF16)
    packed = f32_to_bf16_bits(a0) | (f32_to_bf16_bits(a1) << 16);
  else
    packed = f32_to_f16_bits(a0) | (f32_to_f16_bits(a1) << 16);
  reinterpret_cast<uint32_t*>(out + (int64_t)row * o_rs + (int64_t)head * o_hs)[lane] = packed;
  if (lse && lane == 0)
    lse[unit] = total > 0.0f ? (top_use + __builtin_log2f(total)) * kLn2 : -__builtin_inff();
}

}  // namespace
}  // namespace xt

using namespace xt;

extern "C" size_t xt_sparse_decode_workspace_bytes(int rows, int q_heads, int dim, int splits) {
  if (rows < 0 || q_heads <= 0 || dim <= 0 || splits <= 0) return 0;
  const size_t units = (size_t)rows * splits * q_heads;
  return units * (size_t)(dim + 2) * sizeof(float) + 256;
}

extern "C" int xt_sparse_decode_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                                      const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales,
                                      const uint8_t* v_scales, const float* gk, const float* gv, int64_t pool_slots,
                                      int kv_heads, int q_heads, int dim, const int32_t* table, int64_t table_stride,
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
  if (!aligned(k_pay, 16) || !aligned(v_pay, 16) || !aligned(k_scales, 2) || !aligned(v_scales, 2))
    return fail(XT_EINVAL, "%s: payload must be 16-byte and scales 2-byte aligned", what);
  if (lse && !aligned(lse, 4)) return fail(XT_EINVAL, "%s: lse must be 4-byte aligned", what);
  const size_t need = xt_sparse_decode_workspace_bytes(rows, q_heads, dim, splits);
  if (workspace_bytes < need)
    return fail(XT_EWORKSPACE, "%s: workspace %zu bytes < %zu needed", what, workspace_bytes, need);
  if (!aligned(workspace, 16)) return fail(XT_EINVAL, "%s: workspace must be 16-byte aligned", what);
  const int per_split = (topk + splits - 1) / splits;
  const int kps = ((per_split + kStep - 1) / kStep) * kStep;
  const size_t lds_bytes = (size_t)kWavesPerBlock * (kps + kStep) * sizeof(int32_t);
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
  a.kv_heads = kv_heads;
  a.q_heads = q_heads;
  a.group = group;
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
  char* ws = static_cast<char*>(workspace);
  const size_t units = (size_t)rows * splits * q_heads;
  a.part_acc = reinterpret_cast<float*>(ws);
  a.part_ml = reinterpret_cast<float*>(ws + units * kDim * sizeof(float));

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t waves = (int64_t)rows * kv_heads * splits;
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(decode_split_kernel, dim3((unsigned)blocks), dim3(64 * kWavesPerBlock), lds_bytes, s, a);
  if (int e = check_launch(what)) return e;
  const int64_t cwaves = (int64_t)rows * q_heads;
  hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)((cwaves + kWavesPerBlock - 1) / kWavesPerBlock)),
                     dim3(64 * kWavesPerBlock), 0, s, a.part_acc, a.part_ml, rows, q_heads, splits, gv,
                     static_cast<uint16_t*>(out), out_row_stride, out_head_stride, out_dtype, lse);
  return check_launch(what);
}
