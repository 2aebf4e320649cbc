// Ceilings the kernels' roofline fractions are read against: what this GPU sustains on the two resources the attention
// kernels are bound by, measured with nothing else in the way.
//   MFMA: v_mfma_f32_32x32x16_f16 back to back from registers, four independent accumulators per wavefront, several
//         wavefronts per SIMD (a launch of 4 workgroups of 4 wavefronts per CU; one wavefront alone does not keep the
//         matrix core busy).
//   Gather: the fused decode's HBM access pattern, slot records at page-table positions of per-row index lists, with
//           no dequantization or math: the bytes arrive and are folded into one word per thread. Two forms: whole
//           records per workgroup, and the decode's own decomposition (one KV head's pieces of each record per
//           workgroup, key splits, slices of 8 wavefronts, four steps of loads in flight).
//   Launch: an empty kernel, the floor under every short kernel; and the split arrival of the decode kernels on its
//           own (partials written through, the count, the last arriver's reload and merge), with the fenced form
//           beside it.
#include "xt_common.h"
#include "xt_host.h"

namespace xt {
namespace {

typedef float float16_t __attribute__((ext_vector_type(16)));

// A = B = all ones: every MFMA adds 16 to every accumulator element, so out = 64 * iters for every thread (exact in
// FP32 up to iters = 2^18).
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(float* out, int iters) {
  const half8_t one = half8_t{1, 1, 1, 1, 1, 1, 1, 1};
  float16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int i = 0; i < iters; ++i) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(one, one, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(one, one, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(one, one, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(one, one, c3, 0, 0, 0);
  }
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = c0[0] + c1[0] + c2[0] + c3[0];
}

constexpr int kGatherKeys = 256;   // keys per workgroup (8 wavefronts of 32 keys)

// Workgroup = (row, 256 keys); the keys' slots are resolved into LDS as the decode does (index -> page table entry),
// then wave w reads the records of keys 32w .. 32w+31 as one run of 32 * record / 16 granules, granule 64 r + lane in
// load r, so consecutive lanes read consecutive granules of a record. G granules per lane (G = record / 32: 18 for the
// 576-byte KV record) are all in flight before the first is used; other record sizes take the generic loop. Keys past
// topk, invalid positions and slots outside the pool are skipped.
template <int G>
__global__ __launch_bounds__(512) void gather_ceiling_kernel(const uint8_t* pool, int64_t record_bytes,
                                                             int64_t pool_records, const int32_t* page_table,
                                                             int64_t pt_stride, int page_size, int pt_width,
                                                             const int32_t* indices, int topk, uint32_t* sink) {
  __shared__ int32_t slots[kGatherKeys];
  const int chunks = (topk + kGatherKeys - 1) / kGatherKeys;
  const int row = blockIdx.x / chunks, k0 = (blockIdx.x % chunks) * kGatherKeys;
  if (threadIdx.x < kGatherKeys) {
    const int k = k0 + (int)threadIdx.x;
    int32_t slot = -1;
    if (k < topk) {
      const int32_t pos = indices[(int64_t)row * topk + k];
      if (pos >= 0 && pos / page_size < pt_width) {
        const int32_t ent = page_table[(int64_t)row * pt_stride + pos / page_size];
        const int64_t s = (int64_t)ent * page_size + pos % page_size;
        if (ent >= 0 && s < pool_records) slot = (int32_t)s;
      }
    }
    slots[threadIdx.x] = slot;
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int gpr = (int)(record_bytes / 16);   // granules per record
  uint32_t acc = 0;
  if constexpr (G > 0) {
    uint4 v[G];
#pragma unroll
    for (int r = 0; r < G; ++r) {
      const int g = 64 * r + lane, key = g / gpr, gi = g - key * gpr;
      const int32_t s = slots[32 * wave + key];
      v[r] = s >= 0 ? *reinterpret_cast<const uint4*>(pool + s * record_bytes + 16 * gi) : uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int r = 0; r < G; ++r) acc ^= v[r].x ^ v[r].y ^ v[r].z ^ v[r].w;
  } else {
    for (int g = lane; g < 32 * gpr; g += 64) {
      const int key = g / gpr, gi = g - key * gpr;
      const int32_t s = slots[32 * wave + key];
      if (s >= 0) {
        const uint4 v = *reinterpret_cast<const uint4*>(pool + s * record_bytes + 16 * gi);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
      }
    }
  }
  sink[(int64_t)blockIdx.x * 512 + threadIdx.x] = acc;
}

// The decode's own decomposition on the interleaved pool (576-byte records: per KV head h, K payload 64 B and V payload
// 64 B at 128 h, then per head 8 + 8 scale bytes at 512 + 16 h; 4 KV heads of D = 128). Workgroup = unit (row, KV
// head, key split), numbered as the decode numbers them (XCD x takes a contiguous unit range, so a row's heads and
// splits share one L2); its keys_per_split slots are resolved into LDS; wave w takes keys w * per_wave .. as steps of
// 32: lane (hl, j) reads 16 B of K and of V of keys hl and 16 + hl at byte 16 j of the head's pieces, and each lane
// pair the 16 scale bytes of key lane / 2, four steps in flight. Invalid keys read slot 0 and count as zero.
constexpr int kPieceMaxKeys = 2048;   // keys per split

__global__ __launch_bounds__(512) void gather_pieces_kernel(const uint8_t* pool, int64_t pool_records,
                                                            const int32_t* page_table, int64_t pt_stride,
                                                            int page_size, int pt_width, const int32_t* indices,
                                                            int topk, int kv_heads, int splits, uint32_t* sink) {
  __shared__ int32_t slots[kPieceMaxKeys];
  const uint32_t g = blockIdx.x, xcd = g & 7u, units = gridDim.x;
  const uint32_t u = xcd * (units / 8) + min(xcd, units % 8) + (g >> 3);
  const int split = (int)(u % (uint32_t)splits), head = (int)((u / splits) % (uint32_t)kv_heads);
  const int row = (int)(u / splits / kv_heads);
  const int kps = topk / splits, t0 = split * kps;
  for (int i = threadIdx.x; i < kps; i += 512) {
    const int32_t pos = indices[(int64_t)row * topk + t0 + i];
    int32_t slot = -1;
    if (pos >= 0 && pos / page_size < pt_width) {
      const int32_t ent = page_table[(int64_t)row * pt_stride + pos / page_size];
      const int64_t v = (int64_t)ent * page_size + pos % page_size;
      if (ent >= 0 && v < pool_records) slot = (int32_t)v;
    }
    slots[i] = slot;
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, hl = lane & 15, j = lane >> 4;
  const int per_wave = kps / 8, steps = per_wave / 32;
  const int32_t* ws = slots + wave * per_wave;
  const uint8_t* hp = pool + 128 * head + 16 * j;
  const uint8_t* sp = pool + 512 + 16 * head + 8 * (lane & 1);
  uint4 kv[4][4];
  uint2 sc[4];
  bool ok[4][3];
  auto load = [&](int st, int b) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int32_t s = ws[32 * st + 16 * tt + hl];
      ok[b][tt] = s >= 0;
      const int64_t off = (int64_t)(s < 0 ? 0 : s) * 576;
      kv[b][2 * tt] = *reinterpret_cast<const uint4*>(hp + off);
      kv[b][2 * tt + 1] = *reinterpret_cast<const uint4*>(hp + off + 64);
    }
    const int32_t s = ws[32 * st + (lane >> 1)];
    ok[b][2] = s >= 0;
    sc[b] = *reinterpret_cast<const uint2*>(sp + (int64_t)(s < 0 ? 0 : s) * 576);
  };
  uint32_t acc = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b)
    if (b < steps) load(b, b);
  for (int s0 = 0; s0 < steps; s0 += 4) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (s0 + b < steps) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t x = kv[b][q].x ^ kv[b][q].y ^ kv[b][q].z ^ kv[b][q].w;
          acc ^= ok[b][q >> 1] ? x : 0u;
        }
        acc ^= ok[b][2] ? (sc[b].x ^ sc[b].y) : 0u;
        if (s0 + b + 4 < steps) load(s0 + b + 4, b);
      }
    }
  }
  sink[(int64_t)g * 512 + threadIdx.x] = acc;
}

// An empty kernel: what a launch costs with no work in it (dispatch, wave launch, completion).
__global__ __launch_bounds__(512) void launch_ceiling_kernel() {}

// The split arrival of the decode kernels on its own, with their helpers (store_partial, arrive_last, load_partial):
// groups of S consecutive workgroups of 512 threads; each writes `bytes` of partial (16-byte words {offset, 1, 2, 3})
// written through, counts its arrival, and the last of its group reloads the group's S partials and sums them into
// one word per thread: out[group * 512 + t] = S * (sum of its word offsets + its word count). FENCED: the form with
// plain stores, an agent-scope release fence before every count and an acquire fence in the last arriver, then plain
// loads (the fences write back / invalidate the L2 instead of bypassing it per access).
template <int S, bool FENCED>
__global__ __launch_bounds__(512) void split_merge_kernel(uint8_t* part, int bytes, int32_t* counters, uint32_t* out) {
  const int grp = blockIdx.x / S;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(part + (int64_t)grp * S * bytes, (short)0, S * bytes, 0x00020000);
  const int mine = (blockIdx.x % S) * bytes;
  for (int o = threadIdx.x * 16; o < bytes; o += 512 * 16) {
    const float4_t v = {__uint_as_float((uint32_t)o), __uint_as_float(1u), __uint_as_float(2u), __uint_as_float(3u)};
    if (FENCED)
      __builtin_amdgcn_raw_buffer_store_b128(
          xt_u32x4_t{(uint32_t)o, 1u, 2u, 3u}, r, mine + o, 0, 0);
    else
      store_partial(r, mine + o, v);
  }
  __shared__ int flag;
  bool last;
  if (FENCED) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      flag = __hip_atomic_fetch_add(counters + grp, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
      if (flag) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    last = flag;
  } else {
    last = arrive_last(counters + grp, S, &flag);
  }
  if (!last) return;
  uint32_t sum0 = 0, sum1 = 0;
  for (int o = threadIdx.x * 16; o < bytes; o += 512 * 16) {
    xt_u32x4_t w[S];
#pragma unroll
    for (int k = 0; k < S; ++k) {
      if (FENCED) {
        w[k] = __builtin_amdgcn_raw_buffer_load_b128(r, k * bytes + o, 0, 0);
      } else {
        const float4_t f = load_partial(r, k * bytes + o);
        w[k] = xt_u32x4_t{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
      }
    }
#pragma unroll
    for (int k = 0; k < S; ++k) {
      sum0 += w[k][0];
      sum1 += w[k][1];
    }
  }
  out[grp * 512 + threadIdx.x] = sum0 + sum1;
  if (FENCED) {
    if (threadIdx.x == 0) __hip_atomic_store(counters + grp, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    reset_counter(counters + grp);
  }
}

// One wavefront: `iters` dependent FMAs between two reads of the core clock counter and the 100 MHz constant clock.
__global__ __launch_bounds__(64) void clock_probe_kernel(uint64_t* out, int iters) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  float x = (float)threadIdx.x;
  for (int i = 0; i < iters; ++i) x = __builtin_fmaf(x, 0.999999f, 1.0f);
  asm volatile("" : "+v"(x));
  const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = r1 - r0;
    out[2] = __float_as_uint(x);
  }
}

}  // namespace
}  // namespace xt

using namespace xt;

extern "C" int xt_clock_probe(uint64_t* out, int iters, xt_stream_t stream) {
  const char* what = "xt_clock_probe";
  if (!out || iters <= 0 || iters > (1 << 24)) return fail(XT_EINVAL, "%s: out must be given, iters in 1..2^24", what);
  hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), out, iters);
  return check_launch(what);
}

extern "C" int xt_ceiling_launch(int blocks, xt_stream_t stream) {
  const char* what = "xt_ceiling_launch";
  if (blocks <= 0 || blocks > (1 << 20)) return fail(XT_EINVAL, "%s: blocks in 1..2^20", what);
  hipLaunchKernelGGL(launch_ceiling_kernel, dim3((unsigned)blocks), dim3(512), 0, reinterpret_cast<hipStream_t>(stream));
  return check_launch(what);
}

template <int S>
static void launch_split_merge(int fenced, uint8_t* p, int bytes, int32_t* counters, uint32_t* out, int blocks,
                               hipStream_t st) {
  if (fenced)
    hipLaunchKernelGGL((split_merge_kernel<S, true>), dim3((unsigned)blocks), dim3(512), 0, st, p, bytes, counters, out);
  else
    hipLaunchKernelGGL((split_merge_kernel<S, false>), dim3((unsigned)blocks), dim3(512), 0, st, p, bytes, counters,
                       out);
}

extern "C" int xt_ceiling_split_merge(void* part, int bytes, int32_t* counters, uint32_t* out, int splits, int blocks,
                                      int fenced, xt_stream_t stream) {
  const char* what = "xt_ceiling_split_merge";
  if (!part || !counters || !out) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if ((splits != 2 && splits != 4 && splits != 8) || blocks <= 0 || blocks % splits || blocks > (1 << 16))
    return fail(XT_EINVAL, "%s: splits 2, 4 or 8; blocks a multiple of splits up to 2^16", what);
  if (bytes <= 0 || bytes % 16 || (int64_t)bytes * splits > (1 << 24) || !aligned(part, 16) || !aligned(counters, 4))
    return fail(XT_EINVAL, "%s: bytes a multiple of 16 with bytes * splits up to 2^24; 16-byte aligned part", what);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* p = static_cast<uint8_t*>(part);
  if (splits == 2) launch_split_merge<2>(fenced, p, bytes, counters, out, blocks, st);
  else if (splits == 4) launch_split_merge<4>(fenced, p, bytes, counters, out, blocks, st);
  else launch_split_merge<8>(fenced, p, bytes, counters, out, blocks, st);
  return check_launch(what);
}

extern "C" int xt_ceiling_mfma(float* out, int iters, int blocks, xt_stream_t stream) {
  const char* what = "xt_ceiling_mfma";
  if (!out || iters <= 0 || iters > (1 << 18) || blocks <= 0 || blocks > (1 << 20))
    return fail(XT_EINVAL, "%s: out must be given, iters in 1..2^18, blocks in 1..2^20", what);
  hipLaunchKernelGGL(mfma_ceiling_kernel, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     out, iters);
  return check_launch(what);
}

extern "C" int xt_ceiling_gather(const void* pool, int64_t record_bytes, int64_t pool_records,
                                 const int32_t* page_table, int64_t pt_stride, int page_size, int pt_width,
                                 const int32_t* indices, int batch, int topk, uint32_t* sink, xt_stream_t stream) {
  const char* what = "xt_ceiling_gather";
  if (batch < 0 || topk < 0) return fail(XT_EINVAL, "%s: negative batch or topk", what);
  if (batch == 0 || topk == 0) return ok();
  if (!pool || !page_table || !indices || !sink) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  if (record_bytes <= 0 || record_bytes % 16 || record_bytes > 4096 || !aligned(pool, 16))
    return fail(XT_EINVAL, "%s: records of %lld bytes (multiples of 16 up to 4096, 16-byte aligned pool)", what,
                (long long)record_bytes);
  if (pool_records <= 0 || page_size <= 0 || pt_width <= 0 || pt_stride < pt_width)
    return fail(XT_EINVAL, "%s: pool / page table sizes", what);
  const int64_t blocks = (int64_t)batch * ((topk + kGatherKeys - 1) / kGatherKeys);
  if (blocks > 0x7FFFFFFF) return fail(XT_EUNSUPPORTED, "%s: %lld workgroups", what, (long long)blocks);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* p = static_cast<const uint8_t*>(pool);
  if (record_bytes == 576)
    hipLaunchKernelGGL(gather_ceiling_kernel<18>, dim3((unsigned)blocks), dim3(512), 0, st, p, record_bytes,
                       pool_records, page_table, pt_stride, page_size, pt_width, indices, topk, sink);
  else
    hipLaunchKernelGGL(gather_ceiling_kernel<0>, dim3((unsigned)blocks), dim3(512), 0, st, p, record_bytes,
                       pool_records, page_table, pt_stride, page_size, pt_width, indices, topk, sink);
  return check_launch(what);
}

extern "C" size_t xt_ceiling_gather_sink_words(int batch, int topk) {
  if (batch <= 0 || topk <= 0) return 0;
  return (size_t)batch * ((topk + kGatherKeys - 1) / kGatherKeys) * 512;
}

extern "C" int xt_ceiling_gather_pieces(const void* pool, int64_t pool_records, const int32_t* page_table,
                                        int64_t pt_stride, int page_size, int pt_width, const int32_t* indices,
                                        int batch, int topk, int kv_heads, int splits, uint32_t* sink,
                                        xt_stream_t stream) {
  const char* what = "xt_ceiling_gather_pieces";
  if (batch < 0 || topk < 0 || kv_heads != 4 || splits < 1) return fail(XT_EINVAL, "%s: bad sizes", what);
  if (batch == 0 || topk == 0) return ok();
  if (!pool || !page_table || !indices || !sink) return fail(XT_EINVAL, "%s: a required pointer is null", what);
  const int kps = topk / splits;
  if (topk % splits || kps > kPieceMaxKeys || kps % 256)
    return fail(XT_EINVAL, "%s: keys per split %d must divide topk and be a multiple of 256 up to %d", what, kps,
                kPieceMaxKeys);
  if (!aligned(pool, 16) || pool_records <= 0 || page_size <= 0 || pt_width <= 0 || pt_stride < pt_width)
    return fail(XT_EINVAL, "%s: bad pool or page table", what);
  hipLaunchKernelGGL(gather_pieces_kernel, dim3((unsigned)(batch * kv_heads * splits)), dim3(512), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint8_t*>(pool), pool_records,
                     page_table, pt_stride, page_size, pt_width, indices, topk, kv_heads, splits, sink);
  return check_launch(what);
}
