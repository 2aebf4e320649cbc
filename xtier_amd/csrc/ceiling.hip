// Ceilings the kernels' roofline fractions are read against: what this GPU sustains on the two resources the attention
// kernels are bound by, measured with nothing else in the way.
//   MFMA: v_mfma_f32_32x32x16_f16 back to back from registers, four independent accumulators per wavefront, several
//         wavefronts per SIMD (a launch of 4 workgroups of 4 wavefronts per CU; one wavefront alone does not keep the
//         matrix core busy).
//   Gather: the fused decode's exact HBM access pattern, whole slot records at page-table positions of per-row index
//           lists, with no dequantization or math: the bytes arrive and are folded into one word per thread.
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

}  // namespace
}  // namespace xt

using namespace xt;

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
