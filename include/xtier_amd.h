/* C ABI of libxtier_amd.so: sparse attention over an NVFP4 paged KV pool on AMD Instinct MI355X (gfx950).
 *
 * Every entry point takes raw device pointers, element strides and sizes, runs on the caller's HIP stream, allocates
 * nothing, never synchronizes and copies nothing between host and device, so a call can be captured in a HIP graph.
 * Buffers are caller-owned; outputs are written in place. Return value: XT_OK or a negative status; the text of the
 * last error of the calling thread is in xt_last_error().
 *
 * Pool layout (SGLang's NVFP4 KV pool as the reference reads it, xtier/packs/qwen4_exp/qsa_fp4.py:43-58, :94-101):
 *   payload  uint8 [slots, kv_heads, dim / 2]   byte i of a head row = element 2i (bits 0-3), element 2i+1 (bits 4-7)
 *   scales   uint8 [slots, kv_heads, dim / 16]  OCP E4M3, one per 16 elements
 *   global   float [1] on the device            value = (e2m1 * e4m3) * global
 * pay_stride / sf_stride (bytes from one slot to the next; 0 = heads * the head stride) and, where an entry point takes
 * them, pay_head_stride / sf_head_stride (bytes from one KV head's row to the next within a slot; 0 = dim/2, dim/16)
 * also admit the interleaved pool of this library. Per slot it holds, for each KV head, that head's K payload row then
 * its V payload row, then for each KV head its K scales then its V scales. One key's K and V are then one contiguous
 * record (576 bytes at 4 heads x 128), and a head's K and V payload (128 bytes) are adjacent.
 * Slot lookup: page_size 1 -> table is token-granular (SGLang req_to_token, qsa_fp4.py:135);
 *              page_size P > 1 -> table holds page ids, slot = table[pos / P] * P + pos % P.
 */
#ifndef XTIER_AMD_H
#define XTIER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XT_OK 0
#define XT_EINVAL (-1)       /* bad shape, stride, alignment or pointer: the reference raises ValueError */
#define XT_EUNSUPPORTED (-2) /* shape the kernels do not cover: the reference raises NotImplementedError */
#define XT_ELAUNCH (-3)      /* the HIP launch failed */
#define XT_EWORKSPACE (-4)   /* workspace smaller than the *_workspace_bytes query returned */

#define XT_DTYPE_BF16 0
#define XT_DTYPE_F16 1

typedef struct ihipStream_t* xt_stream_t; /* hipStream_t; 0 = the null stream */

/* Library version (major * 10000 + minor * 100 + patch). */
int xt_version(void);

/* Text of the last error returned to the calling thread ("" if none). */
const char* xt_last_error(void);

/* --- NVFP4 quantization --------------------------------------------------------------------------------------- */

/* Per-tensor global scale of the reference quantizer, on the device: g = max(amax(|src|) / (6 * 448), 1e-12) in FP32
 * (xtier/backend/formats.py:122). src: BF16 [n_rows, heads, dim] with element strides src_row_stride and
 * src_head_stride (last dim contiguous). workspace: at least 4 bytes of device memory (an atomic maximum).
 * Replaces the global-scale half of nvfp4_encode (formats.py:114-128). */
int xt_nvfp4_global_scale(const void* src, int64_t n_rows, int heads, int dim, int64_t src_row_stride,
                          int64_t src_head_stride, float* g_out, void* workspace, xt_stream_t stream);

/* NVFP4 quantize-on-append: row r of src (BF16 [n_rows, heads, dim], strided as above, 16-byte aligned rows) is
 * quantized with the device global scale *g and written to pool slot slots[r] (payload [pool_slots, heads, dim/2],
 * scales [pool_slots, heads, dim/16]); a negative slot skips the row. Per 16-element block (formats.py:123-128):
 *   s = e4m3(blockamax / (6 * g)); q = x / max(s * g, 1e-30); code = nearest E2M1 magnitude of min(|q|, 6), a value
 *   on a midpoint taking the smaller one; sign bit when q < 0 and code > 0.
 * saturate = 0: a scale that rounds above 448 becomes E4M3 NaN, as the reference's torch cast (formats.py:124);
 * saturate = 1: it becomes 448 (the satfinite conversion of xtier/arch.py:57-75), so a row that exceeds a fixed
 * global scale never stores NaN. Pool strides as above (payload slot and head strides multiples of 8). The reference's
 * GPU write path is SGLang's quantizer behind the hook at xtier/packs/qwen4_exp/qsa_fp4.py:202-205 (fused store:
 * xtier/packs/minimax_m3/kv_fp4.py:546-559). */
int xt_nvfp4_quantize_append(const void* src, int64_t n_rows, int heads, int dim, int64_t src_row_stride,
                             int64_t src_head_stride, const int64_t* slots, const float* g, uint8_t* pay,
                             uint8_t* scales, int64_t pool_slots, int64_t pay_stride, int64_t sf_stride,
                             int64_t pay_head_stride, int64_t sf_head_stride, int saturate, xt_stream_t stream);

/* One tensor of a KV append (xt_nvfp4_store_kv): src BF16 [n_rows, heads, dim] (element strides; dim a multiple of 16,
 * 16-byte aligned rows) written to the pool at each row's slot s, the slot's page p = s / page_size and row
 * t = s % page_size: head h's payload at pay + p * pay_page_stride + t * pay_row_stride + h * pay_head_stride
 * (dim / 2 bytes) and its E4M3 scales at scales + p * sf_page_stride + t * sf_row_stride + h * sf_head_stride
 * (dim / 16 bytes), quantized with the device global scale *g as xt_nvfp4_quantize_append does. g == NULL stores the
 * BF16 values as they are (dim * 2 bytes at the payload address; scales unused): the rope rows of a latent cache.
 * Token-major pools: page_size 1 and the slot stride as the page stride. All strides in bytes. */
typedef struct {
  const void* src;
  int64_t src_row_stride, src_head_stride;
  int heads, dim;
  const float* g;
  uint8_t* pay;
  uint8_t* scales;
  int64_t pay_page_stride, pay_row_stride, pay_head_stride;
  int64_t sf_page_stride, sf_row_stride, sf_head_stride;
} xt_kv_store;

/* The fused KV-write epilogue: the n_stores (1..4) tensors of one append (K and V, plus the MiniMax index K or a latent
 * cache's rope rows) quantized and written at the same slots[n_rows] (int64; negative or >= pool_slots: skipped) in ONE
 * launch, bytes identical to one xt_nvfp4_quantize_append per tensor. page_size: rows per page, a power of 2 (1 for
 * token-major pools). Replaces SGLang's fused quantize + store that the MiniMax pack enables
 * (xtier/packs/minimax_m3/kv_fp4.py:546-559, nvfp4_store_kv_index as tests/minimax_kv_fp4_check.py:152-175 calls it)
 * and the per-buffer quantize of the QSA hook (xtier/packs/qwen4_exp/qsa_fp4.py:202-205). */
int xt_nvfp4_store_kv(const xt_kv_store* stores, int n_stores, int64_t n_rows, const int64_t* slots,
                      int64_t pool_slots, int page_size, int saturate, xt_stream_t stream);

/* --- QSA gather and pack (bit-exact BF16/FP16 rows) -------------------------------------------------------------- */

/* QSA decode/verify gather (xtier/packs/qwen4_exp/qsa_fp4.py:119-143, :174-180; hook extraction :223-228):
 * for request b < batch and column c of indices[b] (int32, row stride idx_stride, topk columns):
 *   pos = indices[b, c]; valid = c < cu_k[b+1] - cu_k[b] && 0 <= pos < seq_lens[b];
 *   slot = req_to_token[req_indices[b] * req_stride + pos];
 *   out[cu_k[b] + c, h, :] = dtype((e2m1 * e4m3) * g) for every head h (K with gk, V with gv).
 * zero_fill_cols = 0: only valid columns are written; > 0: every column below zero_fill_cols is written, invalid
 * ones as zeros. out_k / out_v: [rows, heads, dim] contiguous, out_dtype XT_DTYPE_BF16 or XT_DTYPE_F16. */
int xt_qsa_gather_nvfp4(const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales, const uint8_t* v_scales,
                        const float* gk, const float* gv, int64_t pool_slots, int heads, int dim,
                        const int32_t* req_to_token, int64_t req_stride, const int64_t* req_indices,
                        const int32_t* indices, int64_t idx_stride, const int32_t* seq_lens, const int32_t* cu_k,
                        void* out_k, void* out_v, int out_dtype, int batch, int topk, int zero_fill_cols,
                        xt_stream_t stream);

/* QSA prefill prefix packing (qsa_fp4.py:146-162, :183-192; hook pack_qsa_prefill_kv :216-220): request b's
 * positions t < cu_k[b+1] - cu_k[b] -> out[cu_k[b] + t] from slot req_to_token[req_indices[b] * sr0 + t * sr1]. */
int xt_qsa_pack_nvfp4(const uint8_t* k_pay, const uint8_t* v_pay, const uint8_t* k_scales, const uint8_t* v_scales,
                      const float* gk, const float* gv, int64_t pool_slots, int heads, int dim,
                      const int32_t* req_to_token, int64_t sr0, int64_t sr1, const int64_t* req_indices, int batch,
                      const int32_t* cu_k, int max_k, void* out_k, void* out_v, int out_dtype, xt_stream_t stream);

/* The QSA gather and prefix pack on an FP8 (E4M3) pool (the FP8 branch of qsa_fp4.py:104-116 and :160-162, checked by
 * tests/qsa_fp8_check.py): k / v are E4M3 bytes [pool_slots, heads, dim] with no block or global scale, and each value
 * is its plain E4M3 value (exact in BF16 and FP16). Arguments and layouts otherwise as xt_qsa_gather_nvfp4 /
 * xt_qsa_pack_nvfp4; K and V 8-byte aligned. */
int xt_qsa_gather_fp8(const uint8_t* k, const uint8_t* v, int64_t pool_slots, int heads, int dim,
                      const int32_t* req_to_token, int64_t req_stride, const int64_t* req_indices,
                      const int32_t* indices, int64_t idx_stride, const int32_t* seq_lens, const int32_t* cu_k,
                      void* out_k, void* out_v, int out_dtype, int batch, int topk, int zero_fill_cols,
                      xt_stream_t stream);
int xt_qsa_pack_fp8(const uint8_t* k, const uint8_t* v, int64_t pool_slots, int heads, int dim,
                    const int32_t* req_to_token, int64_t sr0, int64_t sr1, const int64_t* req_indices, int batch,
                    const int32_t* cu_k, int max_k, void* out_k, void* out_v, int out_dtype, xt_stream_t stream);

/* The packed-row layout of a decode gather (SGLang's qwen_sparse_fa2_cu_seqlens_triton as qsa_fp4.py:255-256 calls
 * it): valid_counts[b] = the number of indices[b, :topk] (row stride idx_stride) with 0 <= index < seq_lens[b], and
 * cu_seqlens_k [batch + 1] their running sum from 0. As in the reference, a row's valid indices are expected to come
 * first (top-k lists padded with -1 at the end). One workgroup on `stream`. */
int xt_qsa_valid_counts(const int32_t* seq_lens, const int32_t* indices, int64_t idx_stride, int batch, int topk,
                        int32_t* valid_counts, int32_t* cu_seqlens_k, xt_stream_t stream);

/* --- fused sparse attention over the NVFP4 pool ------------------------------------------------------------------ */

/* Device workspace the fused decode needs for `rows` query rows, q_heads heads of size dim and `splits` key splits
 * (split-K partials: running max, sum and the output normalized by the split's sum, in FP16, per row, split and head;
 * the size reserves room for FP32 outputs). 0 on a bad argument. */
size_t xt_sparse_decode_workspace_bytes(int rows, int q_heads, int dim, int splits);

/* Fused NVFP4 sparse GQA attention, one query per row (decode, verify, or a chunked prefill with one row per query
 * token). Replaces the QSA decode pipeline gather -> varlen attention (qsa_fp4.py:231-268 with qsa_decode.py:89-113)
 * and the MiniMax fused decode (xtier/packs/minimax_m3/kv_fp4.py:52-153, token-granular indices here).
 * Row r (q: [rows, q_heads, dim] BF16, strides q_row_stride / q_head_stride elements) attends to the keys at the
 * positions indices[r, c] (int32, row stride idx_stride, topk columns) that are valid:
 *   c < counts[r] (counts NULL: all topk columns), 0 <= pos < seq_lens[r], and pos <= query_pos[r] when query_pos is
 *   not NULL (causal prefill);
 * resolved to pool slots through table row row_req[r] (row_req NULL: row r) with the page_size rule above.
 * K/V are dequantized in registers; out[r, h] = sum_k softmax_k(q.k * scale) v_k in the dtype out_dtype, a row
 * without valid keys writing 0. Any finite BF16 query is taken exactly: each head's query enters the FP16 MFMA as
 * q * 2^-e, with 2^e from the head's largest magnitude, and scale * log2(e) * 2^e multiplies the FP32 scores. lse (optional, FP32 [rows, q_heads]): natural log-sum-exp of the scaled scores,
 * -inf for an empty row. q_heads must be a multiple of kv_heads with q_heads / kv_heads <= 16; dim 64, 128 or 256. Pool
 * pointers and strides as above: payload 16-byte and scales 4-byte aligned.
 * splits: key splits per row (1..64); workspace: xt_sparse_decode_workspace_bytes(rows, q_heads, dim, splits) bytes,
 * 256-byte aligned. With splits > 1 it holds a fixed 64 KB region of arrival counters (one per row and KV head group,
 * rows * kv_heads <= 16384) followed by the split partials: zero-filled before its first use, the counters are left
 * zero by every call, so calls of any shape (and sparse MLA calls) may share one workspace; calls that overlap in time
 * need separate workspaces. One launch on `stream`; a workgroup handles 4 KV heads of one (row, key split) when
 * rows * kv_heads / 4 * splits fills every CU, else 2 when rows * kv_heads / 2 * splits does, else 1, and with
 * splits > 1 the last workgroup of each (row, head group) to finish merges the split partials. */
int xt_sparse_decode_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride, const uint8_t* k_pay,
                           const uint8_t* v_pay, const uint8_t* k_scales, const uint8_t* v_scales, const float* gk,
                           const float* gv, int64_t pool_slots, int64_t pay_stride, int64_t sf_stride,
                           int64_t pay_head_stride, int64_t sf_head_stride, int kv_heads, int q_heads, int dim,
                           const int32_t* table, int64_t table_stride, int page_size, const int64_t* row_req,
                           const int32_t* indices, int64_t idx_stride, int topk, const int32_t* counts,
                           const int32_t* seq_lens, const int32_t* query_pos, float scale, void* out,
                           int64_t out_row_stride, int64_t out_head_stride, int out_dtype, float* lse, int rows,
                           int splits, void* workspace, size_t workspace_bytes, xt_stream_t stream);

/* No counterpart in the reference: xt_sparse_decode_nvfp4 for callers that cannot allocate device memory (code under
 * graph capture that must not grow a memory pool, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results without the workspace: it uses a fixed 8 MiB array in the library's device memory, one per
 * GPU, held until the process ends (64 KB of arrival counters, then the split partials), and calls no allocator. A
 * call whose xt_sparse_decode_workspace_bytes(rows, q_heads, dim, splits) exceeds 8 MiB fails with XT_EWORKSPACE.
 * Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU race (as two calls sharing a
 * workspace would). The first call on a device looks the array up and zeroes its counters on `stream`. */
int xt_sparse_decode_nvfp4_static(const void* q, int64_t q_row_stride, int64_t q_head_stride, const uint8_t* k_pay,
                                  const uint8_t* v_pay, const uint8_t* k_scales, const uint8_t* v_scales,
                                  const float* gk, const float* gv, int64_t pool_slots, int64_t pay_stride,
                                  int64_t sf_stride, int64_t pay_head_stride, int64_t sf_head_stride, int kv_heads,
                                  int q_heads, int dim, const int32_t* table, int64_t table_stride, int page_size,
                                  const int64_t* row_req, const int32_t* indices, int64_t idx_stride, int topk,
                                  const int32_t* counts, const int32_t* seq_lens, const int32_t* query_pos,
                                  float scale, void* out, int64_t out_row_stride, int64_t out_head_stride,
                                  int out_dtype, float* lse, int rows, int splits, xt_stream_t stream);

/* Block-sparse NVFP4 decode over head-major pages (the MiniMax cache layout; replaces
 * xtier/packs/minimax_m3/kv_fp4.py:119-153, fp4_sparse_decode, behind the hook _decode_main :579-590).
 * Pool: page p, KV head h, row t (t < block_size) holds payload at k_pay + p * page_stride + h * head_stride +
 * t * row_stride (dim/2 bytes) and E4M3 scales at k_scales + p * sf_page_stride + h * sf_head_stride + t *
 * sf_row_stride (dim/16 bytes), V alike; the buffers hold `pages` pages. No global scale: kv_scale multiplies the
 * scores and the output. Row b (q [rows, q_heads, dim] BF16) reads request slot_ids[b] (int64): its
 * length L = min(seq_lens[b], max_kv_len); KV head h's block ids topk_idx[h * idx_head_stride + b * idx_row_stride +
 * i] (int32, i < topk_blocks, -1: none) name positions c = id * block_size .. c + block_size - 1 below L, stored at
 * page s / block_size, rows s % block_size + n for s = req_to_token[slot_ids[b] * req_stride + c] (blocks start on a
 * page row, as the reference assumes; a block that starts mid-page continues on the next page here, where the
 * reference reads past the page). out[b, h'] = sum softmax(q.k * sm_scale * kv_scale) v * kv_scale over the query
 * heads h' of KV head h (natural exp, kv_fp4.py:100-113), 0 for a row without keys; lse (optional) as above.
 * Requirements: dim 64, 128 or 256, q_heads / kv_heads <= 16, block_size a power of 2, page_stride / row_stride ==
 * sf_page_stride / sf_row_stride >= block_size. splits and workspace as xt_sparse_decode_nvfp4 (workgroups hold one
 * KV head, so the arrival counters need rows * kv_heads <= 16384 when splits > 1). */
int xt_block_sparse_decode_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride, const uint8_t* k_pay,
                                 const uint8_t* v_pay, const uint8_t* k_scales, const uint8_t* v_scales,
                                 float kv_scale, int64_t pages, int kv_heads, int q_heads, int dim,
                                 int block_size, int64_t page_stride, int64_t head_stride, int64_t row_stride,
                                 int64_t sf_page_stride, int64_t sf_head_stride, int64_t sf_row_stride,
                                 const int32_t* req_to_token, int64_t req_stride, int max_kv_len,
                                 const int64_t* slot_ids, const int32_t* topk_idx, int64_t idx_head_stride,
                                 int64_t idx_row_stride, int topk_blocks, const int32_t* seq_lens, float sm_scale,
                                 void* out, int64_t out_row_stride, int64_t out_head_stride, int out_dtype, float* lse,
                                 int rows, int splits, void* workspace, size_t workspace_bytes, xt_stream_t stream);

/* Block-sparse NVFP4 prefill over head-major pages (replaces xtier/packs/minimax_m3/kv_fp4.py:293-366 and :369-404,
 * fp4_prefill_gqa_share_sparse, behind the hook _prefill_main :593-598). Pages, kv_scale and outputs as
 * xt_block_sparse_decode_nvfp4; one row per query token: row r reads request row_req[r] (int64), its block list
 * topk_idx[h * idx_head_stride + row_idx[r] * idx_row_stride + i] (row_idx: the query block of the row), and attends
 * to positions c = id * block_size .. + block_size - 1 below row_seq_lens[r] and at most row_query_pos[r] (causal,
 * kv_fp4.py:330-331, :345), each resolved through its own req_to_token entry (:338-340). */
int xt_block_sparse_prefill_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride, const uint8_t* k_pay,
                                  const uint8_t* v_pay, const uint8_t* k_scales, const uint8_t* v_scales,
                                  float kv_scale, int64_t pages, int kv_heads, int q_heads, int dim, int block_size,
                                  int64_t page_stride, int64_t head_stride, int64_t row_stride,
                                  int64_t sf_page_stride, int64_t sf_head_stride, int64_t sf_row_stride,
                                  const int32_t* req_to_token, int64_t req_stride, const int64_t* row_req,
                                  const int32_t* row_seq_lens, const int32_t* row_query_pos, const int32_t* topk_idx,
                                  int64_t idx_head_stride, int64_t idx_row_stride, int topk_blocks,
                                  const int32_t* row_idx, float sm_scale, void* out, int64_t out_row_stride,
                                  int64_t out_head_stride, int out_dtype, float* lse, int rows, int splits,
                                  void* workspace, size_t workspace_bytes, xt_stream_t stream);

/* BF16 copy of each request's context from head-major NVFP4 pages (replaces kv_fp4.py:496-530, dequantize_context):
 * for request b < batch and position pos < min(seq_lens[b], rows_per_req), token slot
 * s = req_to_token[sid * req_stride + pos] (sid = slot_ids[b]; both wrapped into [0, pages * block_size) as the
 * reference wraps them) -> out[b * rows_per_req + pos, h, :] (BF16 [batch * rows_per_req, heads, dim], contiguous)
 * = e2m1 * e4m3 of page s / block_size, row s % block_size (unit global scale, exact in BF16); other rows are left as
 * they are. Strides as xt_block_sparse_decode_nvfp4 (head strides may be 0 for the one-head index cache); dim and
 * block_size powers of 2, dim >= 32. */
int xt_dequantize_context_nvfp4(const uint8_t* pay, const uint8_t* scales, int64_t pages, int heads, int dim,
                                int block_size, int64_t page_stride, int64_t head_stride, int64_t row_stride,
                                int64_t sf_page_stride, int64_t sf_head_stride, int64_t sf_row_stride,
                                const int32_t* req_to_token, int64_t req_stride, const int64_t* slot_ids,
                                const int32_t* seq_lens, int batch, int rows_per_req, void* out, xt_stream_t stream);

/* --- split-K decode over packed BF16 rows ------------------------------------------------------------------------ */

/* Device workspace of xt_varlen_decode_bf16 for `rows` rows, `heads` query heads of size dim and `splits` key splits
 * (0 on a bad argument). */
size_t xt_varlen_decode_workspace_bytes(int rows, int heads, int dim, int splits);

/* Split-K GQA decode over packed BF16 K/V rows (replaces xtier/packs/qwen4_exp/qsa_decode.py:89-113, varlen_decode,
 * with its kernels _split :25-60 and _merge :63-86). Row r (< rows) has one query, q[cu_seqlens_q[r]] ([*, heads, dim]
 * BF16, element strides q_row_stride / q_head_stride), which attends to keys cu_seqlens_k[r] .. cu_seqlens_k[r+1]-1
 * of k / v ([keys, kv_heads, dim] BF16, element strides per key and per KV head); query head h reads KV head
 * h / (heads / kv_heads). Scores q.k in FP32 times softmax_scale * log2(e), exp2, P rounded to BF16 for the PV
 * product, FP32 sums; out[cu_seqlens_q[r], h] (out_dtype BF16 or FP16) = the normalized output, 0 for a row without
 * keys. dim 64, 128 or 256; heads / kv_heads <= 128; max_seqlen_k >= every row's key count (it sizes the splits).
 * splits 1..64, workspace xt_varlen_decode_workspace_bytes(...) bytes (256-byte aligned, zero before its first use,
 * left zero; the arrival counters are the fixed region the other decode entry points use, rows * kv_heads <= 16384
 * when splits > 1). One launch on `stream`. */
int xt_varlen_decode_bf16(const void* q, int64_t q_row_stride, int64_t q_head_stride, const void* k,
                          int64_t k_key_stride, int64_t k_head_stride, const void* v, int64_t v_key_stride,
                          int64_t v_head_stride, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int rows,
                          int heads, int kv_heads, int dim, int max_seqlen_k, float softmax_scale, void* out,
                          int64_t out_row_stride, int64_t out_head_stride, int out_dtype, int splits, void* workspace,
                          size_t workspace_bytes, xt_stream_t stream);

/* --- sparse MLA over an NVFP4 latent cache ------------------------------------------------------------------------ */

/* One latent cache: per slot a latent row of latent_dim NVFP4 values (payload latent_dim/2 bytes, E4M3 scales
 * latent_dim/16 bytes, global scale *g) and a rope row of rope_dim BF16 values. Strides are bytes from one slot to the
 * next (0 = packed: latent_dim/2, latent_dim/16, 2*rope_dim), so one 416-byte record per token
 * [payload 256 | scales 32 | rope 128] is pay = base, scales = base + 256, rope = base + 288, all strides 416. */
typedef struct {
  const uint8_t* pay;
  const uint8_t* scales;
  const void* rope;
  const float* g;
  int64_t slots;
  int64_t pay_stride, sf_stride, rope_stride;
} xt_mla_cache;

/* A key list: indices[r * stride + c] for c < topk are slots of the cache (-1: none); lengths[r] (NULL: topk)
 * limits the columns of row r. */
typedef struct {
  const int32_t* indices;
  int64_t stride;
  int topk;
  const int32_t* lengths;
} xt_mla_keys;

/* Device workspace of xt_sparse_mla_nvfp4 for `rows` rows, `heads` heads and `splits` key splits. */
size_t xt_sparse_mla_workspace_bytes(int rows, int heads, int splits);

/* Sparse MLA (DeepSeek-style; replaces sparse_mla / the hook flash_mla_with_kvcache of
 * xtier/packs/deepseek_v4/sparse_mla.py:167-231 on an NVFP4 latent cache). Row r of q (BF16 [rows, heads,
 * latent_dim + rope_dim], element strides q_row_stride / q_head_stride) attends to the valid keys of `keys` in `cache`
 * followed by those of `extra_keys` in `extra_cache` (both NULL: one list), key = [(e2m1 * e4m3) * g latent,
 * rope], value = the latent:
 *   out[r, h] = sum_k exp(s_k - m) v_k / (sum_k exp(s_k - m) + exp(sink[h] - m)),  s_k = scale * q[r, h] . key_k,
 * written in out_dtype to out (BF16/FP16 [rows, heads, latent_dim], strides in elements); sink NULL: no sink term.
 * lse (optional FP32 [rows, heads]): natural log of sum_k exp(s_k) over the keys only (sparse_mla.py:73-85); a row
 * without valid keys writes zeros and lse -inf. latent_dim 512, rope_dim 64, heads <= 128 are supported. The FP16
 * operands are exact: e2m1 * e4m3 latents and each head's query as q * 2^-e (2^e from its largest magnitude, so any
 * finite BF16 query fits); g multiplies the latent part of the FP32 scores and the normalized output (with two
 * caches the probabilities carry each key's g relative to the larger of the two).
 * splits: key splits per row (1..64); with splits > 1 a second launch on `stream` merges the split partials (FP16
 * outputs normalized per split before the global scale, so within FP16's range for any g).
 * workspace: xt_sparse_mla_workspace_bytes bytes, 256-byte aligned; its first 64 KB are left untouched (the counter
 * region of the decode entry points), so one zero-filled workspace may serve decode and MLA calls of any shape, one at
 * a time. */
int xt_sparse_mla_nvfp4(const void* q, int64_t q_row_stride, int64_t q_head_stride, int heads, int latent_dim,
                        int rope_dim, const xt_mla_cache* cache, const xt_mla_keys* keys,
                        const xt_mla_cache* extra_cache, const xt_mla_keys* extra_keys, const float* sink, float scale,
                        void* out, int64_t out_row_stride, int64_t out_head_stride, int out_dtype, float* lse, int rows,
                        int splits, void* workspace, size_t workspace_bytes, xt_stream_t stream);

/* DeepSeek V4 FP8 KV pages (the layout of xtier/packs/deepseek_v4/sparse_mla.py:38-59, 156-160): page p holds
 * page_size token data rows of 576 bytes (448 E4M3 latent values, then 64 BF16 rope values) followed by page_size
 * scale rows of 8 bytes (7 UE8M0 exponents, one per 64 latent values, value 2^(e - 127); 1 byte of padding); the
 * next page starts page_stride bytes later. Token t is row t % page_size of page t / page_size. */
typedef struct {
  const uint8_t* pages;
  int64_t num_pages;
  int page_size;          /* a power of 2 */
  int64_t page_stride;    /* bytes, >= page_size * 584, a multiple of 16 */
} xt_mla_fp8_cache;

/* Device workspace of xt_sparse_mla_fp8 (FP32 split partials). */
size_t xt_sparse_mla_fp8_workspace_bytes(int rows, int heads, int splits);

/* The most keys (both lists together) one key split of xt_sparse_mla_nvfp4 (fp8 = 0) or xt_sparse_mla_fp8 (fp8 = 1)
 * takes: its slot list shares the 160 KB of LDS with the key and query tiles, so rows * ceil(keys / this) splits is
 * the fewest a call may ask for. No counterpart in the reference (its kernels take any top-k). */
int xt_sparse_mla_max_split_keys(int fp8);

/* Sparse MLA on DeepSeek V4 FP8 pages (replaces sparse_mla / _attend / _merge of sparse_mla.py:88-217 and the hook
 * flash_mla_with_kvcache :220-231 on that layout). As xt_sparse_mla_nvfp4, with key = value = [e4m3 * 2^(e - 127)
 * (448), rope (64)], 512 wide, and q BF16 [rows, heads, 512]: scores are q . key on BF16 operands with FP32
 * accumulation, times scale; P is rounded to BF16 for the value product; splits merge in FP32. A scale byte of 0
 * (2^-127) reads as 0. */
int xt_sparse_mla_fp8(const void* q, int64_t q_row_stride, int64_t q_head_stride, int heads,
                      const xt_mla_fp8_cache* cache, const xt_mla_keys* keys, const xt_mla_fp8_cache* extra_cache,
                      const xt_mla_keys* extra_keys, const float* sink, float scale, void* out, int64_t out_row_stride,
                      int64_t out_head_stride, int out_dtype, float* lse, int rows, int splits, void* workspace,
                      size_t workspace_bytes, xt_stream_t stream);

/* --- Top-k producers: the indexer logits and the selection of each query's keys ----------------------------- */

/* Replaces qsa_prefill.qsa_mqa_prefill (xtier/packs/qwen4_exp/qsa_prefill.py:77-102, the kernel at :22-74 and the
 * mask SGLang applies after it): logits[r, n] = sum_h ReLU(q[r, h, :] . k[n, :]) / score_scale for start[r] <= n <
 * end[r], -inf elsewhere; FP32 [rows, ld] (columns 0 .. keys - 1 written). q [rows, heads, dim] and k [keys, dim]
 * (key row stride in elements) are BF16 or FP16 (dtype), products exact and summed in FP32; heads a power of 2 up to
 * 32, dim 64, 128 or 256; score_scale > 0 (the reference's default is sqrt(dim), applied by the caller). */
int xt_qsa_indexer_logits(const void* q, int64_t q_row_stride, int64_t q_head_stride, int rows, int heads, int dim,
                          const void* k, int64_t k_row_stride, int keys, const int32_t* starts, const int32_t* ends,
                          float score_scale, int dtype, float* logits, int64_t ld, xt_stream_t stream);

/* Replaces indexer_torch.fp8_mqa_logits (xtier/packs/glm5_next/indexer_torch.py:28-45, DeepGEMM's fp8_mqa_logits):
 * logits[q, n] = sum_h w[q, h] ReLU(q[q, h, :] . k[n, :]) * k_scale[n] for ks[q] <= n < ke[q] (ks / ke may be
 * NULL: all keys), else 0 (clean_logits 0) or -inf; FP32 [num_q, ld], columns 0 .. num_kv - 1 written. q [num_q,
 * heads, dim] and k [num_kv, dim] (k_row_stride bytes per key) are FP8 E4M3, products exact in FP32 and summed in
 * FP32; heads a multiple of 32 up to 128, dim 64, 128 or 256. */
int xt_dsa_mqa_logits(const void* q, int64_t q_row_stride, int64_t q_head_stride, int num_q, int heads, int dim,
                      const void* k, int64_t k_row_stride, const float* k_scale, int num_kv, const float* weights,
                      int64_t w_row_stride, const int32_t* ks, const int32_t* ke, int clean_logits, float* logits,
                      int64_t ld, xt_stream_t stream);

/* Replaces indexer_torch.fp8_paged_mqa_logits (indexer_torch.py:48-72, DeepGEMM's fp8_paged_mqa_logits; one query
 * per row): key t of row b is row t % block of page block_table[b, t / block] of the paged cache (num_pages pages
 * of page_bytes: block x dim E4M3 values, then block FP32 scales); logits [batch, ld] FP32, columns 0 .. max_seq_len
 * - 1 written, positions at or past context_lens[b], past the table or on a page past the cache 0 / -inf as for
 * xt_dsa_mqa_logits; a negative table entry reads page 0, as the reference's clamp does. */
int xt_dsa_paged_mqa_logits(const void* q, int64_t q_row_stride, int64_t q_head_stride, int batch, int heads, int dim,
                            const void* kvcache, int64_t num_pages, int64_t page_bytes, int block,
                            const int32_t* block_table,
                            int64_t bt_stride, int bt_width, const int32_t* context_lens, const float* weights,
                            int64_t w_row_stride, int max_seq_len, int clean_logits, float* logits, int64_t ld,
                            xt_stream_t stream);

/* The selection that turns logits into the index lists the attention entry points read (the int32 [batch, topk],
 * -1 padded format the reference's top-k producers hand to them, e.g. qsa_fp4.py:122 topk_indices): for each row of
 * x (FP32 [rows, ld], columns 0 .. cols - 1) the positions of the topk largest finite values in ascending order, ties
 * toward the lower position (-0 and +0 tie), -1 after the last (a row with fewer finite values than topk). out int32
 * [rows, out_ld]. Only columns 0 .. cols - 1 of a row are read; with cols == 0 nothing is read (x may be null) and
 * every entry is -1. */
int xt_topk_rows(const float* x, int64_t ld, int rows, int cols, int topk, int32_t* out, int64_t out_ld,
                 xt_stream_t stream);

/* MiniMax index block scores over the NVFP4 index pool (payload [pages, 128, dim/2], E4M3 scale bytes [pages, 128,
 * dim/16], byte strides of a page and a slot row; max_slots = pages * 128; slot s is page s / 128, row s % 128, and
 * slots and slot_ids wrap as (s + max_slots) % max_slots). The score of position p for head h is (q_h . k_p) *
 * score_factor, score_factor = (sm_scale * 1.4426950409) * k_scale in FP32; q BF16 / FP16 (q_dtype XT_DTYPE_*),
 * products exact and summed in FP32; dim 64, 128 or 256; block_size a multiple of 32 up to 256. req_to_token [reqs,
 * r2t_stride], seq_lens / slot_ids (and prefix_lens / cu_seqlens) are int32, or int64 where bit 0 (req_to_token),
 * 1 (seq_lens), 2 (slot_ids), 3 (prefix_lens), 4 (cu_seqlens) of index_int64 is set. Scores are written in
 * score_dtype (0 FP32, 1 BF16, 2 FP16) at the given element strides; entries not named below are left as they are.
 *
 * Replaces _fp4_decode_score_kernel (xtier/packs/minimax_m3/kv_fp4.py:168-222, launched in SGLang's
 * flash_decode_with_topk_idx through the shim at :225-244): scores[h, b, blk] for every head and block blk <
 * ceil(seq_lens[b] / block_size): the maximum (lse 0) or log2 of the sum of exp2 (lse 1; NaN -> -inf) of the block's
 * scores below seq_len; then 1e29 for the last local_blocks blocks, else 1e30 for the first init_blocks. A request
 * with at most skip_topk blocks (skip_topk >= 0) gets nothing. max_blocks_hint (any positive value is correct)
 * sizes the grid. */
int xt_minimax_decode_scores(const void* q, int64_t q_batch_stride, int64_t q_head_stride, int batch, int heads,
                             int dim, int q_dtype, const void* index_payload, int64_t pay_page_stride,
                             int64_t pay_slot_stride, const void* index_scales, int64_t sc_page_stride,
                             int64_t sc_slot_stride, int64_t max_slots, const void* req_to_token, int64_t r2t_stride,
                             const void* seq_lens, const void* slot_ids, int index_int64, int block_size,
                             float score_factor, int init_blocks, int local_blocks, int skip_topk, int lse,
                             void* scores, int score_dtype, int64_t s_head_stride, int64_t s_batch_stride,
                             int64_t s_block_stride, int max_blocks_hint, xt_stream_t stream);

/* Replaces _fp4_index_score_kernel (kv_fp4.py:407-446, launched in SGLang's flash_prefill_with_topk_index through
 * the shim at :449-472): q [total_q, heads, dim]; for query row t of request b (token cu_seqlens[b] + t, position
 * prefix_lens[b] + t) and every head, scores[h, cu_seqlens[b] + t, blk] = the maximum of the scores of the block's
 * positions at or before the row's position and below seq_len (-inf when none), for blk < ceil(min(seq_len,
 * prefix_len + 64 (t / 64 + 1)) / block_size). max_q_len bounds every request's query count. */
int xt_minimax_prefill_scores(const void* q, int64_t q_token_stride, int64_t q_head_stride, int batch, int heads,
                              int dim, int q_dtype, int max_q_len, const void* index_payload, int64_t pay_page_stride,
                              int64_t pay_slot_stride, const void* index_scales, int64_t sc_page_stride,
                              int64_t sc_slot_stride, int64_t max_slots, const void* req_to_token, int64_t r2t_stride,
                              const void* cu_seqlens, const void* seq_lens, const void* prefix_lens,
                              const void* slot_ids, int index_int64, int block_size, float score_factor, void* scores,
                              int score_dtype, int64_t s_head_stride, int64_t s_token_stride, int64_t s_block_stride,
                              xt_stream_t stream);

/* Self-test, no counterpart in the reference: the known-answer test of the hardware conversions the attention kernels
 * use (E4M3 -> FP16 from either half of a dword, two E2M1 codes -> FP16 / FP32 from each byte position, E4M3 with a
 * power-of-2 scale -> BF16), for every byte, written to `out` (xt_selftest_conversions_bytes() bytes, 16-byte
 * aligned) as laid out in xtier_amd/csrc/selftest.hip. The reference checks its own decodes the same way
 * (tests/fp4_decode_check.py:67-107, tests/fp8_decode_check.py:28-45). */
size_t xt_selftest_conversions_bytes(void);
int xt_selftest_conversions(void* out, xt_stream_t stream);

/* Ceilings, no counterpart in the reference: what this GPU sustains on the two resources the attention kernels are
 * bound by, for reading their roofline fractions.
 * xt_ceiling_mfma: `blocks` workgroups of 4 wavefronts, each running `iters` x 4 independent v_mfma_f32_32x32x16_f16
 * from registers (32768 flops each); out[blocks * 256] receives 64 * iters per thread (a result check).
 * xt_ceiling_gather: the fused decode's HBM access pattern alone: for each row of `batch` and each of its `topk`
 * positions (indices int32 [batch, topk]), the slot page_table[row, pos / page_size] * page_size + pos % page_size and
 * the whole `record_bytes`-byte record of it in `pool` (pool_records records), folded by XOR into one word per thread
 * of sink (xt_ceiling_gather_sink_words(batch, topk) words). Invalid positions, table entries and slots are skipped. */
int xt_ceiling_mfma(float* out, int iters, int blocks, xt_stream_t stream);
int xt_ceiling_gather(const void* pool, int64_t record_bytes, int64_t pool_records, const int32_t* page_table,
                      int64_t pt_stride, int page_size, int pt_width, const int32_t* indices, int batch, int topk,
                      uint32_t* sink, xt_stream_t stream);
size_t xt_ceiling_gather_sink_words(int batch, int topk);
/* xt_ceiling_gather_pieces: the same records read the way the fused decode reads them from the interleaved pool
 * (576-byte records of 4 KV heads x D = 128): one workgroup per (row, KV head, key split) numbered as the decode
 * numbers its units, each reading its head's 128 payload bytes and 16 scale bytes of every key of the split, in steps of
 * 32 keys per wavefront with four steps in flight. topk / splits must be a multiple of 256 up to 2048. sink receives
 * batch * 4 * splits * 512 words; the XOR of the 512 words of workgroup g is the XOR of the head pieces of its unit's
 * valid keys (unit of g: x * (n / 8) + min(x, n % 8) + g / 8 with x = g % 8, n = the number of workgroups). */
int xt_ceiling_gather_pieces(const void* pool, int64_t pool_records, const int32_t* page_table, int64_t pt_stride,
                             int page_size, int pt_width, const int32_t* indices, int batch, int topk, int kv_heads,
                             int splits, uint32_t* sink, xt_stream_t stream);
/* xt_ceiling_launch: an empty kernel of `blocks` workgroups of 512 threads: the cost of a launch with no work in it,
 * the floor under every short kernel of this library (no counterpart in the reference). */
int xt_ceiling_launch(int blocks, xt_stream_t stream);
/* xt_ceiling_split_merge: the split arrival of the decode kernels on its own (no counterpart in the reference): groups
 * of `splits` (2, 4 or 8) consecutive workgroups of 512 threads out of `blocks` (a multiple of splits); each writes
 * `bytes` (a multiple of 16) of partial into part (blocks * bytes, 16-byte aligned) as 16-byte words {offset, 1, 2, 3},
 * counts its arrival in counters[group] (int32, zero before the call and again after it), and the last of its group
 * reloads the group's partials and writes out[group * 512 + t] = splits * (sum of thread t's word offsets + their
 * number). fenced = 0: the protocol the kernels use (write-through stores, a system-scope count, cache-bypassing
 * reloads); fenced = 1: plain stores and loads with an agent-scope release fence before every count and an acquire
 * fence in the last arriver. */
int xt_ceiling_split_merge(void* part, int bytes, int32_t* counters, uint32_t* out, int splits, int blocks, int fenced,
                           xt_stream_t stream);
/* xt_clock_probe: the shader clock, read the way the benchmarks record it beside their rates (no counterpart in the
 * reference): one wavefront runs `iters` dependent FMAs between two reads of the core clock counter (s_memtime) and
 * of the constant 100 MHz clock (s_memrealtime); out[0] = core clock ticks, out[1] = 100 MHz ticks, out[2] = a check
 * word (uint64_t[3], device memory). MHz = 100 * out[0] / out[1]. */
int xt_clock_probe(uint64_t* out, int iters, xt_stream_t stream);
/* xt_decode_timeline: a per-wave timeline of the fused decode (no counterpart in the reference; for measurement).
 * With `stamps` (device memory, 8-byte aligned, `bytes` long) set, every later launch of the decode kernel
 * (xt_sparse_decode_nvfp4, its _static variant, the block decode and prefill) makes the first lane of each wavefront w
 * of workgroup g write 8 readings of the 100 MHz constant clock (s_memrealtime) to stamps[(g * waves + w) * 8 + i]:
 * i = 0 entry, 1 the split's slot list in LDS, 2 the first key step computed, 3 the main loop done, 4 the slices merged
 * in LDS, 5 the partials (or, with one split, the outputs) issued, 6 the arrival counted, 7 the last arriver's split
 * merge done; phases a wave does not reach read 0. Workgroups past bytes / (waves * 64) write nothing; waves is 8 for
 * decode batches that fit one round of workgroups, else 4. A process-wide setting; NULL turns it off (the default). */
int xt_decode_timeline(uint64_t* stamps, size_t bytes);
/* xt_mla_timeline: the same for the sparse MLA kernel (xt_sparse_mla_nvfp4, xt_sparse_mla_fp8; no counterpart in the
 * reference): 8 stamps per wavefront of its 8-wave workgroups, stamps[(g * 8 + w) * 8 + i], i = 0 entry, 1 the split's
 * slot list in LDS, 2 the query operands ready, 3 the first key tile dequantized, 4 the main loop done, 5 the outputs
 * (one split) or partials issued (waves without live heads: 0), 6 (one split) the outputs staged in LDS, before 5;
 * 7 reads 0. NULL turns it off (the default). */
int xt_mla_timeline(uint64_t* stamps, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* XTIER_AMD_H */
