"""CPU oracle for the NVFP4-KV sparse-attention path: test infrastructure, not product code.

A numpy restatement of the reference's algorithms (each function cites the reference file:line it follows). Only the
test suite, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import this package, and only to
compare against or to time as a CPU baseline; the library under ``xtier_amd`` never calls into it.

Pinning (what each function is checked against, in ``tests/``):
- ``nvfp4.e2m1_*``: the 16-entry table the reference's tests hold (tests/draft_bf16_check.py:25,
  tests/fp4_decode_check.py:15), exhaustively over all 256 bytes.
- ``nvfp4.e4m3_decode``: torch's float8_e4m3fn values for all 256 bytes (the method of tests/fp8_decode_check.py).
- ``nvfp4.e4m3_encode``: torch's float8_e4m3fn cast (reference semantics) and the satfinite variant on the grid of
  tests/fp8_encode_check.py (every top-20-bit pattern and its halfway neighbours, plus the edge list).
- ``nvfp4.nvfp4_encode`` / ``quantize_blocks``: brute-force nearest-value search with the ties-to-lower rule, the
  one-block-scale round-trip bound of tests/draft_bf16_check.py:41-44, torch.bucketize on the same quotients, and
  special cases (zero blocks, exact midpoints, negative values rounding to zero).
- ``attention.*``: float64 softmax computed directly (no online/split form), single-key and empty-row special
  cases, split-K merge against one pass.
- ``attention.pack_qsa``: torch's own dequantization of the whole pool (float8_e4m3fn scales, the E2M1 table, low
  nibble first), then indexed; the decode gather with every position listed; a one-byte nibble-order case.
- ``attention.flash_precision_attention``: a torch FP32 restatement of tests/qsa_decode_check.py:29-45 and a
  two-key known answer where P rounded to BF16 and P kept in FP32 give different outputs.
- ``attention.block_sparse_decode`` LSE: torch.logsumexp of the scaled scores over the expanded positions.
- ``attention.block_sparse_decode`` / ``block_sparse_prefill``: the token-granular ``sparse_decode`` on the expanded
  block lists (with each query's position as the causal limit for the prefill); with every block listed, dense causal
  softmax over the copied context.
- ``attention.dequantize_context``: the NVFP4 dequantizer on each position's slot bytes.
- ``attention.sparse_mla`` / ``sparse_mla_v4`` / ``v4_keys``: float64 reference with sink and LSE, as
  tests/ds_sparse_mla_check.py:44-67; V4 page decoding against the exact keys of its packing rule.
- ``topk.topk_rows``: brute force over (value, position) pairs with ties, masks, NaN and +inf; hand-worked ties.
- ``topk.qsa_indexer_logits``: a torch head loop in float64 and a hand-worked case where ReLU after the head sum
  would change the answer.
- ``topk.dsa_mqa_logits``: the reference's einsum formula (indexer_torch.py:28-45) in torch float64 and a scalar loop
  over one element.
- ``topk.dsa_paged_mqa_logits``: equal to ``dsa_mqa_logits`` on the keys gathered page by page.
- ``topk.minimax_block_scores_decode`` / ``_prefill``: per-block brute force over keys read through the 16-entry
  E2M1 table (not the dequantizer), torch.logsumexp for the LSE score, the forced init / local blocks with their
  precedence, the skip of requests with at most topk blocks, a negative slot against its wrapped value, and the
  64-row tile that bounds the blocks a prefill row gets.
"""
