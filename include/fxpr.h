/*
 * fxpr.h - C ABI of the MI355X (gfx950) fixed-point reduction kernels.
 *
 * Every entry point takes raw device pointers, element counts and strides,
 * launches asynchronously on the given HIP stream (a hipStream_t passed as
 * void*; NULL = the null stream), never allocates device memory and never
 * synchronises. Return value: 0 on success, a negative FXPR_E_* code when the
 * arguments are rejected before launch, or a positive hipError_t when the
 * launch itself failed. fxpr_error_string() turns either into text.
 *
 * Each function replaces the device half of one reference operator of the
 * `fxpr` torch.library namespace (fxpr_vllm/_lib.py:15-33 in
 * Gursukh/vLLM-Triton-Fixed-Point-Reductions); the citation above each
 * declaration names the Triton launcher and kernel it stands in for. The
 * Python side (fxpr_vllm/_lib.py of this package) keeps the reference's
 * schemas, validation and output allocation and calls these through ctypes.
 */
#ifndef FXPR_H
#define FXPR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
enum {
  FXPR_DTYPE_F16 = 0,
  FXPR_DTYPE_BF16 = 1,
  FXPR_DTYPE_F32 = 2,
  FXPR_DTYPE_F64 = 3,
  FXPR_DTYPE_I16 = 4,
  FXPR_DTYPE_I32 = 5,
  FXPR_DTYPE_I64 = 6
};

/* Negative return codes (argument errors, nothing was launched). */
enum {
  FXPR_OK = 0,
  FXPR_E_DTYPE = -1,     /* element type not supported by this entry point */
  FXPR_E_BITS = -2,      /* int_bits / frac_bits / float_bits out of range */
  FXPR_E_SHAPE = -3,     /* negative or inconsistent sizes */
  FXPR_E_WORKSPACE = -4, /* workspace missing or smaller than required */
  FXPR_E_ARG = -5,       /* any other invalid argument */
  FXPR_E_CAPTURE = -6    /* set-up that cannot run while the stream is capturing */
};

/* Text for a return code of any entry point (static storage). */
const char* fxpr_error_string(int code);

/* ABI revision of this header; bumped on any signature change. */
int fxpr_abi_version(void);

/*
 * q[i] = RNE_sat_b(fl32(x[i]) * 2^frac_bits), NaN -> 0.
 * x: f16 / f32 / f64 (f64 is rounded to f32 first), contiguous, n elements.
 * q: int16 / int32 / int64 for int_bits 16 / 32 / 64. frac_bits in [0, 63].
 * Replaces float_to_fixed_run + _float_to_fixed_kernel
 * (fxpr_vllm/_triton/casts.py:57-89, 21-37; fxp.py:92-108).
 */
int fxpr_float_to_fixed(const void* x, int x_dtype, void* q, int int_bits,
                        int frac_bits, int64_t n, void* stream);

/*
 * y[i] = OUT(fl32(q[i]) * 2^-frac_bits) with OUT = f16 / f32 / f64 for
 * float_bits 16 / 32 / 64 (f64 widens the fp32 value).
 * q: int16 / int32 / int64, contiguous, n elements.
 * Replaces fixed_to_float_run + _fixed_to_float_kernel
 * (fxpr_vllm/_triton/casts.py:92-126, 40-54; fxp.py:111-113).
 */
int fxpr_fixed_to_float(const void* q, int q_dtype, void* y, int float_bits,
                        int frac_bits, int64_t n, void* stream);

/*
 * out[r] = sat_b(sum_j q[r, j]) over a contiguous [rows, cols] integer
 * matrix: the sum is exact (64-bit for int16/int32 inputs, 128-bit for int64)
 * and saturated once into the int_bits range; out has int_bits width.
 * The reference has no kernel for this: it is the fixed-point sum its tests
 * perform with torch (fxpr_vllm/_tests/test_sum.py:12-16).
 */
int fxpr_fixed_row_sum(const void* q, int q_dtype, void* out, int int_bits,
                       int64_t rows, int64_t cols, void* stream);

/*
 * Deterministic RMSNorm over contiguous [rows, hidden] rows of x (f32, f16
 * or bf16; weight and y share that type), hidden <= 2^22. With residual !=
 * NULL the fused form runs: v = x + residual is written back into residual
 * (rounded to the I/O type) and normalised. The sum of squares is an exact
 * integer sum in a per-row block floating-point format: with 2^e <= max|v| <
 * 2^(e+1), T = sum_j RNE(fl32(ldexp(v_j, -e)^2) * 2^40) in 64 bits (cannot
 * overflow), mean_sq = ldexp(fl32(T) / hidden, 2e - 40), so the result is
 * independent of the reduction order and does not saturate. rrms =
 * 1 / sqrt(mean_sq + eps) with IEEE sqrt and division, y = IO((u * w) * rrms)
 * where u is the (rounded) value that was stored. A row holding inf or NaN
 * gets mean_sq = inf or NaN, as an fp32 sum would.
 * Replaces rms_norm_fxp_run / rms_norm_fxp_residual_run + _rms_norm_kernel
 * (fxpr_vllm/_triton/rms_norm.py:137-151, 78-134, 19-64), which take no
 * fixed-point format either.
 */
int fxpr_rms_norm(const void* x, void* residual, const void* weight, void* y,
                  int io_dtype, int64_t rows, int64_t hidden, float eps,
                  void* stream);

/*
 * Deterministic log-softmax over contiguous [rows, cols] rows of x (f32, f16
 * or bf16) into y (same type or f32), cols < 2^31. Per row: m = max x,
 * e_j = exp(x_j - m) by this library's fixed fp32 polynomial, S = exact sum
 * (64- or 128-bit, never saturated) of float_to_fixed(e_j, int_bits,
 * frac_bits), lse = m + log(fl32(S) * 2^-frac_bits) by the matching fixed
 * polynomial, y_j = OUT(x_j - lse).
 * No counterpart kernel exists in the reference: it lists
 * fxpr_vllm/_triton/softmax.py (README.md:60) but does not ship it.
 */
int fxpr_log_softmax(const void* x, int x_dtype, void* y, int y_dtype,
                     int64_t rows, int64_t cols, int int_bits, int frac_bits,
                     void* stream);

/*
 * Vocab-parallel log-softmax (rows whose columns are split over devices, as
 * a vocab-parallel lm_head leaves its logits). Per shard [rows, cols]:
 * fxpr_log_softmax_shard_max writes each row's maximum (fp32, NaN if any
 * element is NaN); the shards' maxima are combined by a MAX. Then
 * fxpr_log_softmax_shard_sum writes each row's exact integer sum (int64) of
 * float_to_fixed(exp(x - m), int_bits, frac_bits) against the combined
 * maximum m, the same terms fxpr_log_softmax sums; the shards' sums are
 * combined by an integer SUM (any order). fxpr_log_softmax_shard_finish then
 * writes the shard's outputs, y = OUT(x - (m + log(fl32(S) * 2^-frac_bits))).
 * The outputs equal fxpr_log_softmax's on the whole rows bit for bit while a
 * row's total stays below 2^63 (frac_bits <= 32, cols < 2^29 per shard).
 * No counterpart in the reference (its log-softmax is not shipped; README.md:60).
 */
int fxpr_log_softmax_shard_max(const void* x, int x_dtype, float* row_max,
                               int64_t rows, int64_t cols, void* stream);
int fxpr_log_softmax_shard_sum(const void* x, int x_dtype,
                               const float* row_max, int64_t* row_sum,
                               int64_t rows, int64_t cols, int int_bits,
                               int frac_bits, void* stream);
int fxpr_log_softmax_shard_finish(const void* x, int x_dtype,
                                  const float* row_max, const int64_t* row_sum,
                                  void* y, int y_dtype, int64_t rows,
                                  int64_t cols, int frac_bits, void* stream);

/*
 * Test hooks of fxpr_log_softmax's split-row kernel (no counterpart in the
 * reference). The kernel's workgroups of one row exchange their span maxima,
 * then their exact span sums, through device memory, polling each exchange
 * at most a number of times (fxpr_debug_lsm_default_spin_limit(): 16384,
 * milliseconds) before a workgroup computes what it waits for (the row's
 * maximum and exact sum) itself from the input, which gives the same bits.
 * fxpr_debug_set_lsm_spin_limit sets the two limits for later launches of
 * this process (0: that poll gives up at once, forcing its path);
 * fxpr_debug_lsm_fallbacks reads, synchronously, how many workgroups on the
 * current device have taken such a path so far.
 */
int fxpr_debug_set_lsm_spin_limit(int max_tries, int sum_tries);
int fxpr_debug_lsm_default_spin_limit(void);
int fxpr_debug_lsm_fallbacks(unsigned long long* count);

/*
 * Deterministic greedy sampling with log-probabilities over contiguous
 * [rows, cols] logits (f32, f16 or bf16), cols < 2^31. Each row's order is
 * largest value first, equal values by ascending index, every NaN above +inf,
 * -0 equal to +0. sampled[r] (int64) is the first element of the order and
 * sampled_logprob[r] (fp32) its log-probability; with num_logprobs = k in
 * [1, min(64, cols)], topk_ids / topk_logprobs [rows, k] hold the first k
 * elements of the order and their log-probabilities (both may be NULL for
 * k = 0). A log-probability is fl32(x_j) - lse with lse computed exactly as in
 * fxpr_log_softmax(int_bits, frac_bits): the values equal that function's
 * fp32 outputs bit for bit.
 * workspace (caller-owned, no zeroing) of at least
 * fxpr_sample_greedy_workspace_bytes(rows, num_logprobs) bytes lets a launch
 * of few rows (at most 128) spread each row over several workgroups; NULL or
 * a smaller workspace runs one workgroup per row. The bits are the same
 * either way.
 * No counterpart exists in the reference: it lists fxpr_vllm/sampling.py
 * (README.md:69) but does not ship it; this is the step after the lm_head
 * GEMM and log_softmax_fxp.
 */
int fxpr_sample_greedy(const void* logits, int x_dtype, int64_t rows,
                       int64_t cols, int num_logprobs, int int_bits,
                       int frac_bits, int64_t* sampled, float* sampled_logprob,
                       int64_t* topk_ids, float* topk_logprobs, void* workspace,
                       int64_t workspace_bytes, void* stream);
/* Workspace bytes fxpr_sample_greedy can use (0: it runs one workgroup per
 * row at this row count). */
int64_t fxpr_sample_greedy_workspace_bytes(int64_t rows, int num_logprobs);

/*
 * Fixed-point GEMM, C[M,N] = IO(fl32(acc) * 2^-frac_bits (+ bias)) with
 * acc = wrapping int_bits sum over K-tiles t (128 wide for bf16/f16, 64 for
 * f32; zero-padded tail) of RNE_sat(fp32 dot(A[m, t], B[t, n]) * 2^f).
 * io_dtype (bf16 / f16 / f32) is the type of A, B and C; bias is NULL or N
 * fp32 values. Strides are in elements: A must have stride_ak == 1; B must
 * have stride_bk == 1 (column-major, e.g. a transposed [N,K] weight) or
 * stride_bn == 1 (row-major [K,N]). split_k: 0 = automatic, >= 1 = that many
 * K-splits (clamped to the K-tile count); split counts never change bits.
 * When the resolved split count is > 1 a workspace of
 * fxpr_gemm_workspace_bytes() bytes is required (caller-owned, no zeroing).
 * Replaces gemm_fxp_run + _gemm_kernel / _gemm_splitk_kernel
 * (fxpr_vllm/_triton/gemm.py:612-763, 123-204, 209-325).
 */
int fxpr_gemm(const void* a, const void* b, const float* bias, void* c,
              int io_dtype, int64_t m, int64_t n, int64_t k,
              int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
              int64_t stride_bn, int64_t stride_cm, int64_t stride_cn,
              int int_bits, int frac_bits, int split_k, void* workspace,
              int64_t workspace_bytes, void* stream);

/*
 * Row-parallel (K-sharded) GEMM. fxpr_gemm_partial writes the integer
 * accumulators acc[m][n] (row-major [m, n]; int32 for int_bits 16 and 32,
 * int64 for 64) = wrapping sum over this call's K-tiles of
 * RNE_sat_b(P_t[m, n] * 2^frac_bits), the sums fxpr_gemm converts. A
 * K-shard's accumulators add up (integer SUM across shards, any order) to
 * the unsharded ones when its first column is a K-tile boundary of the full
 * K (a multiple of 128 for 16-bit inputs, 64 for fp32). fxpr_gemm_finish
 * applies fxpr_gemm's epilogue to summed accumulators (wrapped to int_bits):
 * C = IO(fl32(acc) * 2^-frac_bits (+ bias)), bias fp32 or NULL. Together they
 * give fxpr_gemm's bits. No counterpart in the reference, whose row-parallel
 * linears all-reduce bf16 outputs (quantisation_config.py:80-96).
 */
int fxpr_gemm_partial(const void* a, const void* b, void* acc, int io_dtype,
                      int64_t m, int64_t n, int64_t k, int64_t stride_am,
                      int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                      int int_bits, int frac_bits, void* stream);
int fxpr_gemm_finish(const void* acc, const float* bias, void* c,
                     int io_dtype, int64_t m, int64_t n, int64_t stride_cm,
                     int64_t stride_cn, int int_bits, int frac_bits,
                     void* stream);

/* Split count fxpr_gemm will use for this shape, accumulator width and
 * request. Host-side policy of the reference: _resolve_split_k
 * (gemm.py:385-412), which takes the accumulator width too. */
int fxpr_gemm_splits(int64_t m, int64_t n, int64_t k, int io_dtype,
                     int int_bits, int split_k);

/* Workspace bytes fxpr_gemm needs for this shape and request (0 = none).
 * Replaces the persistent scratch of gemm.py:61-107. */
int64_t fxpr_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k,
                                  int io_dtype, int int_bits, int split_k);

/*
 * Unified paged prefill + decode attention with fixed-point cross-tile
 * reductions: one pass over K and V, softmax statistics per 512-key chunk
 * (each chunk's weights against its own row maximum), chunks folded in
 * ascending order in fixed point; a row whose keys fit in one chunk gets
 * the reference's formula exactly, longer rows agree with it within the
 * fixed-point tolerance. q [num_tokens, num_heads, head_dim] and o share io_dtype
 * (bf16 / f16 / f32) with the caches; k_cache / v_cache are the two halves
 * of a vLLM [num_blocks, 2, page_size, num_kv_heads, head_dim] cache (any
 * strides, unit stride along head_dim). Metadata: query_start_loc
 * [num_requests + 1], seq_lens [num_requests], block_table [num_requests,
 * max_blocks_per_seq], all int32. alibi_slopes: NULL or num_heads fp32 in
 * log2 units. softmax_scale_log2 = scale * log2(e); softcap_log2 =
 * logit_softcap * log2(e) (0 = off); window_size 0 = off. num_kv_splits:
 * 0 = automatic (fxpr_attention_splits() reports the choice), >= 1 = that
 * many KV splits (a launch whose split partials would exceed 1 GiB runs
 * unsplit; the bits are the same). The launch needs a workspace of
 * fxpr_attention_workspace_bytes() bytes when that is non-zero (no zeroing).
 * The output is bitwise independent of num_splits, of the batch the request
 * is in and of max_query_len.
 * Replaces unified_attention_fxp_run + _attn_fused_kernel /
 * _attn_split_max_kernel / _attn_split_dv_kernel
 * (fxpr_vllm/_triton/attention.py:692-953, 127-301, 306-436, 440-652).
 */
int fxpr_unified_attention(
    const void* q, const void* k_cache, const void* v_cache, void* o,
    int io_dtype, const int32_t* query_start_loc, const int32_t* seq_lens,
    const int32_t* block_table, const float* alibi_slopes, int num_requests,
    int64_t num_tokens, int num_heads, int num_kv_heads, int head_dim,
    int page_size, int max_query_len, int max_blocks_per_seq,
    int64_t num_blocks, int64_t stride_q_token, int64_t stride_q_head,
    int64_t stride_k_block, int64_t stride_k_slot, int64_t stride_k_head,
    int64_t stride_v_block, int64_t stride_v_slot, int64_t stride_v_head,
    int64_t stride_o_token, int64_t stride_o_head, int64_t stride_bt_row,
    int is_causal, float softmax_scale_log2, float softcap_log2,
    int window_size, int int_bits, int frac_bits, int num_kv_splits,
    void* workspace, int64_t workspace_bytes, void* stream);

/* Size of the device array fxpr_unified_attention_noalloc keeps its split
 * partials in (per GPU, for the life of the process). */
#define FXPR_STATIC_SCRATCH_BYTES (64LL << 20)

/*
 * fxpr_unified_attention without the workspace arguments: allocates nothing.
 * The split partials go to a static device array of FXPR_STATIC_SCRATCH_BYTES
 * per GPU; a launch whose fxpr_attention_workspace_bytes() exceeds that is
 * rejected with FXPR_E_WORKSPACE before anything runs. The array's device
 * address is looked up at the first split call on each device, which must
 * not be under HIP graph capture (FXPR_E_CAPTURE; any eager call that splits
 * sets it up, and capture is fine after that). Same results as
 * fxpr_unified_attention bit for bit. Calls that overlap on one GPU (two
 * streams, or two host threads) share the array and race: serialise them.
 * The stream must belong to the current device or be NULL.
 * No counterpart in the reference: this is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).
 */
int fxpr_unified_attention_noalloc(
    const void* q, const void* k_cache, const void* v_cache, void* o,
    int io_dtype, const int32_t* query_start_loc, const int32_t* seq_lens,
    const int32_t* block_table, const float* alibi_slopes, int num_requests,
    int64_t num_tokens, int num_heads, int num_kv_heads, int head_dim,
    int page_size, int max_query_len, int max_blocks_per_seq,
    int64_t num_blocks, int64_t stride_q_token, int64_t stride_q_head,
    int64_t stride_k_block, int64_t stride_k_slot, int64_t stride_k_head,
    int64_t stride_v_block, int64_t stride_v_slot, int64_t stride_v_head,
    int64_t stride_o_token, int64_t stride_o_head, int64_t stride_bt_row,
    int is_causal, float softmax_scale_log2, float softcap_log2,
    int window_size, int int_bits, int frac_bits, int num_kv_splits,
    void* stream);

/* KV split count for num_kv_splits = requested (0 = automatic).
 * Replaces _pick_num_splits (fxpr_vllm/_triton/attention.py:664-689). */
int fxpr_attention_splits(int num_requests, int num_kv_heads, int group,
                          int max_query_len, int max_blocks_per_seq,
                          int page_size, int requested);

/* Workspace bytes fxpr_unified_attention needs for this launch (0 = none):
 * with more than one split, per (token, head) the chunk range and per
 * (token, head, chunk) the maximum, the integer denominator and the integer
 * weighted-V row. Replaces the per-call scratch of attention.py:839-851. */
int64_t fxpr_attention_workspace_bytes(int num_requests, int64_t num_tokens,
                                       int num_heads, int num_kv_heads,
                                       int head_dim, int int_bits,
                                       int num_kv_splits, int max_query_len,
                                       int max_blocks_per_seq, int page_size);

/*
 * Paged KV-cache write: for each token t with slot = slot_mapping[t] >= 0,
 * k_cache[slot / block_size, slot % block_size, h, :] = key[t, h, :] and the
 * same for value / v_cache (the two halves of a vLLM [num_blocks, 2,
 * block_size, num_kv_heads, head_size] cache). Negative slots (padding) and
 * slots >= num_blocks * block_size are skipped. dtype: f16 / bf16 / f32 for
 * all four tensors; head rows must be 16-byte aligned (strides in elements).
 * A bit-exact copy.
 * Replaces reshape_and_cache_flash as called by the reference backend's
 * do_kv_cache_update (fxpr_vllm/attention_backend.py:253-277).
 */
int fxpr_reshape_and_cache(const void* key, const void* value, void* k_cache,
                           void* v_cache, int dtype,
                           const int64_t* slot_mapping, int64_t num_tokens,
                           int num_kv_heads, int head_size, int block_size,
                           int64_t num_blocks, int64_t stride_key_token,
                           int64_t stride_key_head, int64_t stride_value_token,
                           int64_t stride_value_head, int64_t stride_kc_block,
                           int64_t stride_kc_slot, int64_t stride_kc_head,
                           int64_t stride_vc_block, int64_t stride_vc_slot,
                           int64_t stride_vc_head, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FXPR_H */
