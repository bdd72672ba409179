// C-ABI entry points of the paged attention (kernels: attn_impl.h,
// instantiated per input type in attn_{bf16,f16,f32}.hip).
#include <algorithm>
#include <mutex>

#include "attn_impl.h"

using namespace fxpr;
using namespace fxpr::attn;

namespace {

constexpr int kMaxSplits = 64;      // automatic policy's largest split count
constexpr int64_t kMaxGridZ = 65535;  // splits are the launch grid's z dimension
// Split launches keep per-chunk partials; above this many bytes of them a
// launch runs unsplit instead (split counts never change the bits).
constexpr int64_t kSplitWsMax = int64_t(1) << 30;

inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

inline int acc_bytes(int int_bits) { return int_bits == 64 ? 8 : 4; }

// Chunks per row that a block-table row of max_blocks pages can hold.
inline int64_t chunk_slots(int max_blocks, int page_size) {
  return cdiv(cdiv(int64_t(max_blocks) * page_size, TILE), CT);
}

// Split-launch workspace: per (token, head) the chunk range, and per
// (token, head, chunk) the row maximum, the integer denominator and the
// integer weighted V row. Unsplit launches need none.
struct WsLayout {
  int64_t crange = -1, pmax = -1, den = -1, wv = -1, total = 0;
};

WsLayout ws_layout(int64_t num_tokens, int num_heads, int head_dim, int int_bits, int splits, int64_t slots) {
  WsLayout w;
  if (splits <= 1) return w;
  const int64_t rows = num_tokens * num_heads;
  w.crange = 0;
  w.total = align256(rows * 8);
  w.pmax = w.total;
  w.total += align256(rows * slots * 4);
  w.den = w.total;
  w.total += align256(rows * slots * acc_bytes(int_bits));
  w.wv = w.total;
  w.total += align256(rows * slots * head_dim * acc_bytes(int_bits));
  return w;
}

}  // namespace

// Split policy (this build's own; the reference's _pick_num_splits,
// attention.py:664-689, is the model for its shape). An explicit request wins
// (each workgroup's key chunks dealt evenly over the splits, as the
// reference's _split_tile_range deals tiles), up to the number of 512-key
// chunks a block-table row holds: splits past that would hold no keys (the
// reference's would be empty), so the launch runs that many. Automatic (0):
// no split for short contexts (<= 32 key tiles of 64) or when the
// (request, kv head, 16-row query tile) workgroups already number more than
// 8 x 256; otherwise one chunk per split (up to 64 splits), so every
// workgroup carries about the same work whatever its request's length
// (requests shorter than the longest get empty splits). Split counts never
// change bits.
namespace {
constexpr int kSplitChunks = 1;

struct SplitPlan {
  int splits, chunks_per_split;
};

SplitPlan plan_splits(int num_requests, int num_kv_heads, int group, int max_query_len, int max_blocks,
                      int page_size, int requested) {
  const int64_t tiles = cdiv(int64_t(max_blocks > 0 ? max_blocks : 1) * page_size, TILE);
  if (requested >= 1) {
    const int64_t cap = std::min<int64_t>(std::max<int64_t>(cdiv(tiles, CT), 1), kMaxGridZ);
    return {int(std::min<int64_t>(requested, cap)), 0};
  }
  if (tiles <= 32) return {1, 0};
  const int64_t qtiles = cdiv(int64_t(max_query_len > 1 ? max_query_len : 1) * group, QROWS);
  const int64_t base = int64_t(num_requests > 1 ? num_requests : 1) * num_kv_heads * qtiles;
  if (base > 8 * 256) return {1, 0};
  const int64_t chunks = cdiv(tiles, CT);
  int64_t s = cdiv(chunks, kSplitChunks);
  if (s > kMaxSplits) s = kMaxSplits;
  if (s <= 1) return {1, 0};
  return {int(s), int(cdiv(chunks, s))};
}

// The plan a launch runs: plan_splits, unsplit when the partials would exceed
// kSplitWsMax.
SplitPlan launch_plan(int num_requests, int64_t num_tokens, int num_heads, int num_kv_heads, int head_dim,
                      int int_bits, int max_query_len, int max_blocks, int page_size, int requested) {
  SplitPlan sp = plan_splits(num_requests, num_kv_heads, num_heads / num_kv_heads, max_query_len, max_blocks,
                             page_size, requested);
  if (sp.splits > 1 &&
      ws_layout(num_tokens, num_heads, head_dim, int_bits, sp.splits, chunk_slots(max_blocks, page_size)).total >
          kSplitWsMax)
    sp = {1, 0};
  return sp;
}
}  // namespace

extern "C" int fxpr_attention_splits(int num_requests, int num_kv_heads, int group, int max_query_len,
                                     int max_blocks_per_seq, int page_size, int requested) {
  return plan_splits(num_requests, num_kv_heads, group, max_query_len, max_blocks_per_seq, page_size,
                     requested)
      .splits;
}

extern "C" int64_t fxpr_attention_workspace_bytes(int num_requests, int64_t num_tokens, int num_heads,
                                                  int num_kv_heads, int head_dim, int int_bits,
                                                  int num_kv_splits, int max_query_len,
                                                  int max_blocks_per_seq, int page_size) {
  if (num_requests <= 0 || num_tokens <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      max_blocks_per_seq <= 0 || page_size <= 0 || num_heads % num_kv_heads != 0 || num_kv_splits < 0)
    return 0;
  const SplitPlan sp = launch_plan(num_requests, num_tokens, num_heads, num_kv_heads, head_dim, int_bits,
                                   max_query_len, max_blocks_per_seq, page_size, num_kv_splits);
  return ws_layout(num_tokens, num_heads, head_dim, int_bits, sp.splits,
                   chunk_slots(max_blocks_per_seq, page_size))
      .total;
}

extern "C" int fxpr_unified_attention(
    const void* q, const void* k_cache, const void* v_cache, void* o, int io_dtype,
    const int32_t* query_start_loc, const int32_t* seq_lens, const int32_t* block_table,
    const float* alibi_slopes, int num_requests, int64_t num_tokens, int num_heads,
    int num_kv_heads, int head_dim, int page_size, int max_query_len, int max_blocks_per_seq,
    int64_t num_blocks, int64_t stride_q_token, int64_t stride_q_head, int64_t stride_k_block,
    int64_t stride_k_slot, int64_t stride_k_head, int64_t stride_v_block, int64_t stride_v_slot,
    int64_t stride_v_head, int64_t stride_o_token, int64_t stride_o_head, int64_t stride_bt_row,
    int is_causal, float softmax_scale_log2, float softcap_log2, int window_size, int int_bits,
    int frac_bits, int num_kv_splits, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!valid_int_bits(int_bits) || frac_bits < 0 || frac_bits > 63) return FXPR_E_BITS;
  if (num_requests < 0 || num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      page_size <= 0 || num_kv_splits < 0 || num_heads % num_kv_heads != 0)
    return FXPR_E_SHAPE;
  if (num_requests == 0 || num_tokens == 0) return FXPR_OK;
  if (max_blocks_per_seq <= 0 || num_blocks <= 0) return FXPR_E_SHAPE;
  const SplitPlan sp = launch_plan(num_requests, num_tokens, num_heads, num_kv_heads, head_dim, int_bits,
                                   max_query_len, max_blocks_per_seq, page_size, num_kv_splits);
  const int num_splits = sp.splits;
  if (!q || !k_cache || !v_cache || !o || !query_start_loc || !seq_lens || !block_table) return FXPR_E_ARG;
  if (io_dtype != FXPR_DTYPE_BF16 && io_dtype != FXPR_DTYPE_F16 && io_dtype != FXPR_DTYPE_F32)
    return FXPR_E_DTYPE;
  const int ch = io_dtype == FXPR_DTYPE_F32 ? 4 : 8;
  // vector loads of q / k / v rows need 16-byte alignment
  if (head_dim % ch != 0 || head_dim > 256 || (io_dtype == FXPR_DTYPE_F32 && head_dim > 128))
    return FXPR_E_SHAPE;
  if (stride_q_token % ch || stride_q_head % ch || stride_k_block % ch || stride_k_slot % ch ||
      stride_k_head % ch || stride_v_block % ch || stride_v_slot % ch || stride_v_head % ch ||
      !aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return FXPR_E_ARG;
  // the kernels form cache offsets as 32 x 32 -> 64-bit products
  for (int64_t sv : {stride_k_block, stride_k_slot, stride_k_head, stride_v_block, stride_v_slot, stride_v_head})
    if (sv < 0 || sv > int64_t(0xffffffff)) return FXPR_E_ARG;
  const int64_t slots = chunk_slots(max_blocks_per_seq, page_size);
  if (slots > 0x7fffffff) return FXPR_E_SHAPE;
  const WsLayout wl = ws_layout(num_tokens, num_heads, head_dim, int_bits, num_splits, slots);
  if (wl.total > 0 && (!workspace || workspace_bytes < wl.total)) return FXPR_E_WORKSPACE;

  AttnArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.o = o;
  a.qsl = query_start_loc;
  a.seq_lens = seq_lens;
  a.bt = block_table;
  a.alibi = alibi_slopes;
  char* base = static_cast<char*>(workspace);
  if (wl.crange >= 0) a.crange = reinterpret_cast<int*>(base + wl.crange);
  if (wl.pmax >= 0) a.pmax = reinterpret_cast<float*>(base + wl.pmax);
  if (wl.den >= 0) a.den_ws = base + wl.den;
  if (wl.wv >= 0) a.wv_ws = base + wl.wv;
  a.chunk_slots = int(slots);
  a.sq_t = stride_q_token;
  a.sq_h = stride_q_head;
  a.sk_b = stride_k_block;
  a.sk_s = stride_k_slot;
  a.sk_h = stride_k_head;
  a.sv_b = stride_v_block;
  a.sv_s = stride_v_slot;
  a.sv_h = stride_v_head;
  a.so_t = stride_o_token;
  a.so_h = stride_o_head;
  a.sbt = stride_bt_row;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_heads / num_kv_heads;
  a.head_dim = head_dim;
  a.page_size = page_size;
  a.num_splits = num_splits;
  a.chunks_per_split = sp.chunks_per_split;
  a.window = window_size > 0 ? window_size : 0;
  a.causal = is_causal ? 1 : 0;
  a.max_blocks = max_blocks_per_seq;
  a.num_requests = num_requests;
  a.num_blocks = num_blocks;
  a.num_tokens = num_tokens;
  a.lmax = int64_t(max_blocks_per_seq) * page_size;
  a.ps_shift = (page_size & (page_size - 1)) == 0 ? __builtin_ctz(unsigned(page_size)) : -1;
  a.scale_log2 = softmax_scale_log2;
  a.softcap_log2 = softcap_log2;
  a.fxp_scale = pow2f(frac_bits);
  a.fxp_inv = pow2f(-frac_bits);
  const int max_qtiles = int(cdiv(int64_t(max_query_len > 1 ? max_query_len : 1) * a.group, QROWS));
  hipStream_t st = as_stream(stream);
  switch (io_dtype) {
    case FXPR_DTYPE_BF16: return run_attn_bf16(a, int_bits, num_requests, max_qtiles, num_tokens, st);
    case FXPR_DTYPE_F16: return run_attn_f16(a, int_bits, num_requests, max_qtiles, num_tokens, st);
    default: return run_attn_f32(a, int_bits, num_requests, max_qtiles, num_tokens, st);
  }
}

// ---------------------------------------------------------------------------
// The same launch without a caller workspace: split partials go to `scratch`,
// a file-scope device array of kStaticScratchBytes that each GPU the library
// runs on holds until the process ends. Its device address is looked up once
// per device (hipGetSymbolAddress with that device current) and kept in
// scratch_ptr; host code never passes the array's own name to a kernel. The
// partials need no zeroing (every slot a combine reads was written by the
// same launch). Calls that overlap on one GPU share the array and race.

namespace {

constexpr int64_t kStaticScratchBytes = FXPR_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the stream's device (the current device
// for the null stream).
int static_scratch(hipStream_t st, void** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return static_cast<int>(e);
  int dev = cur;
  if (st != nullptr) {
    e = hipStreamGetDevice(st, &dev);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  if (dev < 0 || dev >= kMaxDevices) return FXPR_E_ARG;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_ptr[dev] == nullptr) {
    // the look-up (and a device switch) stays out of graph capture
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(st, &cs)) != hipSuccess) return static_cast<int>(e);
    if (cs != hipStreamCaptureStatusNone) return FXPR_E_CAPTURE;
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return static_cast<int>(e);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess) return static_cast<int>(e);
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return FXPR_OK;
}

}  // namespace

extern "C" int fxpr_unified_attention_noalloc(
    const void* q, const void* k_cache, const void* v_cache, void* o, int io_dtype,
    const int32_t* query_start_loc, const int32_t* seq_lens, const int32_t* block_table,
    const float* alibi_slopes, int num_requests, int64_t num_tokens, int num_heads,
    int num_kv_heads, int head_dim, int page_size, int max_query_len, int max_blocks_per_seq,
    int64_t num_blocks, int64_t stride_q_token, int64_t stride_q_head, int64_t stride_k_block,
    int64_t stride_k_slot, int64_t stride_k_head, int64_t stride_v_block, int64_t stride_v_slot,
    int64_t stride_v_head, int64_t stride_o_token, int64_t stride_o_head, int64_t stride_bt_row,
    int is_causal, float softmax_scale_log2, float softcap_log2, int window_size, int int_bits,
    int frac_bits, int num_kv_splits, void* stream) {
  const int64_t need = fxpr_attention_workspace_bytes(num_requests, num_tokens, num_heads, num_kv_heads,
                                                      head_dim, int_bits, num_kv_splits, max_query_len,
                                                      max_blocks_per_seq, page_size);
  if (need > kStaticScratchBytes) return FXPR_E_WORKSPACE;
  void* ws = nullptr;
  if (need > 0) {
    const int rc = static_scratch(as_stream(stream), &ws);
    if (rc != FXPR_OK) return rc;
  }
  return fxpr_unified_attention(q, k_cache, v_cache, o, io_dtype, query_start_loc, seq_lens, block_table,
                                alibi_slopes, num_requests, num_tokens, num_heads, num_kv_heads, head_dim,
                                page_size, max_query_len, max_blocks_per_seq, num_blocks, stride_q_token,
                                stride_q_head, stride_k_block, stride_k_slot, stride_k_head, stride_v_block,
                                stride_v_slot, stride_v_head, stride_o_token, stride_o_head, stride_bt_row,
                                is_causal, softmax_scale_log2, softcap_log2, window_size, int_bits, frac_bits,
                                num_kv_splits, ws, need, stream);
}
