// Paged KV-cache write: the scatter that precedes attention in a decode /
// prefill step. Token t's key and value rows (num_kv_heads x head_size) go to
// slot slot_mapping[t] = block * block_size + offset of the
// [num_blocks, 2, block_size, num_kv_heads, head_size] cache. Negative slots
// (padding tokens) and slots past the cache are skipped. A pure copy: the
// cache holds the same bits as the inputs.
//
// Replaces the reshape_and_cache_flash call of the reference backend's
// do_kv_cache_update (fxpr_vllm/attention_backend.py:253-277), which lives in
// vLLM's compiled extension.
#include "fxpr_internal.h"

namespace fxpr {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct CacheArgs {
  const char* key;
  const char* value;
  char* k_cache;
  char* v_cache;
  const int64_t* slots;
  int64_t num_tokens, num_slots;
  int num_kv_heads, chunks_per_head, block_size;
  // strides in bytes
  int64_t sk_t, sk_h, sv_t, sv_h, skc_b, skc_s, skc_h, svc_b, svc_s, svc_h;
};

// One thread per 16-byte chunk of one (token, head) row, for K and V.
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(CacheArgs a) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t per_token = int64_t(a.num_kv_heads) * a.chunks_per_head;
  if (idx >= a.num_tokens * per_token) return;
  const int64_t t = idx / per_token;
  const int rem = int(idx - t * per_token);
  const int h = rem / a.chunks_per_head, c = rem % a.chunks_per_head;
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.num_slots) return;
  const int64_t blk = slot / a.block_size, off = slot % a.block_size;
  const u32x4 k = *reinterpret_cast<const u32x4*>(a.key + t * a.sk_t + h * a.sk_h + c * 16);
  const u32x4 v = *reinterpret_cast<const u32x4*>(a.value + t * a.sv_t + h * a.sv_h + c * 16);
  *reinterpret_cast<u32x4*>(a.k_cache + blk * a.skc_b + off * a.skc_s + h * a.skc_h + c * 16) = k;
  *reinterpret_cast<u32x4*>(a.v_cache + blk * a.svc_b + off * a.svc_s + h * a.svc_h + c * 16) = v;
}

inline int elem_bytes(int dtype) {
  switch (dtype) {
    case FXPR_DTYPE_F16:
    case FXPR_DTYPE_BF16: return 2;
    case FXPR_DTYPE_F32: return 4;
    default: return 0;
  }
}

}  // namespace
}  // namespace fxpr

using namespace fxpr;

extern "C" int fxpr_reshape_and_cache(const void* key, const void* value, void* k_cache, void* v_cache,
                                      int dtype, const int64_t* slot_mapping, int64_t num_tokens,
                                      int num_kv_heads, int head_size, int block_size, int64_t num_blocks,
                                      int64_t stride_key_token, int64_t stride_key_head,
                                      int64_t stride_value_token, int64_t stride_value_head,
                                      int64_t stride_kc_block, int64_t stride_kc_slot, int64_t stride_kc_head,
                                      int64_t stride_vc_block, int64_t stride_vc_slot, int64_t stride_vc_head,
                                      void* stream) {
  const int esz = elem_bytes(dtype);
  if (esz == 0) return FXPR_E_DTYPE;
  if (num_tokens < 0 || num_kv_heads <= 0 || head_size <= 0 || block_size <= 0 || num_blocks < 0)
    return FXPR_E_SHAPE;
  if (num_tokens == 0 || num_blocks == 0) return FXPR_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return FXPR_E_ARG;
  // 16-byte chunks: rows and every stride must keep 16-byte alignment
  const int64_t row_bytes = int64_t(head_size) * esz;
  if (row_bytes % 16 != 0) return FXPR_E_SHAPE;
  const int64_t strides[] = {stride_key_token, stride_key_head, stride_value_token, stride_value_head,
                             stride_kc_block,  stride_kc_slot,  stride_kc_head,     stride_vc_block,
                             stride_vc_slot,   stride_vc_head};
  for (int64_t s : strides)
    if ((s * esz) % 16 != 0) return FXPR_E_ARG;
  if (!aligned(key, 16) || !aligned(value, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return FXPR_E_ARG;

  CacheArgs a{};
  a.key = static_cast<const char*>(key);
  a.value = static_cast<const char*>(value);
  a.k_cache = static_cast<char*>(k_cache);
  a.v_cache = static_cast<char*>(v_cache);
  a.slots = slot_mapping;
  a.num_tokens = num_tokens;
  a.num_slots = num_blocks * block_size;
  a.num_kv_heads = num_kv_heads;
  a.chunks_per_head = int(row_bytes / 16);
  a.block_size = block_size;
  a.sk_t = stride_key_token * esz;
  a.sk_h = stride_key_head * esz;
  a.sv_t = stride_value_token * esz;
  a.sv_h = stride_value_head * esz;
  a.skc_b = stride_kc_block * esz;
  a.skc_s = stride_kc_slot * esz;
  a.skc_h = stride_kc_head * esz;
  a.svc_b = stride_vc_block * esz;
  a.svc_s = stride_vc_slot * esz;
  a.svc_h = stride_vc_head * esz;
  const int64_t total = num_tokens * num_kv_heads * a.chunks_per_head;
  if (cdiv(total, 256) > 0x7fffffff) return FXPR_E_SHAPE;
  reshape_and_cache_kernel<<<dim3(unsigned(cdiv(total, 256))), 256, 0, as_stream(stream)>>>(a);
  return launch_status();
}
