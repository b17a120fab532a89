// Internal interface of the KV-cache, paged-attention and RoPE kernels
// (w4a16_attention.hip) for the C ABI (w4a16_capi.hip).  Not installed; the
// public ABI is include/drofell_w4a16.h.
#pragma once

#include "w4a16_internal.h"

namespace dw4 {

// Paged-attention decode over the block pointer tables of a KV cache.
constexpr int kAttnMaxPartTokens = 512;  // tokens per context partition, at most
constexpr int kAttnMaxGroup = 8;         // query heads per kv head, at most
struct PagedAttnArgs {
  int num_seqs, num_heads, num_kv_heads, head_size, block_size;
  const uint16_t* query;  // [num_seqs][num_heads][head_size], q_stride per sequence
  int64_t q_stride;
  uint16_t* out;          // same shape, o_stride per sequence
  int64_t o_stride;
  const int64_t* kptr;    // per-block key / value base addresses
  const int64_t* vptr;
  int kv_head_stride;     // elements between kv heads within a block
  float scale;
  const int32_t* block_tables;  // [num_seqs][max_blocks]
  int max_blocks;
  const int32_t* context_lens;  // [num_seqs], each >= 1
  const float* alibi;           // [num_heads] or null
};
struct PagedAttnPlan {
  int part_tokens = kAttnMaxPartTokens;
  int num_parts = 1;
  int waves = 4;  // per workgroup: 4, or 16 for one workgroup per (sequence, kv head)
};
// The 16-wave form: contexts up to this many tokens in one partition, for
// the (head size, block size, query-head group) variants whose per-wave
// partial outputs fit LDS and whose registers fit 1024-thread workgroups.
constexpr int kAttnWideMaxTokens = 1024;
constexpr bool attn_wide_ok(int hs, int bs, int gmax) {
  return bs == 16 && hs <= 128 && gmax * hs <= 512;
}
// Dynamic LDS of a paged-attention workgroup: the scaled queries [gmax][hs],
// the logits [gmax][part_tokens], the waves' partial outputs
// [waves][gmax][hs] and one float per wave for block reductions.
inline size_t attn_smem_bytes(int hs, int gmax, int part_tokens, int waves) {
  return sizeof(float) * ((size_t)gmax * hs + (size_t)gmax * part_tokens +
                          (size_t)waves * gmax * hs + waves);
}
PagedAttnPlan plan_paged_attention(int num_seqs, int num_heads, int num_kv_heads, int head_size,
                                   int block_size, int max_context_len, int cus);
size_t paged_attention_ws_bytes(const PagedAttnPlan& p, int num_seqs, int num_heads,
                                int head_size);
hipError_t launch_paged_attention(const PagedAttnArgs& a, const PagedAttnPlan& p, float* ws,
                                  hipStream_t stream);
// Token rows to their cache slots (restore: slots back to rows); slot < 0 skips a row.
hipError_t launch_reshape_and_cache(uint16_t* key, int64_t key_stride, uint16_t* value,
                                    int64_t value_stride, const int64_t* kptr, const int64_t* vptr,
                                    const int64_t* slots, int num_tokens, int num_kv_heads,
                                    int head_size, int block_size, int kv_head_stride,
                                    bool restore, hipStream_t stream);

// Rotary embedding in place on fp16 rows [batch][rows][hd] (reference half-precision form).
hipError_t launch_rope(uint16_t* x, const uint16_t* sinp, const uint16_t* cosp, int batch,
                       int rows, int hd, int heads, int max_pos, int past_len,
                       const int32_t* past_lens, hipStream_t stream);

// Decode-step rotary embedding of q and k plus the KV-cache write, one launch.
struct RopeCacheArgs {
  int num_seqs, heads, kv_heads, hd, bs;
  uint16_t* q;
  int64_t q_stride;
  uint16_t* k;
  int64_t k_stride;
  const uint16_t* v;
  int64_t v_stride;
  const uint16_t* sinp;
  const uint16_t* cosp;
  int max_pos;
  const int32_t* positions;
  const int32_t* block_tables;
  int max_blocks;
  const int64_t* kptr;
  const int64_t* vptr;
  int kv_head_stride;
  int32_t* lens_out;
};
hipError_t launch_rope_cache(const RopeCacheArgs& a, hipStream_t stream);

}  // namespace dw4
