// Host entry points of the any-shape decode kernel (decode_any.hip), called
// by the C ABI in decode.hip for the shapes the other kernels do not cover.
#pragma once

#include <stdint.h>

#define IRIS_INTERNAL __attribute__((visibility("hidden")))

namespace iris {

// head_dim a multiple of 32, at most 512 (any page size, any number of
// query heads per kv head).
IRIS_INTERNAL bool any_supported(int64_t head_dim);

// Waves of the kernel's workgroups.
IRIS_INTERNAL int any_waves();

// Chunk plan over cap_tokens = the tokens a block-table row can address:
// chunk_tiles in 32-token units (even: the kernel's tiles are 64 tokens),
// max_chunks chunks a sequence, the split-KV workspace size.
IRIS_INTERNAL int any_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                           int64_t cap_tokens, int64_t total_tokens, int64_t max_tokens, int32_t tokens_per_split,
                           int32_t* out_chunk_tiles, int32_t* out_max_chunks, int64_t* out_workspace_bytes);

// Launch: batch x num_kv_heads x ceil(g / 16) x max_chunks workgroups; page
// table entry e of a row covers tokens [e * page_size, (e + 1) * page_size).
IRIS_INTERNAL int any_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale,
                             const void* v_scale, const int32_t* block_table, const int32_t* seq_lens, void* output,
                             int32_t output_is_f32, void* workspace, int64_t workspace_bytes_avail, int64_t batch,
                             int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                             int64_t bt_cols, float softmax_scale, int32_t chunk_tiles, int32_t max_chunks,
                             void* stream);

}  // namespace iris
