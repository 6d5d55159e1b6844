// Host entry points of the page-streaming decode kernel (decode_pages.hip),
// called by the C ABI in decode.hip for the shapes it supports.
#pragma once

#include <stdint.h>

// Internal to libiris_hip.so: not exported.
#define IRIS_INTERNAL __attribute__((visibility("hidden")))

namespace iris {

// Hkv 1, 2, 4 or 8; head_dim 64 with Hq / Hkv <= 16 or head_dim 128 with
// Hq / Hkv <= 8; and the merge weights of a block_table this wide fit in
// LDS.
IRIS_INTERNAL bool pages_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_pages);

// Waves per workgroup of every page-streaming launch (the general kernel
// uses at most 4, so waves_per_block tells the two apart).
IRIS_INTERNAL int pages_waves();

// allow_stream: a plan for the streaming kernel where it covers the shape
// (its launch will run it), else for this kernel.
IRIS_INTERNAL int pages_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                             int64_t max_pages, int64_t total_tokens, int64_t max_tokens, int32_t tokens_per_split,
                             bool allow_stream, int32_t* out_chunk_tiles, int32_t* out_max_chunks, int32_t* out_waves,
                             int64_t* out_workspace_bytes);

IRIS_INTERNAL int64_t pages_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t max_chunks);

IRIS_INTERNAL int pages_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale,
                               const void* v_scale, const int32_t* block_table, const int32_t* seq_lens, void* output,
                               int32_t output_is_f32, void* workspace, int64_t workspace_bytes_avail, int64_t batch,
                               int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_pages,
                               int64_t bt_cols, int32_t page_mul, float softmax_scale, int32_t chunk_tiles,
                               int32_t max_chunks, bool allow_stream, void* stream);

}  // namespace iris
