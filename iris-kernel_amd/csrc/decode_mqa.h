// Host entry points of the MQA streaming decode kernel (decode_mqa.hip),
// called by the C ABI in decode.hip for the shapes it supports.
#pragma once

#include <stdint.h>

#define IRIS_INTERNAL __attribute__((visibility("hidden")))

namespace iris {

// One kv head, head_dim 64, at most 16 query heads.
IRIS_INTERNAL bool mqa_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim);

// Waves of the kernel's workgroups (the plan's waves_per_block names it).
IRIS_INTERNAL int mqa_waves();

// Chunk plan: chunk_tiles (a multiple of 16, at most 128) and max_chunks
// for a grid of about one workgroup per CU; workspace bytes for the split.
IRIS_INTERNAL int mqa_plan(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t max_pages,
                           int64_t max_tokens, int32_t tokens_per_split, int32_t* out_chunk_tiles,
                           int32_t* out_max_chunks, int32_t* out_waves, int64_t* out_workspace_bytes);

// Chunk-mode launch: batch x max_chunks workgroups of chunk_tiles 32-token tiles.
IRIS_INTERNAL int mqa_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale,
                             const void* v_scale, const int32_t* block_table, const int32_t* seq_lens, void* output,
                             int32_t output_is_f32, void* workspace, int64_t workspace_bytes_avail, int64_t batch,
                             int64_t num_q_heads, int64_t max_pages, int64_t bt_cols, int32_t page_shift,
                             float softmax_scale, int32_t chunk_tiles, int32_t max_chunks, void* stream);

}  // namespace iris
