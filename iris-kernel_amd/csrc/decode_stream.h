// Host entry points of the streaming decode kernel (decode_stream.hip),
// called by the C ABI in decode.hip / decode_pages.hip for the shapes it
// supports.
#pragma once

#include <stdint.h>

#define IRIS_INTERNAL __attribute__((visibility("hidden")))

namespace iris {

// head_dim 128, 8 kv heads, 4 or 8 query heads per kv head (chunk mode).
IRIS_INTERNAL bool stream_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim);

// The shapes of the balanced mode: head_dim 128, 8 kv heads, 4 query heads per kv head.
IRIS_INTERNAL bool stream_balanced_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim);

// Most chunks per sequence a launch can merge.
IRIS_INTERNAL int stream_max_chunks();

// Balanced-mode plan for ragged lengths (total_tokens known): about one
// range of the sequences' tiles, plus a per-sequence start cost, a CU;
// chunk_tiles negative (minus the units a range holds at most).
IRIS_INTERNAL int stream_balanced_plan(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t total_tokens,
                                       int32_t* out_chunk_tiles, int32_t* out_max_chunks,
                                       int64_t* out_workspace_bytes);

// Split-KV workspace of a chunk-mode launch with max_chunks chunks per sequence.
IRIS_INTERNAL int64_t stream_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                             int64_t head_dim, int64_t max_chunks);

// Chunk-mode launch: batch x max_chunks workgroups of chunk_tiles 32-token tiles.
IRIS_INTERNAL int stream_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale,
                                const void* v_scale, const int32_t* block_table, const int32_t* seq_lens,
                                void* output, int32_t output_is_f32, void* workspace, int64_t workspace_bytes_avail,
                                int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                int64_t max_pages, int64_t bt_cols, int32_t page_mul, float softmax_scale,
                                int32_t chunk_tiles, int32_t max_chunks, void* stream);

}  // namespace iris
