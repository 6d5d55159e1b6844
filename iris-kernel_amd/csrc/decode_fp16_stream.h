// Host entry points of the page-streaming FP16 decode kernel
// (decode_fp16_stream.hip), called by the C ABI in decode_fp16.hip for the
// shapes it supports.
#pragma once

#include <stdint.h>

#define IRIS_INTERNAL __attribute__((visibility("hidden")))

namespace iris {

// head_dim 128 with 4 or 8 kv heads, head_dim 64 with 8 or 16; at most 16
// query heads per kv head.
IRIS_INTERNAL bool fp16_stream_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim);

// Whether the plan takes this kernel: batches of similar lengths, enough of
// them to fill half the CUs, at least 64 MB of K/V.
IRIS_INTERNAL bool fp16_stream_preferred(int64_t batch, int64_t num_kv_heads, int64_t head_dim,
                                         int64_t total_tokens, int64_t max_tokens);

// Chunks of at most 128 pages, at most 16 a sequence, covering the block table.
IRIS_INTERNAL bool fp16_stream_plan_fits(int64_t max_pages, int32_t chunk_pages, int32_t max_chunks);

// Chunk plan (pages a chunk, chunks a sequence); kInvalidArgument when the
// block table needs chunks longer than 128 pages.
IRIS_INTERNAL int fp16_stream_plan(int64_t batch, int64_t max_pages, int64_t total_tokens, int64_t max_tokens,
                                   int32_t tokens_per_split, int32_t* out_chunk_pages, int32_t* out_max_chunks);

// Split-KV workspace of a launch with max_chunks chunks a sequence.
IRIS_INTERNAL int64_t fp16_stream_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim,
                                                  int64_t max_chunks);

// Launch: batch x max_chunks workgroups of one wave a kv head.
IRIS_INTERNAL int fp16_stream_launch(const void* query, const void* k_cache, const void* v_cache,
                                     const int32_t* block_table, const int32_t* seq_lens, void* output,
                                     int32_t output_is_f32, void* workspace, int64_t workspace_bytes_avail,
                                     int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                     int64_t max_pages, float softmax_scale, int32_t chunk_pages,
                                     int32_t max_chunks, void* stream);

}  // namespace iris
