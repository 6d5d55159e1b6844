// Host entry points of the decode kernel for head dims 96, 160, 192 and 224
// and of its token-page mode (decode_hd.hip), called by the C ABI in decode.hip.
#pragma once

#include <stdint.h>

#define IRIS_INTERNAL __attribute__((visibility("hidden")))

namespace iris {

// head_dim 96, 160, 192 or 224 (any number of kv heads and of query heads
// per kv head; pages of 16 m tokens).
IRIS_INTERNAL bool hd_supported(int64_t head_dim);

// Token-page mode (any page size, tokens looked up one by one): head_dim
// 64 to 256 in steps of 32, any number of kv heads.
IRIS_INTERNAL bool hd_tok_supported(int64_t head_dim, int64_t num_kv_heads);

// Waves of the kernel's workgroups at head_dim (16 at 64, 12 at 96, 8 above).
IRIS_INTERNAL int hd_waves(int64_t head_dim);

// Chunk plan: chunk_tiles (a multiple of the waves, at most 32 tiles of 32
// tokens a wave) and max_chunks, a chunk about one CU's share of the tiles of
// the (sequence, kv head, block of 16 query heads) units; workspace bytes for
// the split.  total_tokens / max_tokens may be -1 (unknown).  max_pages
// counts the 16-token pages a table row addresses (rounded up in token-page
// mode).
IRIS_INTERNAL int hd_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                          int64_t max_pages, int64_t total_tokens, int64_t max_tokens, int32_t tokens_per_split,
                          bool token_pages,
                          int32_t* out_chunk_tiles, int32_t* out_max_chunks, int32_t* out_waves,
                          int64_t* out_workspace_bytes);

// Launch: num_kv_heads x ceil(g / 16) x (batch x max_chunks, rounded up to
// 8) workgroups (the kv heads and query blocks of one unit on one XCD) of
// `waves` (= hd_waves) waves; max_pages counts 16-token pages, page_code is
// virtual_page's (common.h).  token_pages: pages of page_size tokens (any
// size), the grid covering bt_cols x page_size tokens; page_code unused.
IRIS_INTERNAL int hd_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale,
                            const void* v_scale, const int32_t* block_table, const int32_t* seq_lens, void* output,
                            int32_t output_is_f32, void* workspace, int64_t workspace_bytes_avail, int64_t batch,
                            int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_pages,
                            int64_t bt_cols, int32_t page_code, int64_t page_size, bool token_pages,
                            float softmax_scale, int32_t chunk_tiles, int32_t max_chunks, int32_t waves,
                            void* stream);

}  // namespace iris
