/*
 * iris_hip.h -- C ABI of libiris_hip.so, the gfx950 (MI355X) implementation
 * of Iris-Kernel's compressed paged KV-cache hot path.
 *
 * Plain pointers and sizes only; every pointer is device memory (HBM) except
 * the out-parameters of iris_decode_plan.  All launches are asynchronous on
 * the given HIP stream (NULL = legacy default stream).  Every function
 * returns 0 (IRIS_OK) or one of the IRIS_ERR_* codes below; no function
 * allocates device memory.
 *
 * Cache format (README.md:64-84 and torch_eager_kv.py:203-248 of the
 * reference, Hunter2030ZeRo/Iris-Kernel):
 *   k_data, v_data   [num_pages, page_size, num_kv_heads, head_dim / 2] uint8,
 *                    two signed INT4 codes per byte, even dim in the low
 *                    nibble, codes in [-7, 7];
 *   k_scale, v_scale [num_pages, page_size, num_kv_heads, head_dim / 32] fp16,
 *                    one scale per 32 consecutive dims;
 *   a token's slot is page * page_size + offset.
 * All tensors are dense row-major.  16-byte alignment is required for key,
 * value, query, cos_cache, sin_cache, k_data and v_data; 4-byte alignment for
 * the others.
 */
#ifndef IRIS_HIP_H
#define IRIS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IRIS_OK 0
#define IRIS_ERR_INVALID_ARGUMENT 1 /* shape or size outside the supported scope */
#define IRIS_ERR_LAUNCH 2           /* the HIP runtime rejected a kernel launch */
#define IRIS_ERR_WORKSPACE 3        /* split-KV workspace missing or too small */

/* Bytes of split-KV arrival counters at the head of a decode workspace for a
 * batch of `batch` sequences: 128 uint32 per sequence, rounded up to 256. */
#define IRIS_COUNTER_BYTES(batch) ((((int64_t)(batch) * 512) + 255) / 256 * 256)

/*
 * Fused RoPE(K) + group-32 INT4 quantisation of K and V + nibble packing +
 * paged scatter.  Replaces the TileLang launch of `_rope_int4_paged_append`
 * made by `fused_rope_int4_paged_append` (src/iris_kernel/fused_kv.py:766-780;
 * kernel fused_kv.py:419-597), with the same contract: the result is
 * bit-identical to `torch_eager_append` (torch_eager_kv.py:110-337) for fp16
 * inputs and group_size == 32.  K's first rotary_dim dims are rotated and
 * the rest pass through, as in the eager path (torch_eager_kv.py:35-49); the
 * reference's fused kernel only takes rotary_dim == head_dim
 * (fused_kv.py:644-645), which its launch passes as head_dim.
 *
 *   key, value         [num_tokens, num_kv_heads, head_dim] fp16
 *   positions          [num_tokens] int32, row of cos/sin_cache per token
 *   slot_mapping       [num_tokens] int32, destination slot; < 0 = skip token
 *   cos_cache, sin_cache [max_position, rotary_dim / 2] fp16
 *   k_data .. v_scale  the cache, written in place at the valid slots only
 *
 * head_dim must be a multiple of 32 and at most 512 (the reference's fused
 * kernel takes multiples of 64, fused_kv.py:636-637; its eager path any
 * multiple of the group size); rotary_dim even, in
 * [0, head_dim] (a multiple of 16 keeps the vector RoPE path; other values
 * read each rotated dim's partner, cos and sin separately).  Like the reference
 * kernel, this function does not check slot or position ranges or duplicate
 * slots (fused_kv.py:741-759 does that on the host before launching).
 * num_pages and max_position are accepted for symmetry with the reference
 * signature and are not read.
 */
int iris_rope_int4_paged_append(const void *key, const void *value, const int32_t *positions,
                                const int32_t *slot_mapping, const void *cos_cache,
                                const void *sin_cache, void *k_data, void *v_data, void *k_scale,
                                void *v_scale, int64_t num_tokens, int64_t num_kv_heads,
                                int64_t head_dim, int64_t rotary_dim, int64_t page_size,
                                int64_t num_pages, int64_t max_position, void *stream);

/*
 * RoPE(K) + paged append into an fp16 cache.  Replaces the TileLang launch
 * of `_rope_fp16_paged_append` made by `fused_rope_fp16_append`
 * (src/iris_kernel/fused_kv.py:284-297; kernel :8-150): K's first
 * rotary_dim dims are rotated (rotate-half, cos/sin rows `positions`), the
 * remaining dims pass through, V is copied, and both are written to slot
 * slot_mapping[t] of the cache; tokens with slot < 0 are skipped.  Every
 * product and sum is rounded to fp16, so the written rows are bit-identical
 * to torch_eager_kv.apply_rope's (torch_eager_kv.py:6-49).
 *
 *   key, value           [num_tokens, num_kv_heads, head_dim] fp16
 *   positions, slot_mapping [num_tokens] int32
 *   cos_cache, sin_cache [max_position, rotary_dim / 2] fp16
 *   k_cache, v_cache     [num_pages, page_size, num_kv_heads, head_dim] fp16
 *
 * rotary_dim must be even and at most head_dim.  Slot, position and
 * duplicate checks are the caller's (fused_kv.py:263-282 does them on the
 * host); num_pages and max_position are not read.
 */
int iris_rope_fp16_paged_append(const void *key, const void *value, const int32_t *positions,
                                const int32_t *slot_mapping, const void *cos_cache, const void *sin_cache,
                                void *k_cache, void *v_cache, int64_t num_tokens, int64_t num_kv_heads,
                                int64_t head_dim, int64_t rotary_dim, int64_t page_size, int64_t num_pages,
                                int64_t max_position, void *stream);

/*
 * Group-32 INT4 quantisation + nibble packing of a dense tensor.  Replaces
 * the TileLang launch of `_quantize_pack_int4_g32` made by
 * `fused_quantize_pack_int4` (src/iris_kernel/fused_kv.py:410-416; kernel
 * :300-362): bit-identical to pack_int4(quantize_int4_groupwise(x, 32))
 * (torch_eager_kv.py:52-107).
 *
 *   x       [num_tokens, num_heads, head_dim] fp16 (16-byte aligned)
 *   packed  [num_tokens, num_heads, head_dim / 2] uint8, even dim in the low nibble
 *   scales  [num_tokens, num_heads, head_dim / 32] fp16
 *
 * head_dim must be a multiple of 64 and at most 512.
 */
int iris_quantize_pack_int4(const void *x, void *packed, void *scales, int64_t num_tokens,
                            int64_t num_heads, int64_t head_dim, void *stream);

/*
 * Split plan for iris_int4_paged_decode_attention (no reference
 * counterpart: the reference decode kernel has no split-KV,
 * README.md:425).  Chooses how many 32-token tiles each workgroup handles
 * (out_chunk_tiles), how many chunks the longest sequence can need
 * (out_max_chunks), the waves per workgroup (out_waves) and the workspace
 * size in bytes (0 when no sequence can need more than one chunk).
 * total_tokens and max_tokens (sum and max of seq_lens) may be -1 if
 * unknown; max_pages (columns of block_table) bounds them.
 * tokens_per_split > 0 and waves_per_block > 0 override the heuristic:
 * its low 8 bits ask for a wave count (16: a page-streaming kernel; 1-4:
 * the general kernel; head_dim 96, 160, 192 and 224 have a kernel of their
 * own whose wave count, 12 or 8, the plan sets; at head_dim 64 and 128 the
 * plan may return that kernel's token-page mode, 16 or 8 waves with
 * IRIS_DECODE_TOKEN_PAGES), and one of the selection
 * bits below may be or-ed in.  out_waves carries the wave count and the
 * selection bit into the launch, so a plan and its launch always run the
 * same kernel.
 * max_pages counts 16-token pages: ceil(block_table columns * page_size /
 * 16), the tokens a row addresses.  head_dim any multiple of 32 up to 512;
 * any num_q_heads / num_kv_heads.
 */
/* Kernel selection bits of waves_per_block (no reference counterpart; for
 * A/B measurements and tests).  IRIS_DECODE_PAGE_KERNEL: 16-wave plans run
 * the general page-streaming kernel even at the shapes the streaming
 * (head_dim 128, 8 kv heads, 4 query heads each) or MQA (one kv head,
 * head_dim 64) kernels cover.  IRIS_DECODE_VALU_TILE: the general kernel
 * with VALU dot products in place of MFMA (4 query heads per kv head at
 * head_dim 128, 16 at head_dim 64; other shapes are refused). */
#define IRIS_DECODE_PAGE_KERNEL 0x100
#define IRIS_DECODE_VALU_TILE 0x200
/* IRIS_DECODE_ANY_KERNEL: the any-shape kernel, which takes every head_dim
 * that is a multiple of 32 up to 512 and every page size, with fp32
 * dequantisation as the eager path does it.  iris_decode_plan sets it by
 * itself for head dims other than 64, 96, 128, 160, 192, 224 and 256 (it
 * may be asked for at those too); a caller whose page size
 * is not a multiple of 16 up to 256 must ask for it (the plan is not told
 * the page size), and iris_int4_paged_decode_attention refuses such a page
 * size without it.  At most one selection bit may be set. */
#define IRIS_DECODE_ANY_KERNEL 0x400
/* IRIS_DECODE_TOKEN_PAGES: the MFMA kernel of head dims 96-224 in its
 * token-page mode, which takes every page size (each token's page looked
 * up through the table), at head_dim 64 to 256 in steps of 32 and any
 * number of kv heads.  Asked for at other head dims, iris_decode_plan
 * returns the any-shape kernel's plan (out_waves then carries
 * IRIS_DECODE_ANY_KERNEL).  Where head_dim / 32 x num_kv_heads and
 * num_pages x page_size are both odd (the scale tensors end on half a
 * dword) the launch runs the any-shape kernel with the same plan.  It is the bit to ask for when the page
 * size is not a multiple of 16 up to 256; it may be asked for at any page
 * size.  The mode addresses token slots (page id x page_size + offset) in
 * 32 bits: a pool of at most 2^32 token slots. */
#define IRIS_DECODE_TOKEN_PAGES 0x800
int iris_decode_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                     int64_t max_pages, int64_t total_tokens, int64_t max_tokens,
                     int32_t tokens_per_split, int32_t waves_per_block, int32_t *out_chunk_tiles,
                     int32_t *out_max_chunks, int32_t *out_waves, int64_t *out_workspace_bytes);

/*
 * INT4 paged decode attention.  Replaces the TileLang launch of
 * `_int4_paged_decode_attention` made by `fused_int4_paged_decode_attention`
 * (src/iris_kernel/fused_attention.py:508-524; kernel :11-220): for each
 * sequence b and query head h, softmax(q[b,h] . K^T * softmax_scale) . V over
 * the first seq_lens[b] tokens, K/V read from kv head h / (Hq / Hkv) through
 * block_table, as `torch_eager_int4_paged_decode_attention`
 * (torch_eager_attention.py:154-239).
 *
 *   query        [batch, num_q_heads, head_dim] fp16
 *   block_table  [batch, max_pages] int32 physical page ids
 *   seq_lens     [batch] int32, each in [1, max_pages * page_size]
 *   output       [batch, num_q_heads, head_dim], fp16, or fp32 when
 *                output_is_f32 != 0 (fp32 is a test aid: the values before
 *                the final rounding)
 *   workspace    device buffer of at least the planned workspace bytes when
 *                max_chunks > 1 (may be NULL otherwise).  Its first
 *                IRIS_COUNTER_BYTES(batch) bytes are the split-KV arrival
 *                counters, 128 uint32 per sequence at the same place for
 *                every kernel, plan and shape (the FP16 decode included);
 *                the chunks of a split sequence are merged inside this
 *                launch by the workgroup that arrives last, which resets its
 *                counter, so every call leaves them at zero.  The bytes
 *                after them hold partial results that each call rewrites.
 *                Zero-fill the counter region before the first call, and
 *                again before a call whose batch exceeds the previous
 *                call's (the previous call's partials may cover the
 *                counters of the extra sequences).  Calls that share a
 *                workspace must not overlap in time (issue them on one
 *                stream).
 *   chunk_tiles, max_chunks, waves_per_block: from iris_decode_plan, as
 *                it returned them (|chunk_tiles| at most 64; a negative
 *                chunk_tiles selects the page kernel's balanced split, for
 *                ragged lengths the plan knew: it stays valid while the
 *                lengths' 32-token tiles, summed, are at most 64 *
 *                max_chunks; past that the launch writes NaN into every
 *                output element rather than a wrong result)
 *
 * Any page_size >= 1, any head_dim that is a multiple of 32 up to 512, and
 * any num_q_heads / num_kv_heads, as the eager path takes them
 * (torch_eager_attention.py:72, :93; the reference's fused path takes
 * page_size 16, head_dim 64 or 128 and at most 16 query heads per kv head,
 * fused_attention.py:390-403).  Page sizes that are not a multiple of 16
 * up to 256 need a plan made with IRIS_DECODE_TOKEN_PAGES or
 * IRIS_DECODE_ANY_KERNEL.  max_pages is the number of
 * block_table columns; plan with ceil(max_pages * page_size / 16).
 * num_pages is the pool's page count (k_data's first dimension): the
 * token-page mode reads it to stay within the scale tensors.
 * Page ids and lengths are not
 * range-checked on the device (fused_attention.py:415-429 does that on the
 * host).  Tokens of the last page beyond seq_lens[b] are read but never
 * contribute, even if their scales are NaN.
 */
int iris_int4_paged_decode_attention(const void *query, const void *k_data, const void *v_data,
                                     const void *k_scale, const void *v_scale,
                                     const int32_t *block_table, const int32_t *seq_lens,
                                     void *output, int32_t output_is_f32, void *workspace,
                                     int64_t workspace_bytes, int64_t batch, int64_t num_q_heads,
                                     int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                     int64_t num_pages, int64_t max_pages, float softmax_scale,
                                     int32_t chunk_tiles, int32_t max_chunks,
                                     int32_t waves_per_block, void *stream);

/*
 * iris_int4_paged_decode_attention without the workspace arguments.  No
 * counterpart in the reference (its decode has no split-KV workspace): for
 * callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  The
 * split-KV workspace is an 8 MiB array inside the library, one per GPU,
 * held until the process ends; a plan that needs more returns
 * IRIS_ERR_WORKSPACE without launching the decode.  The first call on a GPU
 * looks the array up (hipGetSymbolAddress); a split call whose batch exceeds
 * the previous split call's first clears the counters of its sequences with
 * a fill kernel on `stream`.  Every call on a GPU shares that GPU's array:
 * calls that overlap in time race (issue them on one stream).  Nothing is
 * allocated.  Other arguments and results as iris_int4_paged_decode_attention.
 */
int iris_int4_paged_decode_attention_noalloc(const void *query, const void *k_data, const void *v_data,
                                             const void *k_scale, const void *v_scale,
                                             const int32_t *block_table, const int32_t *seq_lens,
                                             void *output, int32_t output_is_f32, int64_t batch,
                                             int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                             int64_t page_size, int64_t num_pages, int64_t max_pages,
                                             float softmax_scale, int32_t chunk_tiles, int32_t max_chunks,
                                             int32_t waves_per_block, void *stream);

/*
 * Split plan for iris_fp16_paged_decode_attention (no reference counterpart;
 * see iris_decode_plan): pages per chunk (out_chunk_pages), chunks per
 * sequence for the widest block_table (out_max_chunks) and the workspace
 * size in bytes (0 when no sequence can need more than one chunk).
 * total_tokens and max_tokens may be -1 if unknown (the widest batch
 * block_table admits stands in); tokens_per_split > 0 steers the chunk size.
 * Two kernels: a negative out_chunk_pages (chunks of -out_chunk_pages <= 128
 * pages, at most 16 a sequence) selects the page-streaming kernel (head_dim
 * 128 with 4 or 8 kv heads, head_dim 64 with 8 or 16; the plan takes it for
 * batches of similar lengths, 4 * total_tokens >= 3 * batch * max_tokens,
 * of at least 8 sequences and 64 MB of K/V); a positive one the per-kv-head
 * kernel (at most 256 pages a chunk, at most 512 chunks per (sequence, kv
 * head)).  tokens_per_split < 0 (no reference counterpart; for A/B runs and
 * tests) asks for the page-streaming kernel with chunks of -tokens_per_split
 * tokens; unsupported shapes and chunks past 128 pages give status 1.
 */
int iris_fp16_decode_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                          int64_t max_pages, int64_t total_tokens, int64_t max_tokens,
                          int32_t tokens_per_split, int32_t *out_chunk_pages, int32_t *out_max_chunks,
                          int64_t *out_workspace_bytes);

/*
 * FP16 paged decode attention, the matched baseline of the INT4 path.
 * Replaces the TileLang launch of `_fp16_paged_decode_attention` made by
 * `fused_fp16_paged_decode_attention` (src/iris_kernel/fused_attention.py:
 * 567-581; kernel :223-370): softmax(q . K^T * softmax_scale) . V as
 * `torch_eager_fp16_paged_decode_attention` (torch_eager_attention.py:
 * 242-294), with P rounded to fp16 before the PV product as the reference
 * kernel does.
 *
 *   query        [batch, num_q_heads, head_dim] fp16
 *   k_cache, v_cache [num_pages, page_size, num_kv_heads, head_dim] fp16
 *   block_table, seq_lens, output, output_is_f32: as for
 *                iris_int4_paged_decode_attention
 *   workspace    at least the planned workspace bytes when max_chunks > 1,
 *                with the counter region of iris_int4_paged_decode_attention
 *                (the same layout, shared with the INT4 kernels): zero-filled
 *                before the first call and before a call whose batch exceeds
 *                the previous call's.  Calls sharing a workspace must not
 *                overlap in time.
 *   chunk_pages, max_chunks: from iris_fp16_decode_plan (the sign of
 *                chunk_pages selects the kernel)
 *
 * page_size must be 16, head_dim 64 or 128, num_q_heads / num_kv_heads at
 * most 16 (fused_attention.py:390-403).  16-byte alignment is required for
 * query, k_cache and v_cache.  Tokens of the last page beyond seq_lens[b]
 * never contribute, whatever their bytes.
 */
int iris_fp16_paged_decode_attention(const void *query, const void *k_cache, const void *v_cache,
                                     const int32_t *block_table, const int32_t *seq_lens, void *output,
                                     int32_t output_is_f32, void *workspace, int64_t workspace_bytes,
                                     int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                     int64_t head_dim, int64_t page_size, int64_t num_pages,
                                     int64_t max_pages, float softmax_scale, int32_t chunk_pages,
                                     int32_t max_chunks, void *stream);

/*
 * Data-dependent input checks of the decode wrappers, on the device.
 * Replaces the host-side checks of `_validate_common_decode_inputs`
 * (src/iris_kernel/fused_attention.py:373-434): over seq_lens [batch] and
 * block_table [batch, max_pages] (int32, dense), one launch computes
 *   state[0] = 1 if some seq_lens[b] <= 0
 *   state[1] = 1 if some ceil(seq_lens[b] / page_size) > max_pages
 *   state[2] = 1 if some block_table[b, j] with j < ceil(seq_lens[b] /
 *              page_size) lies outside [0, num_pages)
 *   state[3] = sum of max(seq_lens[b], 0)
 *   state[4] = max of seq_lens[b] (when every length is positive)
 * state is a device buffer of 16 int64, zero-filled before its first use;
 * state[8..16) is the launch's accumulators, left at zero.  The results go
 * to host_results[0..5) when it is not NULL: pinned host memory from
 * hipHostMalloc (torch's pin_memory), written by the kernel through its
 * device mapping; the call then synchronises `stream` and returns with the
 * results in place.  Else they go to state[0..5) and the call returns after
 * the launch.  Returns 1 if host_results is not such memory.  Calls sharing a state buffer must not overlap in time
 * (issue them on one stream).
 */
int iris_decode_check(const int32_t *seq_lens, const int32_t *block_table, int64_t batch,
                      int64_t max_pages, int64_t num_pages, int64_t page_size, int64_t *state,
                      int64_t *host_results, void *stream);

/*
 * Data-dependent input checks of the append wrappers, on the device.
 * Replaces the host-side checks of fused_kv.py:741-759 (INT4 append) and
 * fused_kv.py:263-282 (FP16 append): over slot_mapping and positions
 * [num_tokens] (int32, dense), tokens with slot < 0 skipped, one launch
 * computes
 *   state[0] = 1 if some slot >= 0
 *   state[1] = 1 if two tokens share a slot in [0, num_slots)
 *   state[2] = 1 if some slot >= num_slots
 *   state[3] = 1 if some position of a token with slot >= 0 is < 0
 *   state[4] = 1 if some such position is >= num_positions
 * (results numbered as state[0..5) here; they go to host_results or state
 * as in iris_decode_check).  Duplicates among slots >= num_slots are not
 * reported (the reference reports them before the range error; a caller
 * that sees result 2 decides that order itself).  state: 16 int64 and
 * bitmap: bitmap_words >= ceil(num_slots / 32) uint32, both zero-filled
 * before first use and left zero by each launch except state[0..5).  Calls
 * sharing them must not overlap in time (issue them on one stream).
 */
int iris_append_check(const int32_t *slot_mapping, const int32_t *positions, int64_t num_tokens,
                      int64_t num_slots, int64_t num_positions, int64_t *state, uint32_t *bitmap,
                      int64_t bitmap_words, int64_t *host_results, void *stream);

/* Library version: major * 10000 + minor * 100 + patch. */
int iris_version(void);

#ifdef __cplusplus
}
#endif

#endif /* IRIS_HIP_H */
