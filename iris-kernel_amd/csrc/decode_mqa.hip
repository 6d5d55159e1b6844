// INT4 paged decode attention for gfx950 (MI355X): the MQA streaming kernel.
//
// Replaces the TileLang kernel `_int4_paged_decode_attention`
// (src/iris_kernel/fused_attention.py:11-220 in Hunter2030ZeRo/Iris-Kernel)
// for one kv head, head_dim 64 and up to 16 query heads (multi-query
// attention: every query head reads the same K and V); it computes the
// result of `torch_eager_int4_paged_decode_attention`
// (src/iris_kernel/torch_eager_attention.py:154-239).
//
// Streaming
// ---------
// A 16-token page of one kv head at head_dim 64 is 512 bytes of K codes,
// 512 of V codes and 64 of each scale tensor, four small regions.  A
// workgroup of 16 waves owns (sequence, chunk of 32-token tiles); wave w
// streams tiles w, w + 16, w + 32, ... of the chunk through a ring of its
// own in LDS, with no workgroup barrier between tiles:
// * a slot (one tile, 2304 bytes) is filled by three loads straight into
//   LDS: K and V codes (one 16-byte-a-lane load each, covering both pages)
//   and the scales (one dword a lane: K of both pages, then V);
// * one tile is in flight while the previous one is computed (a barrier a
//   step across the 16 waves, with shared scale loads, measured 23.4 us
//   against 21.5 us at configuration 4; deeper rings measured slower);
// * a wave's page ids sit in 16 lanes of one register (read with
//   v_readlane: an LDS table measured 1 us slower, its reads on every
//   tile's load path).
//
// Compute: one tile a wave at a time
// -----------------------------------
// Wave w computes its tiles one at a time, a whole 32-token tile each, with the
// 16 query heads as the MFMA columns (v_mfma_f32_16x16x32_f16):
// * QK: S^T[t][h] = sum_g ks[t][g] * sum_{d in g} (K codes of 16 tokens,
//   one 32-dim group: A) x (q, B); the K codes enter as exact fp16
//   subnormals (nibble + 8), the offset removed by the accumulator's initial
//   value, the K scale applied per (token, group) to the fp32 result;
// * fp32 online softmax in base 2 with lazy rescaling; a head's 32 scores
//   sit in the four 16-lane rows of its column;
// * PV: O^T[d][h] += V codes transposed (A, ds_read_b64_tr_b8) x (p *
//   v_scale rounded once to fp16, B).  The C layout of S^T is the B layout
//   of PV, so p never moves between lanes.  The V codes' +8 offset is a
//   fifth MFMA per group (a constant A operand times the same B), so the
//   weights are never summed on the VALU.
// The 16 waves' softmax states are combined through LDS at the end.
//
// Split-KV: sequences longer than one chunk publish (m, l, o / l) per query
// head; the last chunk to arrive merges them in the same launch.
#include "common.h"
#include "decode_mqa.h"
#include "iris_hip.h"

namespace iris {
namespace mq {

constexpr int kTile = 32;
constexpr int kWaves = 16;
// A wave's ring slots: kRing - 1 tiles in flight while one is computed
// (three or four slots measured 1.3-2.4 us slower at configuration 4).
constexpr int kRing = 2;
constexpr int kJobs = 3;              // loads per wave per tile (K codes, V codes, both scales)
constexpr int kMaxChunkTiles = 128;   // a wave's 2 * 128 / 16 page ids fill 16 lanes
constexpr int kMaxChunks = 64;
constexpr int kMergeBatch = 8;
constexpr int kSC1 = 16;  // cache-policy bit sc1: device-coherent access
constexpr int kNT = 2;    // cache-policy bit nt: streaming

constexpr int D = 64, G = 2;
constexpr uint32_t KPAGE = 16 * 32;  // code bytes of a page (per tensor)
constexpr uint32_t SPAGE = 16 * 4;   // scale bytes of a page (per tensor)
// A wave's slot (one tile): [K codes 1 KiB][V codes 1 KiB][K scales 128 B]
// [V scales 128 B]; wave w's ring is slots w * kRing .. w * kRing + kRing - 1.
constexpr int K_OFF = 0, V_OFF = 1024, KS_OFF = 2048, VS_OFF = 2048 + 128, SLOT = 2304;
constexpr int LDS_BYTES = kWaves * kRing * SLOT;
static_assert(2 * kMaxChunkTiles / kWaves <= 64, "a wave's page ids fit its lanes");
// Epilogue (over the ring once the loop is done): per wave [m 16][l 16]
// [o 16 heads x 65 (64 dims, padded)] fp32.
constexpr int EPI_ROW = 65;
constexpr int EPI_FLOATS = 32 + 16 * EPI_ROW;
constexpr int CTL_OFF = kWaves * EPI_FLOATS * 4;
static_assert(CTL_OFF + 16 <= LDS_BYTES, "epilogue inside the ring");
static_assert(LDS_BYTES <= 160 * 1024, "LDS of a CU");

typedef int int2v_t __attribute__((ext_vector_type(2)));
typedef float float2v_t __attribute__((ext_vector_type(2)));
#define IRIS_LDS __attribute__((address_space(3)))

struct Args {
    const half_t* q;
    const uint8_t* k_data;
    const uint8_t* v_data;
    const uint8_t* k_scale;
    const uint8_t* v_scale;
    const int32_t* block_table;
    const int32_t* seq_lens;
    void* out;
    uint32_t* counters;  // counter of sequence b at b * kCountersPerSeq; zero between calls
    float* part_o;       // [B][max_chunks][16][64] o / l of each chunk
    float* part_ml;      // [B][max_chunks][16][2] (m, l), base-2 logits
    int out_f32;
    int n_q_heads, max_chunks, chunk_tiles;
    int max_pages;            // 16-token pages a block-table row addresses
    int bt_cols, page_shift;  // block-table columns; the page code of virtual_page (page_size = 16 m)
    float log2_scale;
};

// K operand: eight codes (one dword, low nibble first) -> fp16 subnormals in
// the order d0, d4, 16*d1, 16*d5, d2, d6, 16*d3, 16*d7 (units of 2^-24,
// codes offset by +8).  Each half is one v_bitop3 ((x ^ c) & m).
__device__ __forceinline__ half8_t k_operand(uint32_t x) {
    const uint32_t y = x >> 8;
    const u32x4_t r = {(x ^ 0x00080008u) & 0x000F000Fu, (x ^ 0x00800080u) & 0x00F000F0u,
                       (y ^ 0x00080008u) & 0x000F000Fu, (y ^ 0x00800080u) & 0x00F000F0u};
    return __builtin_bit_cast(half8_t, r);
}

// V operands from the 8 bytes of one transposed read (byte k' = token slot
// k'): lo = low nibbles (even dim), hi = 16 * high nibbles (odd dim), in the
// slot order k' = 0, 2, 1, 3, 4, 6, 5, 7.
__device__ __forceinline__ void v_operands(int2v_t w, half8_t& lo, half8_t& hi) {
    const uint32_t a = (uint32_t)w[0], b = (uint32_t)w[1];
    const uint32_t a8 = a >> 8, b8 = b >> 8;
    const u32x4_t l = {(a ^ 0x00080008u) & 0x000F000Fu, (a8 ^ 0x00080008u) & 0x000F000Fu,
                       (b ^ 0x00080008u) & 0x000F000Fu, (b8 ^ 0x00080008u) & 0x000F000Fu};
    const u32x4_t h = {(a ^ 0x00800080u) & 0x00F000F0u, (a8 ^ 0x00800080u) & 0x00F000F0u,
                       (b ^ 0x00800080u) & 0x00F000F0u, (b8 ^ 0x00800080u) & 0x00F000F0u};
    lo = __builtin_bit_cast(half8_t, l);
    hi = __builtin_bit_cast(half8_t, h);
}
// Byte (token slot) k' held by each slot of the V operands.
constexpr int kVSlotByte[8] = {0, 2, 1, 3, 4, 6, 5, 7};

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// v_permlane32_swap / v_permlane16_swap as opaque instructions (through the
// builtins the compiler folds a swap of a value with itself); the s_nop
// covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// max / sum over the four 16-lane rows (lanes n, n + 16, n + 32, n + 48).
__device__ __forceinline__ float row_max4(float x) {
    uint32_t a = as_u32(x), b = a;
    swap32(a, b);
    uint32_t c = as_u32(__builtin_elementwise_maximum(as_f32(a), as_f32(b))), d = c;
    swap16(c, d);
    return __builtin_elementwise_maximum(as_f32(c), as_f32(d));
}
__device__ __forceinline__ float row_sum4(float x) {
    uint32_t a = as_u32(x), b = a;
    swap32(a, b);
    uint32_t c = as_u32(as_f32(a) + as_f32(b)), d = c;
    swap16(c, d);
    return as_f32(c) + as_f32(d);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const IRIS_LDS void*)p;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS reads of data that direct-to-LDS loads wrote are inline assembly that
// waits for its own results: the compiler cannot tell them from the loads
// still streaming into the other slots and would wait for those too.  The
// wave's own vmcnt wait precedes every read of a slot.
// All of a tile's reads at once: K (four dwords, (half e, group g) 256
// bytes apart), K and V scales (16 bytes of page e, 64 bytes apart) and the
// transposed V reads of both groups.
__device__ __forceinline__ void lds_tile_reads(uint32_t k, uint32_t ks, uint32_t vs, uint32_t v0, uint32_t v1,
                                               uint32_t (&kw)[4], u32x4_t (&ksc)[2], u32x4_t (&vsc)[2],
                                               int2v_t (&w)[2]) {
    asm volatile(
        "ds_read_b32 %0, %10\n\t"
        "ds_read_b32 %1, %10 offset:256\n\t"
        "ds_read_b32 %2, %10 offset:512\n\t"
        "ds_read_b32 %3, %10 offset:768\n\t"
        "ds_read_b128 %4, %11\n\t"
        "ds_read_b128 %5, %11 offset:64\n\t"
        "ds_read_b128 %6, %12\n\t"
        "ds_read_b128 %7, %12 offset:64\n\t"
        "ds_read_b64_tr_b8 %8, %13\n\t"
        "ds_read_b64_tr_b8 %9, %14\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(kw[0]), "=&v"(kw[1]), "=&v"(kw[2]), "=&v"(kw[3]), "=&v"(ksc[0]), "=&v"(ksc[1]), "=&v"(vsc[0]),
          "=&v"(vsc[1]), "=&v"(w[0]), "=&v"(w[1])
        : "v"(k), "v"(ks), "v"(vs), "v"(v0), "v"(v1)
        : "memory");
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void store_sc1(float v, float* p) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_sc1(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The scalars the prologue needs come first, as separate arguments: built
// with -mllvm -amdgpu-kernarg-preload-count=9 they arrive in SGPRs with the
// wave, so the page-id and sequence-length loads do not wait for a
// kernel-argument load first (the Args copies are the same values).
__global__ __launch_bounds__(64 * kWaves) void int4_decode_mqa_kernel(
    const int32_t* p_seq_lens, const int32_t* p_block_table, const half_t* p_q, int p_max_chunks, int p_chunk_tiles,
    int p_bt_cols, int p_max_pages, int p_page_shift, int p_n_q_heads, Args a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15;   // MFMA row (A) or column (B, C): token or query head
    const int jq = lane >> 4;  // MFMA k-chunk (A, B) or row quad (C)

    // chunk slowest, sequences rotated by the chunk (rotate_back in common.h)
    const int batch = gridDim.x / p_max_chunks;
    const int chunk = blockIdx.x / batch, b = rotate_back(blockIdx.x - chunk * batch, chunk, batch);
    const int t_begin = chunk * p_chunk_tiles;
    const int p0 = 2 * t_begin;  // first 16-token page of the chunk
    const int32_t* bt = p_block_table + (int64_t)b * p_bt_cols;

    // ---- the chunk's page ids (thread j: page p0 + j, clamped into the
    // table row) and q are in flight together with the sequence length.
    // Lane L < 16 of wave w: the page id of chunk page 2 (16 (L >> 1) + w) +
    // (L & 1), clamped into the table row (this wave's tiles' pages).
    int my_pid = 0;
    if (lane < 2 * (kMaxChunkTiles / kWaves))
        my_pid = virtual_page(bt, min(p0 + 2 * (kWaves * (lane >> 1) + wave) + (lane & 1), p_max_pages - 1),
                              p_page_shift);
    // q as the QK B operand: lane (head n, k-chunk jq) holds dims
    // 32 g + 8 jq .. + 7 of head n (zero for n >= the query heads).
    const bool col_valid = n < p_n_q_heads;
    u32x4_t qraw[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        qraw[g] = u32x4_t{0, 0, 0, 0};
        if (col_valid)
            qraw[g] = *reinterpret_cast<const u32x4_t*>(p_q + ((int64_t)b * p_n_q_heads + n) * D + 32 * g + 8 * jq);
    }
    const int seq_len = p_seq_lens[b];
    asm volatile("" ::: "memory");  // keeps the loads above issued before the early return below

    const int n_tiles = (seq_len + kTile - 1) / kTile;
    if (t_begin >= n_tiles) return;  // uniform over the workgroup
    const int t_end = min(t_begin + p_chunk_tiles, n_tiles);
    const int n_ct = t_end - t_begin;
    const int n_steps = (n_ct + kWaves - 1) / kWaves;
    const int n_chunks = (n_tiles + p_chunk_tiles - 1) / p_chunk_tiles;
    const int last_lp = (seq_len + 15) / 16 - 1;
    // Table entries past jlim (pages past the sequence or the chunk) are
    // never read: a lookup is clamped to the last page that holds tokens.
    const int jlim = min(last_lp - p0, 2 * n_ct - 1);

    // ---- this wave's loads of its tile number s (chunk-relative tile
    // 16 s + wave) into its ring slot s % kRing.  Per-lane parts:
    // * K, 1 KiB at K_OFF: position P = 16 (2 e + g) + m holds token m of
    //   page e, dims of group g (16 bytes), so lane (m, k-chunk c) reads
    //   dword c of position 16 (2 e + g) + m;
    // * V, 1 KiB at V_OFF: position 2 tau + p holds chunk p ^ (tau & 1) of
    //   token tau (tau = 16 e + row), so the transposed reads of a group hit
    //   every bank once;
    // * scales, 256 B at KS_OFF: the 64 bytes of K scales of pages 0 and 1,
    //   then those of V, one dword a lane.
    const uint32_t k_lane = (uint32_t)((lane & 15) * 32 + ((lane >> 4) & 1) * 16);
    const int v_tau = lane >> 1;
    const uint32_t v_lane = (uint32_t)((v_tau & 15) * 32 + 16 * ((lane & 1) ^ (v_tau & 1)));
    const uint32_t s_lane = (uint32_t)(4 * (lane & 15));
    const uint8_t* const s_base = lane >= 32 ? a.v_scale : a.k_scale;
    uint8_t* const ring = smem + wave * kRing * SLOT;

    auto issue = [&](int s) __attribute__((always_inline)) {
        uint8_t* const dst = ring + (s % kRing) * SLOT;
        const int t = kWaves * s + wave;  // chunk-relative tile
        // the tile's first page is within jlim; a second page past it is the first again
        const int pa = __builtin_amdgcn_readlane(my_pid, 2 * s);
        const int pb = 2 * t + 1 > jlim ? pa : __builtin_amdgcn_readlane(my_pid, 2 * s + 1);
        const uint64_t pg = (uint64_t)(uint32_t)((lane >> 5) ? pb : pa);  // K and V: lanes 32-63 read page e = 1
        const uint64_t ps = (uint64_t)(uint32_t)(((lane >> 4) & 1) ? pb : pa);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(a.k_data + pg * KPAGE + k_lane),
                                         (IRIS_LDS void*)(dst + K_OFF), 16, 0, kNT);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(a.v_data + pg * KPAGE + v_lane),
                                         (IRIS_LDS void*)(dst + V_OFF), 16, 0, kNT);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(s_base + ps * SPAGE + s_lane),
                                         (IRIS_LDS void*)(dst + KS_OFF), 4, 0, kNT);
    };
    // This wave's tiles: 16 s + wave < n_ct.
    const int n_my = n_ct > wave ? (n_ct - wave + kWaves - 1) / kWaves : 0;
#pragma unroll
    for (int s = 0; s < kRing - 1; ++s)
        if (s < n_my) issue(s);

    // ---- q operands (in the order of k_operand; high-nibble dims / 16) and
    // the accumulator start that removes the +8 of the K codes: C row (token)
    // of column n starts at -8 * 2^-24 * (sum of q over the group, as the B
    // operand holds it).
    half8_t qm[G];
    float qinit[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const u32x4_t w = qraw[g];
        const half2_t w0 = as_half2(w[0]), w1 = as_half2(w[1]), w2 = as_half2(w[2]), w3 = as_half2(w[3]);
        const half_t s16 = (half_t)0.0625f;
        qm[g] = half8_t{w0.x, w2.x, w0.y * s16, w2.y * s16, w1.x, w3.x, w1.y * s16, w3.y * s16};
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) part += (float)qm[g][i] * ((i & 2) ? 16.0f : 1.0f);
        qinit[g] = -8.0f * 5.9604644775390625e-08f * row_sum4(part);
    }

    // ---- per-lane LDS offsets within a slot (this wave's tile)
    const uint32_t k_rd = (uint32_t)(K_OFF + 16 * n + 4 * jq);
    const uint32_t ks_rd = (uint32_t)(KS_OFF + 16 * jq);
    const uint32_t vs_rd = (uint32_t)(VS_OFF + 16 * jq);
    // Transposed V reads: lane (n, jq) supplies the 8-byte half (n & 1) of
    // token tr_tok's chunk of the group; after the 8 x 8 byte transpose it
    // holds byte column n of tokens 16 (k' >> 2) + 4 jq + (k' & 3), k' the
    // byte index (the rows of its S^T column).
    const int trk = n >> 1;
    const int tr_tok = 4 * jq + (trk & 3) + 16 * (trk >> 2);
    const uint32_t tr0 = (uint32_t)(V_OFF + tr_tok * 32 + 8 * (n & 1) + ((trk & 1) << 4));
    const uint32_t tr1 = tr0 ^ 16u;

    const float c24 = a.log2_scale * 16777216.0f;  // MFMA units -> base-2 logits
    const float lazy = 2.0f / c24;                 // rescale when a maximum grows by more (base 2)
    float m_run = -INFINITY;                       // MFMA units
    float l_part = 0.0f;
    float s_lo = INFINITY;                         // lowest valid score seen
    // oc8[g]: 8 * 2^-24 * (sum of the PV weights of group g) in every row,
    // the V code offset, accumulated by an MFMA with a constant A operand.
    float4_t oc8[G];
    float4_t o[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        oc8[g] = float4_t{0, 0, 0, 0};
        o[g][0] = o[g][1] = float4_t{0, 0, 0, 0};
    }
    const _Float16 c8 = __builtin_bit_cast(_Float16, (uint16_t)8);  // 8 * 2^-24, an exact subnormal
    const half8_t a8 = {c8, c8, c8, c8, c8, c8, c8, c8};

    // One tile whose slot has landed: s[e][i] is token 16 e + 4 jq + i,
    // query head n.
    auto compute = [&](int tile, uint32_t base) __attribute__((always_inline)) {
        const int tok0 = tile * kTile;
        const bool full = tok0 + kTile <= seq_len;
        uint32_t kw[4];
        u32x4_t ksc[2], vsc[2];
        int2v_t vw[2];
        lds_tile_reads(base + k_rd, base + ks_rd, base + vs_rd, base + tr0, base + tr1, kw, ksc, vsc, vw);
        float s[2][4];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            float4_t acc[G];
#pragma unroll
            for (int g = 0; g < G; ++g)
                acc[g] = mfma16x16x32(k_operand(kw[2 * e + g]), qm[g], float4_t{qinit[g], qinit[g], qinit[g], qinit[g]});
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const half2_t k01 = as_half2(ksc[e][i]);
                s[e][i] = __builtin_fmaf((float)k01.y, acc[1][i], __builtin_fmaf((float)k01.x, acc[0][i], 0.0f));
            }
        }
        const int nval = seq_len - tok0 - 4 * jq;
        // lowest score of the valid tokens (-inf: a non-finite K scale or
        // query); v_minimum3 (NaN-propagating: a NaN score poisons the head
        // through p anyway) needs no canonicalised operands
        auto vmin = [](float x, float y) { return __builtin_elementwise_minimum(x, y); };
        if (full) {
            s_lo = vmin(vmin(s_lo, vmin(vmin(s[0][0], s[0][1]), vmin(s[0][2], s[0][3]))),
                        vmin(vmin(s[1][0], s[1][1]), vmin(s[1][2], s[1][3])));
        } else {
            // (the count through an opaque copy made here: the compares below
            // cannot be hoisted out of this branch into every tile)
            const int nv = opaque_int(nval);
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (16 * e + i >= nv) s[e][i] = -INFINITY;
                    else s_lo = vmin(s_lo, s[e][i]);
                }
        }
        auto vmax = [](float x, float y) { return __builtin_elementwise_maximum(x, y); };
        float mx = vmax(vmax(vmax(s[0][0], s[0][1]), vmax(s[0][2], s[0][3])),
                        vmax(vmax(s[1][0], s[1][1]), vmax(s[1][2], s[1][3])));
        mx = row_max4(mx);  // finite: token tok0 < seq_len
        if (__ballot(mx > m_run + lazy) != 0) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c24);
            m_run = m_new;
            l_part *= alpha;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                oc8[g] *= alpha;
                o[g][0] *= alpha;
                o[g][1] *= alpha;
            }
        }
        const float moff = -m_run * c24;
        float p[2][4];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[e][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e][i], c24, moff));
                l_part += p[e][i];
            }
        uint32_t vsd[2][4];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) vsd[e][i] = vsc[e][i];
        if (!full) {
            // Tokens past seq_len may hold any bytes: never let their scale
            // reach the product (0 * NaN).  A real branch.
            const int nv = opaque_int(nval);
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (16 * e + i >= nv) vsd[e][i] = 0u;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            half8_t bp;
#pragma unroll
            for (int sl = 0; sl < 8; ++sl) {
                const int e = kVSlotByte[sl] >> 2, i = kVSlotByte[sl] & 3;
                bp[sl] = (half_t)__builtin_fmaf(p[e][i], (float)as_half2(vsd[e][i])[g], 0.0f);
            }
            oc8[g] = mfma16x16x32(a8, bp, oc8[g]);
            half8_t lo, hi;
            v_operands(vw[g], lo, hi);
            o[g][0] = mfma16x16x32(lo, bp, o[g][0]);
            o[g][1] = mfma16x16x32(hi, bp, o[g][1]);
        }
    };

    // ---- the pipeline, per wave (no workgroup barrier): tile s is computed
    // once this wave's loads of it have landed (vmcnt counts in order), with
    // tiles s + 1 .. s + kRing - 1 in flight; slot (s - 1) % kRing, read to
    // registers by tile s - 1, receives tile s + kRing - 1 first.
    static_assert(kRing >= 2 && kRing <= 4, "ring depth");
    const uint32_t ring_addr = lds_addr(ring);
    for (int s = 0; s < n_my; ++s) {
        const int ahead = min(n_my - 1 - s, kRing - 1);  // tiles in flight behind tile s
        if (ahead == kRing - 1) {
            issue(s + kRing - 1);
            wait_vmcnt<(kRing - 1) * kJobs>();
        } else if (kRing > 3 && ahead == 2) {
            wait_vmcnt<2 * kJobs>();
        } else if (ahead == 1) {
            wait_vmcnt<kJobs>();
        } else {
            wait_vmcnt<0>();
        }
        compute(t_begin + kWaves * s + wave, ring_addr + (uint32_t)((s % kRing) * SLOT));
    }
    wait_vmcnt<0>();
    __syncthreads();

    // ---- each wave's (m, l, o) in LDS area `wave`: [0, 16) m (base-2
    // logits), [16, 32) l, [32 + h EPI_ROW + d] o (code offset removed).
    {
        l_part = row_sum4(poison_if_neg_inf(s_lo, l_part));
        float psr[G];
#pragma unroll
        for (int g = 0; g < G; ++g) psr[g] = oc8[g][0] * 16777216.0f;
        float* const ep = reinterpret_cast<float*>(smem) + wave * EPI_FLOATS;
        if (jq == 0) {
            ep[n] = m_run * c24;
            ep[16 + n] = l_part;
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ep[32 + n * EPI_ROW + 32 * g + 2 * (4 * jq + i) + e] =
                        o[g][e][i] * (e ? 1048576.0f : 16777216.0f) - psr[g];
    }
    __syncthreads();

    // ---- the chunk's result for (query head h, dim d) = thread h * 64 + d:
    // the 16 waves' states combined (a wave without tiles has m = -inf,
    // l = 0, o = 0 and weight 0).
    const int h = threadIdx.x >> 6, d = threadIdx.x & 63;
    const float* const ep0 = reinterpret_cast<const float*>(smem);
    float mc = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mc = fmaxf(mc, ep0[w * EPI_FLOATS + h]);
    float lc = 0.0f, oc = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const float* const ep = ep0 + w * EPI_FLOATS;
        const float f = __builtin_amdgcn_exp2f(ep[h] - mc);
        lc += ep[16 + h] * f;
        oc += ep[32 + h * EPI_ROW + d] * f;
    }
    oc *= 1.0f / lc;

    const int hq = p_n_q_heads;
    auto store_out = [&](float v) {
        if (h >= hq) return;
        const int64_t idx = ((int64_t)b * hq + h) * D + d;
        if (a.out_f32) reinterpret_cast<float*>(a.out)[idx] = v;
        else reinterpret_cast<half_t*>(a.out)[idx] = (half_t)v;
    };
    if (n_chunks == 1) {
        store_out(oc);
        return;
    }

    // ---- split-KV: publish (o / l, m, l) with device-coherent stores; the
    // last chunk to arrive (the protocol of arrive_last) merges every chunk
    // of the sequence.
    const int64_t row0 = (int64_t)b * p_max_chunks;
    store_sc1(oc, a.part_o + (row0 + chunk) * (16 * D) + threadIdx.x);
    if (d == 0) {
        store_sc1(mc, a.part_ml + ((row0 + chunk) * 16 + h) * 2);
        store_sc1(lc, a.part_ml + ((row0 + chunk) * 16 + h) * 2 + 1);
    }
    wait_vmcnt<0>();
    __syncthreads();
    uint32_t* const ctl = reinterpret_cast<uint32_t*>(smem + CTL_OFF);
    if (threadIdx.x == 0)
        ctl[0] = arrive_last(a.counters + (int64_t)b * kCountersPerSeq, (uint32_t)n_chunks) ? 1u : 0u;
    __syncthreads();
    if (ctl[0] == 0) return;

    // Merge: o = sum_c w_c (o / l)_c / sum_c w_c, w_c = l_c 2^(m_c - m*),
    // kMergeBatch partials in flight, m* the running maximum; this chunk's
    // own partial from registers.
    float mstar = -INFINITY, lsum = 0.0f, acc = 0.0f;
    for (int c0 = 0; c0 < n_chunks; c0 += kMergeBatch) {
        float ov[kMergeBatch], mv[kMergeBatch], lv[kMergeBatch];
#pragma unroll
        for (int cb = 0; cb < kMergeBatch; ++cb) {
            const int c = c0 + cb;
            if (c >= n_chunks) {
                ov[cb] = 0.0f;
                mv[cb] = -INFINITY;
                lv[cb] = 0.0f;
            } else if (c == chunk) {
                ov[cb] = oc;
                mv[cb] = mc;
                lv[cb] = lc;
            } else {
                ov[cb] = load_sc1(a.part_o + (row0 + c) * (16 * D) + threadIdx.x);
                mv[cb] = load_sc1(a.part_ml + ((row0 + c) * 16 + h) * 2);
                lv[cb] = load_sc1(a.part_ml + ((row0 + c) * 16 + h) * 2 + 1);
            }
        }
        float mb = mstar;
#pragma unroll
        for (int cb = 0; cb < kMergeBatch; ++cb) mb = fmaxf(mb, mv[cb]);
        const float r = __builtin_amdgcn_exp2f(mstar - mb);  // 0 on the first batch
        acc *= r;
        lsum *= r;
#pragma unroll
        for (int cb = 0; cb < kMergeBatch; ++cb) {
            const float w = lv[cb] * __builtin_amdgcn_exp2f(mv[cb] - mb);
            acc += ov[cb] * w;
            lsum += w;
        }
        mstar = mb;
    }
    store_out(acc * (1.0f / lsum));
}

}  // namespace mq

// ------------------------------------------------------------------ host side

bool mqa_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim) {
    return num_kv_heads == 1 && head_dim == 64 && num_q_heads >= 1 && num_q_heads <= 16;
}

int mqa_waves() { return mq::kWaves; }

static int64_t mqa_workspace_bytes(int64_t batch, int64_t max_chunks) {
    const int64_t o = batch * max_chunks * 16 * mq::D * 4;
    return counter_region_bytes(batch) + (o + 255) / 256 * 256 + batch * max_chunks * 16 * 2 * 4;
}

int mqa_plan(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t max_pages, int64_t max_tokens,
             int32_t tokens_per_split, int32_t* out_chunk_tiles, int32_t* out_max_chunks, int32_t* out_waves,
             int64_t* out_workspace_bytes) {
    if (!mqa_supported(num_q_heads, 1, head_dim) || batch <= 0 || max_pages <= 0) return kInvalidArgument;
    const int64_t cap_tokens = max_pages * 16;
    if (max_tokens < 0 || max_tokens > cap_tokens) max_tokens = cap_tokens;
    // The grid covers every tile block_table can address; the lengths steer
    // the chunk size: about one workgroup per CU (256 on MI355X).
    const int64_t max_tiles = (cap_tokens + mq::kTile - 1) / mq::kTile;
    const int64_t longest = (max_tokens + mq::kTile - 1) / mq::kTile;
    int64_t chunk_tiles;
    if (tokens_per_split > 0) {
        chunk_tiles = (tokens_per_split + mq::kTile - 1) / mq::kTile;
    } else {
        int64_t per_seq = 256 / batch;
        if (per_seq < 1) per_seq = 1;
        chunk_tiles = (longest + per_seq - 1) / per_seq;
    }
    chunk_tiles = (chunk_tiles + 15) / 16 * 16;  // whole steps of 16 tiles
    if (chunk_tiles < 16) chunk_tiles = 16;
    if (chunk_tiles > mq::kMaxChunkTiles) chunk_tiles = mq::kMaxChunkTiles;
    int64_t max_chunks = (max_tiles + chunk_tiles - 1) / chunk_tiles;
    if (max_chunks > mq::kMaxChunks) {
        chunk_tiles = ((max_tiles + mq::kMaxChunks - 1) / mq::kMaxChunks + 15) / 16 * 16;
        if (chunk_tiles > mq::kMaxChunkTiles) return kInvalidArgument;
        max_chunks = (max_tiles + chunk_tiles - 1) / chunk_tiles;
    }
    *out_chunk_tiles = (int32_t)chunk_tiles;
    *out_max_chunks = (int32_t)max_chunks;
    *out_waves = mq::kWaves;
    *out_workspace_bytes = max_chunks > 1 ? mqa_workspace_bytes(batch, max_chunks) : 0;
    return kOk;
}

int mqa_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale, const void* v_scale,
               const int32_t* block_table, const int32_t* seq_lens, void* output, int32_t output_is_f32,
               void* workspace, int64_t workspace_bytes_avail, int64_t batch, int64_t num_q_heads, int64_t max_pages,
               int64_t bt_cols, int32_t page_shift, float softmax_scale, int32_t chunk_tiles, int32_t max_chunks,
               void* stream) {
    if (!mqa_supported(num_q_heads, 1, 64)) return kInvalidArgument;
    if (chunk_tiles <= 0 || chunk_tiles > mq::kMaxChunkTiles || max_chunks <= 0 || max_chunks > mq::kMaxChunks)
        return kInvalidArgument;
    if ((int64_t)chunk_tiles * max_chunks * 2 < max_pages) return kInvalidArgument;  // the grid covers every page
    const int64_t nblocks = batch * (int64_t)max_chunks;
    if (nblocks > 0x7FFFFFFF) return kInvalidArgument;
    mq::Args a;
    a.q = (const half_t*)query;
    a.k_data = (const uint8_t*)k_data;
    a.v_data = (const uint8_t*)v_data;
    a.k_scale = (const uint8_t*)k_scale;
    a.v_scale = (const uint8_t*)v_scale;
    a.block_table = block_table;
    a.seq_lens = seq_lens;
    a.out = output;
    a.out_f32 = output_is_f32;
    a.n_q_heads = (int)num_q_heads;
    a.max_pages = (int)max_pages;
    a.bt_cols = (int)bt_cols;
    a.page_shift = page_shift;
    a.max_chunks = max_chunks;
    a.chunk_tiles = chunk_tiles;
    a.log2_scale = softmax_scale * 1.4426950408889634f;
    a.counters = nullptr;
    a.part_o = a.part_ml = nullptr;
    if (max_chunks > 1) {
        const int64_t need = mqa_workspace_bytes(batch, max_chunks);
        if (workspace == nullptr || workspace_bytes_avail < need) return kWorkspaceTooSmall;
        uint8_t* const ws = (uint8_t*)workspace;
        const int64_t o = batch * max_chunks * 16 * mq::D * 4;
        a.counters = (uint32_t*)ws;
        a.part_o = (float*)(ws + counter_region_bytes(batch));
        a.part_ml = (float*)(ws + counter_region_bytes(batch) + (o + 255) / 256 * 256);
    }
    static std::atomic<uint64_t> lds_raised{0};
    if (allow_full_lds(reinterpret_cast<const void*>(&mq::int4_decode_mqa_kernel), lds_raised) != kOk)
        return kLaunchError;
    hipLaunchKernelGGL(mq::int4_decode_mqa_kernel, dim3((unsigned)nblocks), dim3(64 * mq::kWaves), mq::LDS_BYTES,
                       (hipStream_t)stream, a.seq_lens, a.block_table, a.q, a.max_chunks, a.chunk_tiles, a.bt_cols,
                       a.max_pages, a.page_shift, a.n_q_heads, a);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}

}  // namespace iris
