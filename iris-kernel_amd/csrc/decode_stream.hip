// INT4 paged decode attention for gfx950 (MI355X): the streaming kernel.
//
// Replaces the TileLang kernel `_int4_paged_decode_attention`
// (src/iris_kernel/fused_attention.py:11-220 in Hunter2030ZeRo/Iris-Kernel)
// for head_dim 128, 8 kv heads and 4 or 8 query heads per kv head (the GQA
// shapes of Llama-3-8B and of Llama-3-70B and its relatives); it computes
// the result of
// `torch_eager_int4_paged_decode_attention`
// (src/iris_kernel/torch_eager_attention.py:154-239).
//
// Streaming
// ---------
// HBM serves this cache best as whole pages read by one CU (a page of all 8
// kv heads is an 8 KiB slab per tensor): 151 MB of random 8 KiB pages plus
// their scales stream in 23.6 us on MI355X with 16 waves a CU and two or
// three 1 KiB loads in flight per wave, while 128- or 256-byte head slices
// read by different CUs take 25.7-27.8 us and deeper queues 26-27 us.  So:
// * a workgroup of 16 waves owns (sequence, chunk of 32-token tiles) and
//   reads every kv head of each page;
// * every load moves 1 KiB straight into LDS (buffer_load ... lds);
// * a ring of four slots, two in flight.  Slot s holds the K pages and K
//   scales of tile s and the V pages and V scales of tile s - 1 (36 loads:
//   each wave one K and one V load, waves 0-3 one scale load each).
//
// Compute: two wave sets, one barrier per step
// --------------------------------------------
// Wave w works on kv head w % 8 for the tiles of parity w / 8.  A tile is
// computed in two halves on consecutive steps: the first half (QK and the
// row maxima) on step s reads the K half of slot s; the second (online
// softmax update and PV) on step s + 1 reads the V half of slot s + 1.  On
// every step one set runs first halves and the other set second halves, so
// all 16 waves compute while three slots stream in; the step's barrier both
// publishes slot s and frees slot s - 1 for tile s + 3.
// * QK with the query as the MFMA A operand and K as B
//   (v_mfma_f32_16x16x32_f16): A row (h, g) = query head h, scale group g;
//   a lane of k-chunk jq holds 32 dims of group jq, and A row (h, g) is
//   zero unless g == jq, so C row (h, g) sums group g only.  C lane (token
//   column n, jq) then holds the 4 groups of head jq for one token: the K
//   scale (per token and group) is applied in the lane and the score is
//   4 FMAs, with no cross-lane sum.
// * Codes enter the MFMA as exact fp16 subnormals (nibble + 8), the offset
//   removed by the accumulator's initial value (Q side) and by a running sum
//   of the PV weights (V side).
// * Two MFMA chains per tile, columns n -> tokens T_e(n) = 16 (n >> 3) +
//   4 ((n & 7) >> 1) + (n & 1) + 2 e, so a lane's two scores are tokens t
//   and t + 2, adjacent in the PV operand order below.
// * fp32 online softmax in base 2 with lazy rescaling: a head's 32 scores
//   sit in one 16-lane row (2 per lane); the row maximum is 4 DPP steps.
// * PV with V as the B operand (transposed reads, ds_read_b64_tr_b8) and
//   A row (h, g) = p[h, t] * v_scale[t, g] rounded once to fp16, moved into
//   the A layout through a per-kv-head LDS area (4 dword writes, one 16-byte
//   read).  A PV MFMA covers 16 dims of one group; its C rows (h, g) are
//   kept, the others discarded.
// * The two sets' softmax states of a kv head are combined in the epilogue.
//
// 8 query heads per kv head (GQ 8): the same MFMA counts per tile, the rows
// pairing heads with groups two at a time.
// * QK: A row (h, e) = head h (8), e in {0, 1}; MFMA (P, m) covers groups
//   2 P and 2 P + 1, k-chunks jq = 0, 1 of group 2 P and 2, 3 of group
//   2 P + 1 (16 dims of each group an MFMA, two MFMAs a pair), A row (h, e)
//   zero unless e == jq >> 1.  Accumulator P's C lane (token column n, jq)
//   holds groups 2 P, 2 P + 1 of heads 2 jq and 2 jq + 1: each score is still
//   4 FMAs, two heads a lane.
// * PV: A row (h, e) = p[h, t] * v_scale[t, 2 P + e] for group pair P (two
//   A operands a tile, through the P area one after the other); the
//   transposed V reads take 8 bytes of group 2 P and 8 of group 2 P + 1, so
//   B column n is a byte column of group 2 P + (n >> 3) and half of each
//   MFMA's C rows are kept (a quarter at GQ 4).
// * Loop: 268 VALU and 16 MFMA per two steps a wave against 209 and 16 at
//   GQ 4, for twice the query heads.
// * Chunk mode only; its partials (32 KiB a chunk at 64 query heads) merge in
//   two levels, groups of 8 chunks.
//
// Split-KV: sequences longer than one chunk publish (m, l, o / l) per query
// head; the last chunk to arrive merges them in the same launch.
#include "common.h"
#include "decode_stream.h"
#include "iris_hip.h"

namespace iris {
namespace st {

constexpr int kTile = 32;
constexpr int kPage = 16;
constexpr int kWaves = 16;
constexpr int kSlots = 4;           // ring slots
constexpr int kAhead = 2;           // slots in flight (three measured 0.4 us slower at cfg2)
constexpr int kJobs = 3;            // loads per wave per slot
constexpr int kMaxChunkTiles = 64;  // a chunk's 128 page ids fill two VGPRs
constexpr int kMaxChunks = 64;      // partials the merge reads
constexpr int kMergeBatch = 8;      // partials in flight per thread in the merge
// Balanced mode: a long sequence's pieces (up to 18 at configuration 3) in
// two round trips of 12 instead of three of 8; the merge after the last
// arrival is on the critical path there (53.7-54.0 against 56.8-57.4 us).
// 16 spilled 43 VGPRs (67.7 us).
constexpr int kMergeBatchSeg = 12;
// Chunks merged by the last of each group (two levels past 32): one merge
// reads a partial in about 0.1 us past its ~1.2 us latency, a second level
// costs a publish, an arrival and another merge's latency, so one level is
// the faster up to about 32 partials (configuration 3: up to 20 a sequence).
constexpr int kMergeGroup = 32;
constexpr int kMaxGroups = 64;      // groups merged by the last group
// Chunk mode at 8 query heads per kv head: a chunk's partial is 32 KiB at 64
// query heads (twice the GQ 4 one), and up to 64 chunks a sequence would put
// 2 MiB through the one merging CU; groups of 8 (7 partials read by each
// group's last arrival, then at most 8 group partials by the last group).
constexpr int kMergeGroup8 = 8;
constexpr int kSeqCounter = kCountersPerSeq - 1;  // a sequence's group-level arrival counter
// Balanced mode: what starting a piece costs, in 32-token tiles of
// streaming (the epilogue, publish and arrival of the piece before, the
// page-id round trip and the ring's fill: about 4.6 us at 1.25 us a tile),
// charged to every sequence when the ranges are cut.  Configuration 3
// (interleaved A/B on one box): 53.3 us at 3, 52.1 at 4, 51.8 at 5.
constexpr int kPieceCost = 5;
// Pieces one range can meet: a range has at most kMaxChunkTiles units, and
// every piece but the first takes at least kPieceCost + 1 of them.
constexpr int kMaxPieces = 40;
static_assert(kMaxChunkTiles / (kPieceCost + 1) + 2 <= kMaxPieces, "the piece list of a range");
static_assert(kMaxGroups < kSeqCounter, "group counters and the sequence counter share a sequence's region");
constexpr float kLazy = 2.0f;       // rescale when a row maximum grows by more (base 2)
constexpr int kSC1 = 16;            // cache-policy bit sc1: device-coherent access
constexpr int kNT = 2;              // cache-policy bit nt: streaming

typedef int int2v_t __attribute__((ext_vector_type(2)));
typedef float float2v_t __attribute__((ext_vector_type(2)));
#define IRIS_LDS __attribute__((address_space(3)))

// Geometry of the supported shapes: head_dim 128 (4 scale groups), GQ (4 or
// 8) query heads per kv head, HKV kv heads.
template <int HKV, int GQ_>
struct Geo {
    static constexpr int D = 128, G = 4, GQ = GQ_;
    static constexpr int NH = GQ / 4;  // query heads of a lane (the C row quad jq holds heads NH jq ..)
    static constexpr int CK = HKV * 4;           // 16-byte chunks per token row of K or V data
    static constexpr int KPAGE = 16 * HKV * 64;  // data bytes of a page (per tensor)
    static constexpr int SPAGE = 16 * HKV * 8;   // scale bytes of a page (per tensor)
    // Slot, in load order: [K p0][K p1][V p0][V p1][KS p0][KS p1][VS p0][VS p1]
    // (K of tile s, V of tile s - 1).
    static constexpr int K_OFF = 0, V_OFF = 2 * KPAGE, KS_OFF = 4 * KPAGE, VS_OFF = 4 * KPAGE + 2 * SPAGE;
    static constexpr int SLOT = 4 * KPAGE + 4 * SPAGE;
    // Per-kv-head P areas after the ring (the two waves of a kv head run
    // their PV halves on alternate steps): 16 rows (h, g) of 32 halves,
    // padded to 80 bytes so the writes and the 16-byte reads are free of
    // bank conflicts.
    static constexpr int P_ROW = 80, P_AREA = 16 * P_ROW, P_OFF = kSlots * SLOT;
    // The empty scale-load slot of waves 4-15 writes (zeros) here.
    static constexpr int SINK_OFF = P_OFF + HKV * P_AREA;
    static constexpr int EPI_AREA = (2 * GQ + GQ * D) * 4;  // one set's (m, l, o) of a kv head in the epilogue
    // The balanced mode's piece list (the ring, P areas and sink stay clear of it).
    static constexpr int LIST_OFF = SINK_OFF + 1024;
    static constexpr int LDS_MAIN = LIST_OFF + (6 * kMaxPieces + 4) * 4;
};

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
    // Split-KV slots: chunk c of sequence b owns slot row0(b) + c, row0(b) =
    // b * max_chunks in chunk mode, first(b) + b in the balanced mode (first(b)
    // = the range holding b's first tile), so slots are unique.
    float* part_o;       // [slots][Hq][D] o / l of each chunk
    float* part_ml;      // [slots][Hq][2] (m, l), base-2 logits
    float* grp_o;        // [slots][Hq][D] o / l of group gi of b at slot row0(b) + gi (more than 8 chunks)
    float* grp_ml;       // [slots][Hq][2]
    int out_f32;
    int batch, n_q_heads, max_chunks, chunk_tiles;
    int max_pages;            // 16-token pages a block-table row addresses
    int bt_cols, page_shift;  // block-table columns; the page code of virtual_page (page_size = 16 m)
    float log2_scale;
};

// ---------------------------------------------------------------- operands

// K operand: eight codes (one dword, low nibble first) -> fp16 subnormals in
// the order d0, d4, 16*d1, 16*d5, d2, d6, 16*d3, 16*d7 (units of 2^-24,
// codes offset by +8).  Each half is one v_bitop3 ((x ^ c) & m).
__device__ __forceinline__ half8_t k_operand(uint32_t x) {
    const uint32_t y = x >> 8;
    const u32x4_t r = {(x ^ 0x00080008u) & 0x000F000Fu, (x ^ 0x00800080u) & 0x00F000F0u,
                       (y ^ 0x00080008u) & 0x000F000Fu, (y ^ 0x00800080u) & 0x00F000F0u};
    return __builtin_bit_cast(half8_t, r);
}

// q (8 consecutive dims) in the order of k_operand, high-nibble dims / 16.
__device__ __forceinline__ half8_t q_operand(u32x4_t w) {
    const half2_t w0 = as_half2(w[0]), w1 = as_half2(w[1]), w2 = as_half2(w[2]), w3 = as_half2(w[3]);
    const half_t s16 = (half_t)0.0625f;
    return half8_t{w0.x, w2.x, w0.y * s16, w2.y * s16, w1.x, w3.x, w1.y * s16, w3.y * s16};
}

// V operands from the 8 bytes of one transposed read (8 tokens of one byte
// column): lo = low nibbles (even dim), hi = 16 * high nibbles (odd dim),
// both in the k-slot order of the read (slot s = token 16 r + 4 jq + i with
// 4 r + i = kVSlotByte[s]).
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

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Consecutive logical workgroup ids (the chunks of one sequence) on one XCD.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    constexpr int kXcds = 8;
    if (nblocks % kXcds != 0) return bid;
    return (bid % kXcds) * (nblocks / kXcds) + bid / kXcds;
}

__device__ __forceinline__ uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const IRIS_LDS void*)p;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Reads of tile data, which direct-to-LDS loads wrote, are inline assembly
// waiting for their own results: the compiler cannot tell them from the
// loads still streaming into the other buffers and would wait for those too.
// A vmcnt wait and a workgroup barrier precede every such read.
__device__ __forceinline__ void lds_tile_reads(uint32_t k0, uint32_t k1, uint32_t ks0, uint32_t ks1, u32x4_t& kq0,
                                               u32x4_t& kq1, u32x2_t& ksc0, u32x2_t& ksc1) {
    asm volatile(
        "ds_read_b128 %0, %4\n\t"
        "ds_read_b128 %1, %5\n\t"
        "ds_read_b64 %2, %6\n\t"
        "ds_read_b64 %3, %7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(kq0), "=&v"(kq1), "=&v"(ksc0), "=&v"(ksc1)
        : "v"(k0), "v"(k1), "v"(ks0), "v"(ks1)
        : "memory");
}
// GQ 8: each chain's K operands are two 8-byte pieces (group pairs 0 and 1).
__device__ __forceinline__ void lds_tile_reads8(uint32_t k00, uint32_t k01, uint32_t k10, uint32_t k11, uint32_t ks0,
                                                uint32_t ks1, u32x2_t (&kq)[2][2], u32x2_t& ksc0, u32x2_t& ksc1) {
    asm volatile(
        "ds_read_b64 %0, %6\n\t"
        "ds_read_b64 %1, %7\n\t"
        "ds_read_b64 %2, %8\n\t"
        "ds_read_b64 %3, %9\n\t"
        "ds_read_b64 %4, %10\n\t"
        "ds_read_b64 %5, %11\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(kq[0][0]), "=&v"(kq[0][1]), "=&v"(kq[1][0]), "=&v"(kq[1][1]), "=&v"(ksc0), "=&v"(ksc1)
        : "v"(k00), "v"(k01), "v"(k10), "v"(k11), "v"(ks0), "v"(ks1)
        : "memory");
}
__device__ __forceinline__ void lds_v_reads(uint32_t vs0, uint32_t vs1, const uint32_t (&tr)[4], u32x2_t& vsc0,
                                            u32x2_t& vsc1, int2v_t (&w)[4]) {
    asm volatile(
        "ds_read_b64 %0, %6\n\t"
        "ds_read_b64 %1, %7\n\t"
        "ds_read_b64_tr_b8 %2, %8\n\t"
        "ds_read_b64_tr_b8 %3, %9\n\t"
        "ds_read_b64_tr_b8 %4, %10\n\t"
        "ds_read_b64_tr_b8 %5, %11\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(vsc0), "=&v"(vsc1), "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
        : "v"(vs0), "v"(vs1), "v"(tr[0]), "v"(tr[1]), "v"(tr[2]), "v"(tr[3])
        : "memory");
}
// The kv head's P area: four dword writes (rows of groups 0-3, 80 bytes
// apart), then the 16-byte read of the A operand (same wave, so the writes
// are complete when the read runs).
__device__ __forceinline__ u32x4_t lds_p_transpose(uint32_t wr, const uint32_t (&pw)[4], uint32_t rd) {
    u32x4_t a;
    asm volatile(
        "ds_write_b32 %1, %2\n\t"
        "ds_write_b32 %1, %3 offset:80\n\t"
        "ds_write_b32 %1, %4 offset:160\n\t"
        "ds_write_b32 %1, %5 offset:240\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "ds_read_b128 %0, %6\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a)
        : "v"(wr), "v"(pw[0]), "v"(pw[1]), "v"(pw[2]), "v"(pw[3]), "v"(rd)
        : "memory");
    return a;
}

// GQ 8: both group pairs' A operands through the same P area, with no wait
// between the LDS operations: one wave's LDS instructions execute in program
// order, so each read sees the writes before it and the second pair's writes
// do not overtake the first pair's read.  (The same sequence with a wait
// after each step gave bit-identical results and took 7% longer at
// configuration 5.)
__device__ __forceinline__ void lds_p_transpose2(uint32_t wr, const uint32_t (&pw0)[4], const uint32_t (&pw1)[4],
                                                 uint32_t rd, u32x4_t& a0, u32x4_t& a1) {
    asm volatile(
        "ds_write_b32 %2, %3\n\t"
        "ds_write_b32 %2, %4 offset:80\n\t"
        "ds_write_b32 %2, %5 offset:160\n\t"
        "ds_write_b32 %2, %6 offset:240\n\t"
        "ds_read_b128 %0, %11\n\t"
        "ds_write_b32 %2, %7\n\t"
        "ds_write_b32 %2, %8 offset:80\n\t"
        "ds_write_b32 %2, %9 offset:160\n\t"
        "ds_write_b32 %2, %10 offset:240\n\t"
        "ds_read_b128 %1, %11\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a0), "=&v"(a1)
        : "v"(wr), "v"(pw0[0]), "v"(pw0[1]), "v"(pw0[2]), "v"(pw0[3]), "v"(pw1[0]), "v"(pw1[1]), "v"(pw1[2]),
          "v"(pw1[3]), "v"(rd)
        : "memory");
}

// Position swizzles of a page's 16-byte chunks in LDS (row = token row of
// the page, r = page within the tile, CK chunks per row):
// * K: chunk c of row `row` sits at position c ^ kkey(row, r), so the 16
//   lanes of one k-chunk (8 rows of each page) read 16 different bank
//   groups;
// * V: chunk c of tile token t (0..31) at c ^ vswz(t): a transposed read
//   over tokens of both pages hits every bank once;
// * scales: chunk (row, col) at column col ^ ((row >> 2) & 3).
__device__ __forceinline__ int kkey(int row, int r) { return (row ^ (r << 1)) & 15; }
template <int CK>
__device__ __forceinline__ int vswz(int t) { return ((t & 15) ^ (((t >> 4) & 1) * (CK / 2))) & (CK - 1); }

__device__ __forceinline__ float4_t load4_sc1(const __amdgpu_buffer_rsrc_t& rs, uint32_t off) {
    return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kSC1));
}
__device__ __forceinline__ float2v_t load2_sc1(const __amdgpu_buffer_rsrc_t& rs, uint32_t off) {
    return __builtin_bit_cast(float2v_t, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kSC1));
}
__device__ __forceinline__ void store4_sc1(float4_t v, const __amdgpu_buffer_rsrc_t& rs, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), rs, off, 0, kSC1);
}
__device__ __forceinline__ void store2_sc1(float2v_t v, const __amdgpu_buffer_rsrc_t& rs, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), rs, off, 0, kSC1);
}

template <int HKV, int GQ_, bool SEG>
// The scalars the prologue needs come first, as separate arguments: built
// with -mllvm -amdgpu-kernarg-preload-count=10 they arrive in SGPRs with the
// wave, so the sequence-length and block-table loads do not wait for a
// kernel-argument load first (the Args copies are the same values).
__global__ __launch_bounds__(64 * kWaves) void int4_decode_stream_kernel(
    const int32_t* p_seq_lens, const int32_t* p_block_table, const half_t* p_q, int p_max_chunks, int p_chunk_tiles,
    int p_bt_cols, int p_max_pages, int p_page_shift, int p_n_q_heads, int p_nblocks, Args a) {
    using L = Geo<HKV, GQ_>;
    constexpr int D = L::D, GQ = L::GQ, NH = L::NH, G = L::G, CK = L::CK, SLOT = L::SLOT;
    static_assert(GQ == 4 || GQ == 8, "4 or 8 query heads per kv head");
    constexpr uint32_t KPAGE = L::KPAGE, SPAGE = L::SPAGE;
    constexpr int PER_PAGE = L::KPAGE / 1024;  // 1 KiB loads per page of one tensor
    static_assert(kWaves == 2 * HKV && 2 * PER_PAGE == kWaves, "one K and one V load of each slot per wave");
    static_assert(L::SPAGE == 1024 && kJobs == 3, "four 1 KiB scale loads per slot, waves 0-3");
    static_assert(L::P_ROW == 80, "lds_p_transpose writes rows 80 bytes apart");
    static_assert(L::LDS_MAIN <= 160 * 1024, "LDS of a CU");
    extern __shared__ __align__(16) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15;   // MFMA row (A) or column (B, C)
    const int jq = lane >> 4;  // MFMA k-chunk (A, B) or row quad (C)
    const int kvh = wave % HKV, par = wave / HKV;  // kv head; tiles of this parity

    // ---- the pieces of work: sequence b, tiles [t_begin, t_end), the
    // piece's chunk index in its sequence and the sequence's chunk count, the
    // slot of its chunk 0.  Chunk mode (p_chunk_tiles > 0): one piece a
    // workgroup, (b, chunk) = (wg / max_chunks, wg % max_chunks), tiles
    // chunk * chunk_tiles .. (the chunks of a sequence on one XCD).
    // Balanced mode (p_chunk_tiles < 0, ragged batches): every sequence
    // stands for its tiles plus kPieceCost units (what starting a piece
    // costs: the page-id round trip, the ring's fill, the epilogue); the
    // units of all sequences laid end to end (C in all) are cut into W =
    // max_chunks equal ranges [w C / W, (w + 1) C / W), one a workgroup, and
    // a workgroup computes, one after the other, every piece of a sequence
    // whose tiles meet its range.  Chunk c of sequence b is the piece in the
    // c-th range its tiles meet; it owns workspace slot w + b (unique: the
    // ranges of a later sequence never come before an earlier one's).
    constexpr bool segmented = SEG;  // (the sign of p_chunk_tiles, a template parameter so chunk mode carries no scan)
    auto run_piece = [&](const int b, const int chunk, const int t_begin, const int t_lim, const int seg_chunks,
                         const int64_t row0) __attribute__((always_inline)) {
        const int share = segmented ? -p_chunk_tiles : p_chunk_tiles;
        const int p0 = 2 * t_begin;
        const int seq_len = p_seq_lens[b];

        // ---- page ids of the chunk (logical page p0 + i in lane i of pid0 /
        // pid1) and the raw query rows: neither depends on the sequence length,
        // so they are in flight together with its load.
        const int32_t* bt = p_block_table + (int64_t)b * p_bt_cols;
        // (every lane loads, clamped into the table; no divergent branches
        // around the loads, so none waits for another)
        int pid0 = virtual_page(bt, min(p0 + lane, p_max_pages - 1), p_page_shift);
        int pid1 = virtual_page(bt, min(p0 + 64 + lane, p_max_pages - 1), p_page_shift);
        // Query A operand of QK MFMA m (4 of them).  GQ 4: row n = (h, g) =
        // (n >> 2, n & 3), nonzero only where g == jq: dims 32 jq + 8 m .. + 7
        // (group jq) of head h.  GQ 8: row n = (h, e) = (n >> 1, n & 1) and
        // group pair P = m >> 1 (groups 2 P, 2 P + 1), nonzero only where e ==
        // jq >> 1: dims 64 P + 16 jq + 8 (m & 1) .. + 7 (group 2 P + e).
        const half_t* qh = p_q + ((int64_t)b * p_n_q_heads + kvh * GQ) * D;
        u32x4_t qraw[4];
        if constexpr (GQ == 4) {
            const half_t* qrow = qh + (n >> 2) * D + 32 * jq;
    #pragma unroll
            for (int m = 0; m < 4; ++m) qraw[m] = *reinterpret_cast<const u32x4_t*>(qrow + 8 * m);
        } else {
            const half_t* qrow = qh + (n >> 1) * D + 16 * jq;
    #pragma unroll
            for (int m = 0; m < 4; ++m)
                qraw[m] = *reinterpret_cast<const u32x4_t*>(qrow + 64 * (m >> 1) + 8 * (m & 1));
        }
        asm volatile("" ::: "memory");  // keeps the loads above issued before the early return below

        const int n_tiles = (seq_len + kTile - 1) / kTile;
        if (t_begin >= n_tiles) return;  // uniform over the workgroup
        const int t_end = segmented ? t_lim : min(t_begin + share, n_tiles);
        const int n_stages = t_end - t_begin;
        const int n_chunks = segmented ? seg_chunks : (n_tiles + share - 1) / share;
        const int last_lp = (seq_len + kPage - 1) / kPage - 1;

        // ---- this wave's three loads of a slot (the same every step); each
        // fills 1 KiB of the slot, its lanes fetching the page chunks the
        // swizzles put there:
        // * K piece `wave` of tile s: page kr, token rows 2 qq and 2 qq + 1;
        // * V piece `wave` of tile s - 1, the same rows;
        // * waves 0-3: scales KS p0, KS p1 (tile s), VS p0, VS p1 (tile s - 1);
        //   waves 4-15: an empty load into the sink.
        const int kr = wave / PER_PAGE, qq = wave % PER_PAGE;
        uint32_t k_voff, v_voff, s_voff;
        {
            const int P = qq * 64 + lane, row = P / CK, cpos = P % CK;
            k_voff = (uint32_t)(row * CK + (cpos ^ kkey(row, kr))) * 16;
            v_voff = (uint32_t)(row * CK + (cpos ^ vswz<CK>(16 * kr + row))) * 16;
            const int srow = lane >> 2, scol = lane & 3;
            s_voff = (uint32_t)(srow * 64 + ((scol ^ ((srow >> 2) & 3)) * 16));
        }
        const bool s_job = wave < 4;
        const bool s_is_v = (wave & 2) != 0;
        const int s_r = wave & 1;

        // Physical page of logical page lp (past the sequence: its last page).
        auto page_of = [&](int lp) -> int64_t {
            const int rel = min(lp, last_lp) - p0;
            return (int64_t)__builtin_amdgcn_readlane(rel < 64 ? pid0 : pid1, rel & 63);
        };
        pid0 = (int)opaque((uint32_t)pid0);
        pid1 = (int)opaque((uint32_t)pid1);

        // Slot of step s: K of tile s, V of tile s - 1.  Halves outside the
        // chunk load with zero-size descriptors (no memory access; the load still
        // writes zeros into its LDS bytes), so every wave has kJobs loads of every
        // slot in flight.
        auto issue = [&](int s) __attribute__((always_inline)) {
            uint8_t* const dst = smem + (s & (kSlots - 1)) * SLOT;
            const bool kv = s < n_stages;
            const bool vv = s >= 1 && s <= n_stages;
            const int64_t kp = kv ? page_of(2 * (t_begin + s) + kr) : 0;
            const int64_t vp = vv ? page_of(2 * (t_begin + s - 1) + kr) : 0;
            const bool sv = s_job && (s_is_v ? vv : kv);
            const int64_t sp = sv ? page_of(2 * (t_begin + s - (s_is_v ? 1 : 0)) + s_r) : 0;
            // (the page sizes are the kernel-scope constants: L::KPAGE named in
            // these descriptor expressions makes clang drop the kernel's host
            // launch stub)
            const auto krs = buf_rsrc(a.k_data + kp * KPAGE, kv ? KPAGE : 0u);
            const auto vrs = buf_rsrc(a.v_data + vp * KPAGE, vv ? KPAGE : 0u);
            const auto srs = buf_rsrc((s_is_v ? a.v_scale : a.k_scale) + sp * SPAGE, sv ? SPAGE : 0u);
            uint8_t* const kdst = dst + L::K_OFF + 1024 * wave;
            uint8_t* const vdst = dst + L::V_OFF + 1024 * wave;
            uint8_t* const sdst = s_job ? dst + L::KS_OFF + 1024 * wave : smem + L::SINK_OFF;
            const uint32_t ko = k_voff, vo = v_voff, so = s_voff;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (IRIS_LDS void*)kdst, 16, ko, 0, 0, kNT);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (IRIS_LDS void*)vdst, 16, vo, 0, 0, kNT);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (IRIS_LDS void*)sdst, 16, so, 0, 0, kNT);
        };
        // The first kAhead + 1 slots stream in while the query operands are
        // prepared (one slot more than the steady state keeps in flight: the
        // deeper first queue measured 0.2-0.3 us faster at cfg2, a fourth slot
        // and a single one slower).
    #pragma unroll
        for (int s = 0; s <= kAhead; ++s) issue(s);

        half8_t qa[4];
        {
            const bool mine = GQ == 4 ? (n & 3) == jq : (n & 1) == (jq >> 1);
    #pragma unroll
            for (int m = 0; m < 4; ++m) qa[m] = q_operand(mine ? qraw[m] : u32x4_t{0, 0, 0, 0});
        }
        // Accumulator start that removes the +8 of the K codes: C row r gets
        // -8 * 2^-24 * (sum of q over the row's group, as the A operand holds
        // it, high-nibble dims / 16 counted 16 times).  GQ 4: lane (4 h + g, g)
        // holds group g of head h in qa; C lane (n, jq) needs rows (jq, 0..3).
        // GQ 8, pair P (accumulator init[P]): lanes (2 h + e, 2 e) and (2 h + e,
        // 2 e + 1) hold halves of group 2 P + e of head h in qa[2 P], qa[2 P + 1];
        // C lane (n, jq) needs rows 4 jq + i, i.e. (2 jq + (i >> 1), i & 1).
        float4_t init[NH];
        if constexpr (GQ == 4) {
            float part = 0.0f;
    #pragma unroll
            for (int m = 0; m < 4; ++m)
    #pragma unroll
                for (int i = 0; i < 8; ++i) part += (float)qa[m][i] * ((i & 2) ? 16.0f : 1.0f);
            part *= -8.0f * 5.9604644775390625e-08f;
    #pragma unroll
            for (int g = 0; g < 4; ++g)
                init[0][g] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                          4 * (16 * g + 4 * jq + g), __builtin_bit_cast(int, part)));
        } else {
    #pragma unroll
            for (int P = 0; P < 2; ++P) {
                float part = 0.0f;
    #pragma unroll
                for (int m = 2 * P; m < 2 * P + 2; ++m)
    #pragma unroll
                    for (int i = 0; i < 8; ++i) part += (float)qa[m][i] * ((i & 2) ? 16.0f : 1.0f);
                part *= -8.0f * 5.9604644775390625e-08f;
    #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 4 * jq + i, e = i & 1;
                    const float h0 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                                   4 * (16 * (2 * e) + row), __builtin_bit_cast(int, part)));
                    const float h1 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                                   4 * (16 * (2 * e + 1) + row), __builtin_bit_cast(int, part)));
                    init[P][i] = h0 + h1;
                }
            }
        }

        // ---- per-lane LDS offsets within a slot
        // K operand of chain e: token T = 16 (n >> 3) + 4 ((n & 7) >> 1) + (n & 1) + 2 e,
        // of head kvh: GQ 4, 16 bytes = dims [32 jq, 32 jq + 32); GQ 8, pair P,
        // 8 bytes = dims [64 P + 16 jq, + 16).
        const int T0 = 16 * (n >> 3) + 4 * ((n & 7) >> 1) + (n & 1);
        uint32_t k_off[2][NH], ks_off[2], vs_off[2];
    #pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int T = T0 + 2 * e;
            const int r = T >> 4, row = T & 15;
            if constexpr (GQ == 4) {
                k_off[e][0] = (uint32_t)(L::K_OFF + r * L::KPAGE + (row * CK + ((kvh * 4 + jq) ^ kkey(row, r))) * 16);
            } else {
    #pragma unroll
                for (int P = 0; P < 2; ++P)
                    k_off[e][P] = (uint32_t)(L::K_OFF + r * L::KPAGE +
                                             (row * CK + ((kvh * 4 + 2 * P + (jq >> 1)) ^ kkey(row, r))) * 16 +
                                             8 * (jq & 1));
            }
            const int srow = row * 64 + (((kvh >> 1) ^ ((row >> 2) & 3)) * 16) + (kvh & 1) * 8;
            ks_off[e] = (uint32_t)(L::KS_OFF + r * L::SPAGE + srow);
            vs_off[e] = (uint32_t)(L::VS_OFF + r * L::SPAGE + srow);
        }
        // Transposed V reads, four a tile: lane (n, jq) points at 8 bytes of
        // token tr_tok; after the 8 x 8 byte transpose lane n holds byte column
        // n of 8 tokens (k-slot order of v_operands), the 16 byte columns being
        // the bytes the lanes n & 1 = 0 and 1 point at.  GQ 4, read g: half
        // n & 1 of group g's 16-byte chunk.  GQ 8, read 2 P + hh: half hh of the
        // chunk of group 2 P + (n & 1), so byte column n is byte 8 hh + (n & 7)
        // of group 2 P + (n >> 3).
        uint32_t tr_off[4];
        {
            const int trk = n >> 1;
            const int tr_tok = 4 * jq + (trk & 3) + 16 * (trk >> 2);
    #pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int grp = GQ == 4 ? i : 2 * (i >> 1) + (n & 1);
                const int half = GQ == 4 ? (n & 1) : (i & 1);
                tr_off[i] = (uint32_t)(L::V_OFF + (tr_tok >> 4) * L::KPAGE +
                                       ((tr_tok & 15) * CK + ((kvh * 4 + grp) ^ vswz<CK>(tr_tok))) * 16 + 8 * half);
            }
        }
        // P area of the kv head: 16 rows of 32 halves in k-slot order of the
        // tile's token blocks (block jq' = tokens 4 jq' + i of both pages), row
        // (h, g) = 4 h + g (GQ 4) or, for group pair P, (h, e) = 2 h + e (GQ 8,
        // the pairs one after the other).  Lane (n, jq) writes tokens T0 and
        // T0 + 2, k-slots 4 (n >> 3) + 2 (n & 1) and the next, of block
        // (n & 7) >> 1 in rows 4 jq .. 4 jq + 3; it reads row n, block jq.  A row
        // feeds the PV products of its group's dims; the C rows of the other
        // groups carry the wrong V scale and are discarded.
        const uint32_t p_base = lds_addr(smem + L::P_OFF + kvh * L::P_AREA);
        const uint32_t p_wr =
            p_base + (uint32_t)((jq * 4) * L::P_ROW + (((n & 7) >> 1) * 8 + 4 * (n >> 3) + 2 * (n & 1)) * 2);
        const uint32_t p_rd = p_base + (uint32_t)(n * L::P_ROW + jq * 16);

        const float c24 = a.log2_scale * 16777216.0f;  // MFMA units -> base-2 logits
        float m_run[NH], l_part[NH];  // per query head of the lane: row maximum (base-2 logits), sum of p
        float ps[NH][G];              // sums of the PV weights per head and group (V code offset)
        float4_t o[4][2];             // PV accumulators: [group][lo, hi] (GQ 4), [2 P + hh][lo, hi] (GQ 8)
    #pragma unroll
        for (int h = 0; h < NH; ++h) {
            m_run[h] = -INFINITY;
            l_part[h] = 0.0f;
    #pragma unroll
            for (int g = 0; g < G; ++g) ps[h][g] = 0.0f;
        }
    #pragma unroll
        for (int i = 0; i < 4; ++i) o[i][0] = o[i][1] = float4_t{0, 0, 0, 0};
        float t[2][NH];  // scores (base-2 logits) of tokens T0, T0 + 2: first half -> second half
        float mx[NH];    // their row maxima
    #pragma unroll
        for (int h = 0; h < NH; ++h) mx[h] = 0.0f;

        // First half of tile `stage` (K half of its slot): scores of the lane's
        // two tokens and the row maxima.  The QK chains are interleaved.  C lane
        // (n, jq) holds rows 4 jq .. 4 jq + 3 of token column n: GQ 4, the four
        // groups of head jq; GQ 8, accumulator P, groups 2 P and 2 P + 1 of heads
        // 2 jq and 2 jq + 1.
        auto first_half = [&](int stage, uint32_t base) __attribute__((always_inline)) {
            const int tok0 = (t_begin + stage) * kTile;
            u32x2_t ksc[2];
            if constexpr (GQ == 4) {
                u32x4_t kq[2];
                lds_tile_reads(base + k_off[0][0], base + k_off[1][0], base + ks_off[0], base + ks_off[1], kq[0], kq[1],
                               ksc[0], ksc[1]);
                float4_t acc[2] = {init[0], init[0]};
    #pragma unroll
                for (int e = 0; e < 2; ++e)
    #pragma unroll
                    for (int m = 0; m < 4; ++m) acc[e] = mfma16x16x32(qa[m], k_operand(kq[e][m]), acc[e]);
    #pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const half2_t k01 = as_half2(ksc[e][0]), k23 = as_half2(ksc[e][1]);
                    float s = (float)k01.x * acc[e][0];
                    s = __builtin_fmaf((float)k01.y, acc[e][1], s);
                    s = __builtin_fmaf((float)k23.x, acc[e][2], s);
                    s = __builtin_fmaf((float)k23.y, acc[e][3], s);
                    // base-2 logit; s - s is 0 for a finite score and NaN for +-inf,
                    // so a non-finite K scale or query gives NaN as the eager
                    // dequantisation does, never a -inf that would drop the token
                    t[e][0] = __builtin_fmaf(s, c24, s - s);
                }
            } else {
                u32x2_t kq[2][2];
                lds_tile_reads8(base + k_off[0][0], base + k_off[0][1], base + k_off[1][0], base + k_off[1][1],
                                base + ks_off[0], base + ks_off[1], kq, ksc[0], ksc[1]);
                float4_t acc[2][2] = {{init[0], init[1]}, {init[0], init[1]}};
    #pragma unroll
                for (int m = 0; m < 2; ++m)
    #pragma unroll
                    for (int e = 0; e < 2; ++e)
    #pragma unroll
                        for (int P = 0; P < 2; ++P)
                            acc[e][P] = mfma16x16x32(qa[2 * P + m], k_operand(kq[e][P][m]), acc[e][P]);
    #pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const half2_t k01 = as_half2(ksc[e][0]), k23 = as_half2(ksc[e][1]);
    #pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        float s = (float)k01.x * acc[e][0][2 * h];
                        s = __builtin_fmaf((float)k01.y, acc[e][0][2 * h + 1], s);
                        s = __builtin_fmaf((float)k23.x, acc[e][1][2 * h], s);
                        s = __builtin_fmaf((float)k23.y, acc[e][1][2 * h + 1], s);
                        t[e][h] = __builtin_fmaf(s, c24, s - s);  // (as above)
                    }
                }
            }
            if (tok0 + kTile > seq_len) {
    #pragma unroll
                for (int e = 0; e < 2; ++e)
                    if (tok0 + T0 + 2 * e >= seq_len)
    #pragma unroll
                        for (int h = 0; h < NH; ++h) t[e][h] = -INFINITY;
            }
            // one row a head; its maximum is finite (token tok0 < seq_len) or NaN
    #pragma unroll
            for (int h = 0; h < NH; ++h) mx[h] = row16_max(__builtin_elementwise_maximum(t[0][h], t[1][h]));
        };

        // Second half of tile `stage` (V half of the next slot): online softmax
        // (lazy rescale), PV weights w = p * v_scale (one fp16 rounding), tokens
        // T0 and T0 + 2 packed per row of the P area, and the PV products (GQ 8:
        // one group pair after the other through the same P area).
        auto second_half = [&](int stage, uint32_t base) __attribute__((always_inline)) {
            const int tok0 = (t_begin + stage) * kTile;
            u32x2_t vsc[2];
            int2v_t vw[4];
            uint32_t tra[4];
    #pragma unroll
            for (int i = 0; i < 4; ++i) tra[i] = base + tr_off[i];
            lds_v_reads(base + vs_off[0], base + vs_off[1], tra, vsc[0], vsc[1], vw);
            bool grow = false;
    #pragma unroll
            for (int h = 0; h < NH; ++h) grow = grow || mx[h] > m_run[h] + kLazy;
            if (__ballot(grow) != 0) {
                float alpha[NH];
    #pragma unroll
                for (int h = 0; h < NH; ++h) {
                    const float m_new = fmaxf(m_run[h], mx[h]);
                    alpha[h] = __builtin_amdgcn_exp2f(m_run[h] - m_new);
                    m_run[h] = m_new;
                    l_part[h] *= alpha[h];
    #pragma unroll
                    for (int g = 0; g < G; ++g) ps[h][g] *= alpha[h];
                }
    #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (GQ == 4) {
                        o[i][0] *= alpha[0];
                        o[i][1] *= alpha[0];
                    } else {  // C row 4 jq + r: head 2 jq + (r >> 1)
    #pragma unroll
                        for (int e = 0; e < 2; ++e)
    #pragma unroll
                            for (int r = 0; r < 4; ++r) o[i][e][r] *= alpha[r >> 1];
                    }
                }
            }
            float p[2][NH];
    #pragma unroll
            for (int e = 0; e < 2; ++e)
    #pragma unroll
                for (int h = 0; h < NH; ++h) {
                    p[e][h] = __builtin_amdgcn_exp2f(t[e][h] - m_run[h]);
                    l_part[h] += p[e][h];
                }
            float vs[2][G];
    #pragma unroll
            for (int e = 0; e < 2; ++e) {
                const half2_t v01 = as_half2(vsc[e][0]), v23 = as_half2(vsc[e][1]);
                vs[e][0] = (float)v01.x;
                vs[e][1] = (float)v01.y;
                vs[e][2] = (float)v23.x;
                vs[e][3] = (float)v23.y;
            }
            // tokens past seq_len: p is 0, and their scale may be anything (NaN included)
            if (tok0 + kTile > seq_len) {
    #pragma unroll
                for (int e = 0; e < 2; ++e)
                    if (tok0 + T0 + 2 * e >= seq_len) vs[e][0] = vs[e][1] = vs[e][2] = vs[e][3] = 0.0f;
            }
            const half2_t one2 = {(half_t)1.0f, (half_t)1.0f};
            if constexpr (GQ == 4) {
                uint32_t pw[G];
    #pragma unroll
                for (int g = 0; g < G; ++g) {
                    const half2_t wp = {(half_t)(p[0][0] * vs[0][g]), (half_t)(p[1][0] * vs[1][g])};
                    ps[0][g] = __builtin_amdgcn_fdot2(wp, one2, ps[0][g], false);
                    pw[g] = as_u32(wp);
                }
                const half8_t pa = __builtin_bit_cast(half8_t, lds_p_transpose(p_wr, pw, p_rd));
                // group g's 32 dims as byte columns n (even dim lo, odd hi)
    #pragma unroll
                for (int g = 0; g < G; ++g) {
                    half8_t lo, hi;
                    v_operands(vw[g], lo, hi);
                    o[g][0] = mfma16x16x32(pa, lo, o[g][0]);
                    o[g][1] = mfma16x16x32(pa, hi, o[g][1]);
                }
            } else {
                uint32_t pw[2][4];  // pair P: rows 4 jq + 2 h + e, head 2 jq + h, group 2 P + e
    #pragma unroll
                for (int P = 0; P < 2; ++P)
    #pragma unroll
                    for (int h = 0; h < 2; ++h)
    #pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const int g = 2 * P + e;
                            const half2_t wp = {(half_t)(p[0][h] * vs[0][g]), (half_t)(p[1][h] * vs[1][g])};
                            ps[h][g] = __builtin_amdgcn_fdot2(wp, one2, ps[h][g], false);
                            pw[P][2 * h + e] = as_u32(wp);
                        }
                u32x4_t pa2[2];
                lds_p_transpose2(p_wr, pw[0], pw[1], p_rd, pa2[0], pa2[1]);
    #pragma unroll
                for (int P = 0; P < 2; ++P) {
                    const half8_t pa = __builtin_bit_cast(half8_t, pa2[P]);
                    // byte columns n: bytes 8 hh + (n & 7) of group 2 P + (n >> 3)
    #pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        half8_t lo, hi;
                        v_operands(vw[2 * P + hh], lo, hi);
                        o[2 * P + hh][0] = mfma16x16x32(pa, lo, o[2 * P + hh][0]);
                        o[2 * P + hh][1] = mfma16x16x32(pa, hi, o[2 * P + hh][1]);
                    }
                }
            }
        };

        // ---- the pipeline.  Step s: wait for this wave's loads of slot s (the
        // slot s + 1 stays in flight, and s + 2 at step 0); the barrier makes
        // every wave's slot-s loads visible and frees slot s - 1, which receives
        // slot s + 2;
        // the set of parity s runs the first half of tile s, the other set the
        // second half of tile s - 1.  Every wave passes the n_stages + 1 steps'
        // barriers; each set has a loop of its own, two steps per iteration, so
        // that its halves are straight-line code.
        auto step = [&](int s) __attribute__((always_inline)) -> uint32_t {
            if (s == 0) wait_vmcnt<kAhead * kJobs>();
            else wait_vmcnt<(kAhead - 1) * kJobs>();
            __builtin_amdgcn_s_barrier();
            if (s > 0) issue(s + kAhead);
            return lds_addr(smem) + (uint32_t)((s & (kSlots - 1)) * SLOT);
        };
        if (par == 0) {
            int s = 0;
            for (; s < n_stages; s += 2) {
                first_half(s, step(s));
                second_half(s, step(s + 1));
            }
            if (s == n_stages) step(s);
        } else {
            step(0);
            int s = 1;
            for (; s < n_stages; s += 2) {
                first_half(s, step(s));
                second_half(s, step(s + 1));
            }
            if (s == n_stages) step(s);
        }
        wait_vmcnt<0>();  // the empty loads past the chunk still write LDS
        __syncthreads();

        // ---- each set's (m, l, o) of kv head kvh in LDS area `wave`:
        // [0, GQ) m, [GQ, 2 GQ) l, [2 GQ + h D, ...) o (unnormalised, code
        // offset removed); lane (n, jq) holds heads NH jq .. NH jq + NH - 1.
        {
            float psr[NH][G];
    #pragma unroll
            for (int h = 0; h < NH; ++h) {
                l_part[h] = row16_sum(l_part[h]);
    #pragma unroll
                for (int g = 0; g < G; ++g) psr[h][g] = 8.0f * row16_sum(ps[h][g]);
            }
            float* const ep = reinterpret_cast<float*>(smem + wave * L::EPI_AREA);
            if (n == 0) {
    #pragma unroll
                for (int h = 0; h < NH; ++h) {
                    ep[NH * jq + h] = m_run[h];
                    ep[GQ + NH * jq + h] = l_part[h];
                }
            }
            if constexpr (GQ == 4) {
    #pragma unroll
                for (int g = 0; g < G; ++g)
    #pragma unroll
                    for (int e = 0; e < 2; ++e)
                        ep[2 * GQ + jq * D + 32 * g + 2 * n + e] =
                            o[g][e][g] * (e ? 1048576.0f : 16777216.0f) - psr[0][g];
            } else {
                // accumulator 2 P + hh, column n: dims 16 hh + 2 (n & 7) (+ 1 for
                // hi) of group 2 P + (n >> 3), kept in C rows of that group: 2 h +
                // (n >> 3) for head 2 jq + h
                const bool odd = (n >> 3) != 0;
    #pragma unroll
                for (int P = 0; P < 2; ++P)
    #pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
    #pragma unroll
                        for (int e = 0; e < 2; ++e)
    #pragma unroll
                            for (int h = 0; h < 2; ++h) {
                                const float4_t c = o[2 * P + hh][e];
                                const float v = odd ? c[2 * h + 1] : c[2 * h];
                                const float off = odd ? psr[h][2 * P + 1] : psr[h][2 * P];
                                ep[2 * GQ + (2 * jq + h) * D + 32 * (2 * P + (n >> 3)) + 16 * hh + 2 * (n & 7) + e] =
                                    v * (e ? 1048576.0f : 16777216.0f) - off;
                            }
            }
        }
        __syncthreads();

        // ---- the chunk's result for element idx = (kv head, query head, dim),
        // 4 dims at a time: the two sets' states combined.  A set without tiles
        // (a one-tile chunk) has m = -inf, l = 0, o = 0 and weight 0.
        const int hq = p_n_q_heads;
        const int total = hq * D, n4 = total / 4;
        auto chunk4 = [&](int e4, float& m, float& l) -> float4_t {
            const int idx = 4 * e4;
            const int j = idx / (GQ * D), rem = idx - j * (GQ * D), h = rem / D, d = rem - h * D;
            const float* w0 = reinterpret_cast<const float*>(smem + j * L::EPI_AREA);
            const float* w1 = reinterpret_cast<const float*>(smem + (HKV + j) * L::EPI_AREA);
            m = fmaxf(w0[h], w1[h]);
            const float a0 = __builtin_amdgcn_exp2f(w0[h] - m), a1 = __builtin_amdgcn_exp2f(w1[h] - m);
            l = w0[GQ + h] * a0 + w1[GQ + h] * a1;
            const float4_t o0 = *reinterpret_cast<const float4_t*>(w0 + 2 * GQ + h * D + d);
            const float4_t o1 = *reinterpret_cast<const float4_t*>(w1 + 2 * GQ + h * D + d);
            return (o0 * a0 + o1 * a1) * (1.0f / l);
        };
        const int64_t out_base = (int64_t)b * total;
        auto store_out4 = [&](int e4, float4_t v) {
            if (a.out_f32) {
                *reinterpret_cast<float4_t*>(reinterpret_cast<float*>(a.out) + out_base + 4 * e4) = v;
            } else {
                const half2_t lo = {(half_t)v[0], (half_t)v[1]}, hi = {(half_t)v[2], (half_t)v[3]};
                *reinterpret_cast<u32x2_t*>(reinterpret_cast<half_t*>(a.out) + out_base + 4 * e4) =
                    u32x2_t{as_u32(lo), as_u32(hi)};
            }
        };
        if (n_chunks == 1) {
            for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
                float m, l;
                store_out4(e4, chunk4(e4, m, l));
            }
            return;
        }

        if constexpr (!SEG && GQ == 4) {
            // Chunk mode: at most 64 chunks a sequence, merged in one level.
            // ---- split-KV: publish (o / l, m, l) with device-coherent stores; the
            // last chunk to arrive merges every chunk of the sequence.
            const uint32_t part_o = (uint32_t)total * 4, part_ml = (uint32_t)hq * 8;  // bytes per partial
            const int64_t row0 = (int64_t)b * p_max_chunks;
            {
                const auto ro = buf_rsrc(a.part_o + (row0 + chunk) * total, part_o);
                const auto rm = buf_rsrc(a.part_ml + (row0 + chunk) * hq * 2, part_ml);
                for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
                    float m, l;
                    const float4_t v = chunk4(e4, m, l);
                    store4_sc1(v, ro, (uint32_t)e4 * 16);
                    if ((4 * e4) % D == 0) store2_sc1(float2v_t{m, l}, rm, (uint32_t)(4 * e4 / D) * 8);
                }
            }
            wait_vmcnt<0>();
            __syncthreads();
            uint32_t* const ctl = reinterpret_cast<uint32_t*>(smem + 2 * HKV * L::EPI_AREA);
            if (threadIdx.x == 0)
                ctl[0] = arrive_last(a.counters + (int64_t)b * kCountersPerSeq, (uint32_t)n_chunks) ? 1u : 0u;
            __syncthreads();
            if (ctl[0] == 0) return;

            // Merge the M = n_chunks partials, each thread a float4 of the output:
            // o = sum_c w_c (o / l)_c / sum_c w_c with w_c = l_c 2^(m_c - m*), the
            // partials and their (m, l) loaded together, kMergeBatch chunks at a
            // time, m* the running maximum.  This chunk's own partial comes from LDS
            // (the same values it published).
            const int M = n_chunks;
            const auto ro = buf_rsrc(a.part_o + row0 * total, part_o * (uint32_t)M);
            const auto rm = buf_rsrc(a.part_ml + row0 * hq * 2, part_ml * (uint32_t)M);
            for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
                const int h = 4 * e4 / D;
                float mstar = -INFINITY, lsum = 0.0f;
                float4_t acc = {0, 0, 0, 0};
                for (int c0 = 0; c0 < M; c0 += kMergeBatch) {
                    float4_t oc[kMergeBatch];
                    float2v_t ml[kMergeBatch];
        #pragma unroll
                    for (int cb = 0; cb < kMergeBatch; ++cb) {
                        const int c = min(c0 + cb, M - 1);
                        if (c != chunk) {
                            oc[cb] = load4_sc1(ro, (uint32_t)c * part_o + (uint32_t)e4 * 16);
                            ml[cb] = load2_sc1(rm, ((uint32_t)c * (uint32_t)hq + (uint32_t)h) * 8);
                        } else {
                            float m, l;
                            oc[cb] = chunk4(e4, m, l);
                            ml[cb] = float2v_t{m, l};
                        }
                    }
                    // past M: a repeat of partial M - 1 with weight 0
                    float mb = mstar;
        #pragma unroll
                    for (int cb = 0; cb < kMergeBatch; ++cb) mb = fmaxf(mb, ml[cb][0]);
                    const float r = __builtin_amdgcn_exp2f(mstar - mb);  // 0 on the first batch
                    acc *= r;
                    lsum *= r;
        #pragma unroll
                    for (int cb = 0; cb < kMergeBatch; ++cb) {
                        const float w = c0 + cb < M ? ml[cb][1] * __builtin_amdgcn_exp2f(ml[cb][0] - mb) : 0.0f;
                        acc += oc[cb] * w;
                        lsum += w;
                    }
                    mstar = mb;
                }
                store_out4(e4, acc * (1.0f / lsum));
            }
        } else {
            // Balanced mode (up to 8 x 64 chunks a sequence) and chunk mode at
            // GQ 8 (up to 64 chunks, partials of 32 KiB at 64 query heads): two
            // levels, in groups of MG chunks.
            // ---- split-KV: publish (o / l, m, l) with device-coherent stores; the
            // last chunk of each group of MG chunks to arrive merges the group;
            // with more than one group, the group partials go out the same way
            // and the last group to arrive merges them (two levels, so no
            // workgroup reads more than MG chunk partials or kMaxGroups group
            // partials).
            constexpr int MG = SEG ? kMergeGroup : kMergeGroup8;
            const uint32_t part_o = (uint32_t)total * 4, part_ml = (uint32_t)hq * 8;  // bytes per partial
            {
                const auto ro = buf_rsrc(a.part_o + (row0 + chunk) * total, part_o);
                const auto rm = buf_rsrc(a.part_ml + (row0 + chunk) * hq * 2, part_ml);
                for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
                    float m, l;
                    const float4_t v = chunk4(e4, m, l);
                    store4_sc1(v, ro, (uint32_t)e4 * 16);
                    if ((4 * e4) % D == 0) store2_sc1(float2v_t{m, l}, rm, (uint32_t)(4 * e4 / D) * 8);
                }
            }
            wait_vmcnt<0>();
            __syncthreads();
            uint32_t* const ctl = reinterpret_cast<uint32_t*>(smem + 2 * HKV * L::EPI_AREA);
            uint32_t* const seq_ctr = a.counters + (int64_t)b * kCountersPerSeq;
            // Arrival at a counter (the protocol of arrive_last): true in the
            // workgroup that completes `expect` arrivals.
            auto arrive = [&](uint32_t* counter, int expect) __attribute__((always_inline)) -> bool {
                if (threadIdx.x == 0) ctl[0] = arrive_last(counter, (uint32_t)expect) ? 1u : 0u;
                __syncthreads();
                const bool last = ctl[0] != 0;
                __syncthreads();
                return last;
            };
            // Merge M partials (o / l at po, (m, l) at pm; partial `own` from LDS)
            // into the output, or into the group partial at (wo, wm): each thread
            // float4s of it, o = sum_c w_c (o / l)_c / sum_c w_c with
            // w_c = l_c 2^(m_c - m*), MB partials and their (m, l) in
            // flight, m* the running maximum.
            auto merge = [&](const float* po, const float* pm, int M, int own, bool to_out, float* wo,
                             float* wm) __attribute__((always_inline)) {
                const auto ro = buf_rsrc(po, part_o * (uint32_t)M);
                const auto rm = buf_rsrc(pm, part_ml * (uint32_t)M);
                const auto wro = buf_rsrc(wo, to_out ? 0u : part_o);
                const auto wrm = buf_rsrc(wm, to_out ? 0u : part_ml);
                for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
                    const int h = 4 * e4 / D;
                    float mstar = -INFINITY, lsum = 0.0f;
                    float4_t acc = {0, 0, 0, 0};
                    constexpr int MB = SEG ? kMergeBatchSeg : kMergeBatch;
                    for (int c0 = 0; c0 < M; c0 += MB) {
                        float4_t oc[MB];
                        float2v_t ml[MB];
        #pragma unroll
                        for (int cb = 0; cb < MB; ++cb) {
                            const int c = min(c0 + cb, M - 1);
                            if (c != own) {
                                oc[cb] = load4_sc1(ro, (uint32_t)c * part_o + (uint32_t)e4 * 16);
                                ml[cb] = load2_sc1(rm, ((uint32_t)c * (uint32_t)hq + (uint32_t)h) * 8);
                            } else {
                                float m, l;
                                oc[cb] = chunk4(e4, m, l);
                                ml[cb] = float2v_t{m, l};
                            }
                        }
                        // past M: a repeat of partial M - 1 with weight 0
                        float mb = mstar;
        #pragma unroll
                        for (int cb = 0; cb < MB; ++cb) mb = fmaxf(mb, ml[cb][0]);
                        const float r = __builtin_amdgcn_exp2f(mstar - mb);  // 0 on the first batch
                        acc *= r;
                        lsum *= r;
        #pragma unroll
                        for (int cb = 0; cb < MB; ++cb) {
                            const float w = c0 + cb < M ? ml[cb][1] * __builtin_amdgcn_exp2f(ml[cb][0] - mb) : 0.0f;
                            acc += oc[cb] * w;
                            lsum += w;
                        }
                        mstar = mb;
                    }
                    const float4_t res = acc * (1.0f / lsum);
                    if (to_out) {
                        store_out4(e4, res);
                    } else {
                        store4_sc1(res, wro, (uint32_t)e4 * 16);
                        if ((4 * e4) % D == 0) store2_sc1(float2v_t{mstar, lsum}, wrm, (uint32_t)h * 8);
                    }
                }
            };
            const int grp = chunk / MG;
            const int n_groups = (n_chunks + MG - 1) / MG;
            const int members = min(MG, n_chunks - grp * MG);
            if (!arrive(seq_ctr + grp, members)) return;
            const int64_t c0row = row0 + grp * MG;
            merge(a.part_o + c0row * total, a.part_ml + c0row * hq * 2, members, chunk - grp * MG, n_groups == 1,
                  a.grp_o + (row0 + grp) * total, a.grp_ml + (row0 + grp) * hq * 2);
            if (n_groups == 1) return;
            wait_vmcnt<0>();
            __syncthreads();
            if (!arrive(seq_ctr + kSeqCounter, n_groups)) return;
            merge(a.grp_o + row0 * total, a.grp_ml + row0 * hq * 2, n_groups, -1, true, a.grp_o, a.grp_ml);
        }
    };

    if constexpr (!segmented) {
        const int wg = xcd_remap(blockIdx.x, p_nblocks);
        const int b = wg / p_max_chunks, chunk = wg % p_max_chunks;
        run_piece(b, chunk, chunk * p_chunk_tiles, 0, 0, (int64_t)b * p_max_chunks);
    } else {
        const int W = p_max_chunks;
        const int w_self = xcd_remap(blockIdx.x, W);
        int* const list = reinterpret_cast<int*>(smem + L::LIST_OFF);    // [kMaxPieces][6], then the count
        long long* const red = reinterpret_cast<long long*>(smem + 64);  // [kWaves] (the ring is still free)
        auto units_of = [&](int bb) -> long long {
            const long long t = ((long long)p_seq_lens[bb] + kTile - 1) / kTile;
            return t > 0 ? t + kPieceCost : 0;
        };
        // Units of this thread's sequence (batches up to the workgroup's 1024
        // threads) and their inclusive scan over the workgroup: one pass
        // gives both every sequence's place and the total C.  Larger
        // batches take a first pass for C and scan in steps of 1024 below.
        const bool one_pass = a.batch <= 64 * kWaves;
        long long ub0 = 0, x0 = 0, before0 = 0;
        long long C = 0;
        if (one_pass) {
            ub0 = (int)threadIdx.x < a.batch ? units_of(threadIdx.x) : 0;
            x0 = ub0;
            for (int off = 1; off < 64; off <<= 1) {
                const long long y = __shfl_up(x0, off, 64);
                if (lane >= off) x0 += y;
            }
            if (lane == 63) red[wave] = x0;
        } else {
            long long part = 0;
            for (int bb = threadIdx.x; bb < a.batch; bb += 64 * kWaves) part += units_of(bb);
            for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
            if (lane == 0) red[wave] = part;
        }
        if (threadIdx.x == 0) list[6 * kMaxPieces] = 0;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const long long v = red[w];
            if (w < wave) before0 += v;
            C += v;
        }
        if (!one_pass) __syncthreads();  // red is reused by the scan below
        // At most C ranges, so that none is empty and a sequence's chunks are
        // numbered without gaps.
        const long long Wl = (long long)W < C ? (long long)W : C;
        if (C > (long long)kMaxChunkTiles * Wl) {
            // The lengths outgrew the plan (a balanced plan made for fewer
            // tokens): a range would not fit the page-id window.  Every
            // workgroup sees the same C, so all of them write NaN into the
            // whole output instead of a wrong result.
            const int64_t n_out = (int64_t)a.batch * p_n_q_heads * D;
            for (int64_t i = (int64_t)blockIdx.x * (64 * kWaves) + threadIdx.x; i < n_out;
                 i += (int64_t)gridDim.x * (64 * kWaves)) {
                if (a.out_f32) reinterpret_cast<float*>(a.out)[i] = __builtin_nanf("");
                else reinterpret_cast<half_t*>(a.out)[i] = __builtin_bit_cast(half_t, (uint16_t)0x7E00);
            }
            return;
        }
        if (w_self >= Wl) return;  // no range (uniform over the workgroup)
        const long long lo = w_self * C / Wl, hi = (w_self + 1) * C / Wl;
        auto range_of = [&](long long u) -> long long { return ((u + 1) * Wl - 1) / C; };
        auto add_piece = [&](int bb, long long ts, long long te) {
            const long long f = range_of(ts), l = range_of(te - 1);
            const int k = atomicAdd(&list[6 * kMaxPieces], 1);
            if (k < kMaxPieces) {
                list[6 * k + 0] = bb;
                list[6 * k + 1] = (int)((lo > ts ? lo : ts) - ts);
                list[6 * k + 2] = (int)((hi < te ? hi : te) - ts);
                list[6 * k + 3] = (int)(w_self - f);
                list[6 * k + 4] = (int)(l - f + 1);
                list[6 * k + 5] = (int)f;
            }
        };
        if (one_pass) {
            const long long ts = before0 + x0 - ub0 + kPieceCost, te = before0 + x0;  // the tiles' units
            if (ub0 > 0 && ts < hi && te > lo) add_piece((int)threadIdx.x, ts, te);
            __syncthreads();
        }
        long long carry = 0;
        for (int b0 = 0; !one_pass && b0 < a.batch; b0 += 64 * kWaves) {
            const int bb = b0 + (int)threadIdx.x;
            const long long ub = bb < a.batch ? units_of(bb) : 0;
            long long x = ub;  // inclusive scan over the wave
            for (int off = 1; off < 64; off <<= 1) {
                const long long y = __shfl_up(x, off, 64);
                if (lane >= off) x += y;
            }
            if (lane == 63) red[wave] = x;
            __syncthreads();
            long long before = 0, sum = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const long long v = red[w];
                if (w < wave) before += v;
                sum += v;
            }
            const long long ts = carry + before + x - ub + kPieceCost, te = carry + before + x;  // the tiles' units
            if (ub > 0 && ts < hi && te > lo) add_piece(bb, ts, te);
            carry += sum;
            __syncthreads();
        }
        const int n_pieces = min(__builtin_amdgcn_readfirstlane(list[6 * kMaxPieces]), kMaxPieces);
        for (int i = 0; i < n_pieces; ++i) {
            const int pb = __builtin_amdgcn_readfirstlane(list[6 * i + 0]);
            const int pt0 = __builtin_amdgcn_readfirstlane(list[6 * i + 1]);
            const int pt1 = __builtin_amdgcn_readfirstlane(list[6 * i + 2]);
            const int pc = __builtin_amdgcn_readfirstlane(list[6 * i + 3]);
            const int pn = __builtin_amdgcn_readfirstlane(list[6 * i + 4]);
            const int pf = __builtin_amdgcn_readfirstlane(list[6 * i + 5]);
            __syncthreads();  // every wave is done with the previous piece's LDS
            run_piece(pb, pc, pt0, pt1, pn, (int64_t)pf + pb);
        }
    }
}

}  // namespace st

// ------------------------------------------------------------------ host side

namespace {

template <int HKV, int GQ>
int stream_lds_bytes() {
    using L = st::Geo<HKV, GQ>;
    const int epi = 2 * HKV * L::EPI_AREA + 16;
    return L::LDS_MAIN > epi ? L::LDS_MAIN : epi;
}

template <int HKV, int GQ, bool SEG>
int launch_stream(dim3 grid, hipStream_t s, const st::Args& a) {
    const int lds = stream_lds_bytes<HKV, GQ>();
    if (lds > kMaxLdsBytes) return kInvalidArgument;
    static std::atomic<uint64_t> lds_raised{0};
    if (allow_full_lds(reinterpret_cast<const void*>(&st::int4_decode_stream_kernel<HKV, GQ, SEG>), lds_raised) != kOk)
        return kLaunchError;
    hipLaunchKernelGGL((st::int4_decode_stream_kernel<HKV, GQ, SEG>), grid, dim3(64 * st::kWaves), lds, s, a.seq_lens, a.block_table, a.q,
                       a.max_chunks, a.chunk_tiles, a.bt_cols, a.max_pages, a.page_shift, a.n_q_heads, (int)grid.x, a);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}

}  // namespace

int stream_max_chunks() { return st::kMaxChunks; }

bool stream_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim) {
    return head_dim == 128 && num_kv_heads == 8 && (num_q_heads == 4 * num_kv_heads || num_q_heads == 8 * num_kv_heads);
}

bool stream_balanced_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim) {
    return head_dim == 128 && num_kv_heads == 8 && num_q_heads == 4 * num_kv_heads;
}

// Chunk mode merges in one level at 4 query heads per kv head, in groups of
// kMergeGroup8 at 8.
static bool chunk_two_level(int64_t num_q_heads, int64_t num_kv_heads, int64_t max_chunks) {
    return num_q_heads == 8 * num_kv_heads && max_chunks > st::kMergeGroup8;
}

// Split-KV workspace: [counters][chunk partials o][chunk (m, l)] and, when a
// sequence can have more than kMergeGroup chunks, [group partials o][group
// (m, l)], `slots` of each (B x max_chunks in chunk mode, W + B in the
// balanced mode).
struct StreamWorkspace {
    int64_t part_o, part_ml, grp_o, grp_ml, total;
};
static StreamWorkspace stream_workspace(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t slots,
                                        bool two_level) {
    auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
    StreamWorkspace w;
    w.part_o = counter_region_bytes(batch);
    w.part_ml = w.part_o + up(slots * num_q_heads * head_dim * 4);
    w.grp_o = w.part_ml + up(slots * num_q_heads * 2 * 4);
    const int64_t g = two_level ? slots : 0;
    w.grp_ml = w.grp_o + up(g * num_q_heads * head_dim * 4);
    w.total = w.grp_ml + g * num_q_heads * 2 * 4;
    return w;
}

int stream_balanced_plan(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t total_tokens,
                         int32_t* out_chunk_tiles, int32_t* out_max_chunks, int64_t* out_workspace_bytes) {
    // Units: every sequence's tiles plus kPieceCost (at most units_ub of
    // them for these lengths); one range a CU (256), each within the page-id
    // window and at least one piece's start cost plus a tile long.
    const int64_t units_ub = (total_tokens + st::kTile - 1) / st::kTile + batch * (1 + st::kPieceCost);
    int64_t per_wg = (units_ub + 255) / 256;
    if (per_wg < st::kPieceCost + 1) per_wg = st::kPieceCost + 1;
    if (per_wg > st::kMaxChunkTiles) per_wg = st::kMaxChunkTiles;
    const int64_t wgs = (units_ub + per_wg - 1) / per_wg;
    if (wgs > st::kMergeGroup * st::kMaxGroups) return kInvalidArgument;
    const int64_t share = (units_ub + wgs - 1) / wgs;
    *out_chunk_tiles = -(int32_t)share;  // negative: the balanced mode
    *out_max_chunks = (int32_t)wgs;
    *out_workspace_bytes =
        wgs > 1 ? stream_workspace(batch, num_q_heads, head_dim, wgs + batch, wgs > st::kMergeGroup).total : 0;
    return kOk;
}

int64_t stream_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                               int64_t max_chunks) {
    return stream_workspace(batch, num_q_heads, head_dim, batch * max_chunks,
                            chunk_two_level(num_q_heads, num_kv_heads, max_chunks))
        .total;
}

int stream_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale, const void* v_scale,
                  const int32_t* block_table, const int32_t* seq_lens, void* output, int32_t output_is_f32,
                  void* workspace, int64_t workspace_bytes_avail, int64_t batch, int64_t num_q_heads,
                  int64_t num_kv_heads, int64_t head_dim, int64_t max_pages, int64_t bt_cols, int32_t page_shift,
                  float softmax_scale, int32_t chunk_tiles, int32_t max_chunks, void* stream) {
    if (!stream_supported(num_q_heads, num_kv_heads, head_dim)) return kInvalidArgument;
    const bool gq8 = num_q_heads == 8 * num_kv_heads;
    // chunk_tiles > 0: chunk mode, batch x max_chunks workgroups; < 0: the
    // balanced mode, max_chunks ranges of at most -chunk_tiles units, a
    // workgroup each (stream_balanced_plan).
    const bool balanced = chunk_tiles < 0;
    const int64_t share = balanced ? -(int64_t)chunk_tiles : chunk_tiles;
    if (share <= 0 || share > st::kMaxChunkTiles || max_chunks <= 0) return kInvalidArgument;
    if (balanced && gq8) return kInvalidArgument;  // (balanced mode: 4 query heads per kv head)
    if (balanced ? max_chunks > st::kMergeGroup * st::kMaxGroups : max_chunks > st::kMaxChunks) return kInvalidArgument;
    if (!balanced && share * max_chunks * 2 < max_pages) return kInvalidArgument;  // the grid covers every page
    const int64_t nblocks = balanced ? max_chunks : batch * (int64_t)max_chunks;
    if (nblocks > 0x7FFFFFFF) return kInvalidArgument;
    st::Args a;
    a.q = (const half_t*)query;
    a.k_data = (const uint8_t*)k_data;
    a.v_data = (const uint8_t*)v_data;
    a.k_scale = (const uint8_t*)k_scale;
    a.v_scale = (const uint8_t*)v_scale;
    a.block_table = block_table;
    a.seq_lens = seq_lens;
    a.out = output;
    a.out_f32 = output_is_f32;
    a.batch = (int)batch;
    a.n_q_heads = (int)num_q_heads;
    a.max_pages = (int)max_pages;
    a.bt_cols = (int)bt_cols;
    a.page_shift = page_shift;
    a.max_chunks = max_chunks;
    a.chunk_tiles = chunk_tiles;
    a.log2_scale = softmax_scale * 1.4426950408889634f;
    a.counters = nullptr;
    a.part_o = a.part_ml = a.grp_o = a.grp_ml = nullptr;
    if (max_chunks > 1) {  // (one balanced range: every piece is a whole sequence)
        const StreamWorkspace w = balanced ? stream_workspace(batch, num_q_heads, head_dim, max_chunks + batch,
                                                              max_chunks > st::kMergeGroup)
                                           : stream_workspace(batch, num_q_heads, head_dim, batch * max_chunks,
                                                              chunk_two_level(num_q_heads, num_kv_heads, max_chunks));
        if (workspace == nullptr || workspace_bytes_avail < w.total) return kWorkspaceTooSmall;
        uint8_t* const ws = (uint8_t*)workspace;
        a.counters = (uint32_t*)ws;
        a.part_o = (float*)(ws + w.part_o);
        a.part_ml = (float*)(ws + w.part_ml);
        a.grp_o = (float*)(ws + w.grp_o);
        a.grp_ml = (float*)(ws + w.grp_ml);
    }
    if (balanced) return launch_stream<8, 4, true>(dim3((unsigned)nblocks), (hipStream_t)stream, a);
    if (gq8) return launch_stream<8, 8, false>(dim3((unsigned)nblocks), (hipStream_t)stream, a);
    return launch_stream<8, 4, false>(dim3((unsigned)nblocks), (hipStream_t)stream, a);
}

}  // namespace iris
