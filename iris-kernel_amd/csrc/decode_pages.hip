// INT4 paged decode attention for gfx950 (MI355X), page-streaming kernel.
//
// Replaces the TileLang kernel `_int4_paged_decode_attention`
// (src/iris_kernel/fused_attention.py:11-220 in Hunter2030ZeRo/Iris-Kernel)
// for the shapes where a page's rows of all kv heads form one contiguous
// slab (Hkv a power of two <= 16); it computes the result of
// `torch_eager_int4_paged_decode_attention`
// (src/iris_kernel/torch_eager_attention.py:154-239).
//
// Why whole pages
// ---------------
// HBM delivers ~6.6 TB/s to loads that stream whole 8 KB pages and only
// ~2.6 TB/s when each kv head's 64-byte row pieces are read by a different
// CU.  So a workgroup covers every kv head of a sequence chunk: its waves
// read each page together, one wave per kv head and tile.
//
// Work decomposition
// ------------------
// * Tile = 32 tokens = two 16-token pages.  Workgroup = (sequence, chunk of
//   tiles) with Hkv x TS waves: wave (slot ts, head j) computes head j of
//   tile ts of each stage (TS consecutive tiles).
// * K goes straight into registers: the K operand of the QK MFMA is a
//   contiguous quarter of a token's head row (16 bytes at D = 128), one
//   buffer load per page.  V and the scales go to LDS with direct-to-LDS
//   loads (buffer_load ... lds): the PV MFMA needs V transposed
//   (ds_read_b64_tr_b8) and the scales are read 2 bytes at a time.
// * Three-stage pipeline: stage s + 2 streams in while stage s is computed
//   (two stages of loads in flight, ~80 KB per CU at Hkv = 8, D = 128,
//   plus their K).  One workgroup barrier per stage.  Every wave issues the
//   same number of loads per stage (loads past the chunk use a descriptor of
//   size 0: no memory access), so each stage's wait is one compile-time
//   vmcnt.
// * Sequences longer than one chunk are split (flash decoding; the reference
//   has no split): each chunk publishes (m, l, o / l) per query head; the
//   last of every group of 8 chunks merges the group, and with more than one
//   group the last group merges the groups (two levels, so no workgroup
//   reads more than 8 or (groups) partials).
// * Chunk mode gives workgroup (b, chunk) a fixed chunk of sequence b; the
//   balanced mode, for ragged batches, gives every workgroup an equal range
//   of all sequences' tiles laid end to end (see the segment search at the
//   end of the kernel).
//
// LDS layout of one page (per tile slot and page r of the tile)
// -------------------------------------------------------------
// * V: the page's 16 token rows of C = Hkv * D / 32 16-byte chunks; chunk c
//   of token t (t = 16 r + row) sits at position c ^ swz(t), which keeps the
//   transposed reads free of bank conflicts.  Padded to whole 1 KB loads
//   (padding reads past the page return 0).
// * K and V scales: the page's [16 tokens][Hkv][G] halves each, rows
//   permuted so that a read instruction's four row quads hit different banks.
//
// Arithmetic (as in the general kernel, decode.hip)
// --------------------------------------------------
// * Codes enter v_mfma_f32_16x16x32_f16 as exact fp16 subnormals (nibble
//   + 8), the offset removed with one per-group correction term.
// * Scale groups in the MFMA columns: column n = (query head h = n / GS,
//   scale slot gs = n % GS), GS = min(G, 16 / g rounded down to a power of
//   two), in G / GS passes.  A lane of K row-group jq holds a contiguous
//   quarter of its token's head row, inside one scale group gl; its q enters
//   the columns of slot gl % GS and its K only pass gl / GS, so each
//   accumulator column sums exactly one group.  The K scale is applied per
//   lane and the GS columns of a query head are added with DPP.  PV uses the
//   same columns: B = p * v_scale(token, group of the column), masked to the
//   columns of the MFMA's V group.
// * fp32 online softmax in base 2 with lazy rescaling (p <= 4).
#include <type_traits>

#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "decode_pages.h"
#include "decode_stream.h"
#include "iris_hip.h"

namespace iris {
namespace pg {

constexpr int kTile = 32;
constexpr int kPageSize = 16;
constexpr int kMaxChunkTiles = 64;  // a chunk's 2 * 64 page ids fill two VGPRs
constexpr int kMaxWaves = 16;
constexpr int kLdsBudget = 160 * 1024;
constexpr int kStages = 3;
constexpr int kMergeGroup = 8;  // chunks merged by the last of each group
constexpr int kMaxGroups = 64;  // groups merged by the last group
constexpr int kSeqCounter = kCountersPerSeq - 1;  // a sequence's group-level arrival counter
static_assert(kMaxGroups < kSeqCounter, "group counters and the sequence counter share a sequence's region");
constexpr int kSC1 = 16;        // cache-policy bit sc1: device-coherent access
constexpr int kNT = 2;          // cache-policy bit nt: streaming (the cache pages are read once)

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
    // Split-KV slots: chunk c of sequence b, done by logical workgroup
    // w = first(b) + c, owns slot w + b (unique; slots = workgroups + B).
    uint32_t* counters;  // sequence b: group gi's arrivals at b * kCountersPerSeq + gi, the groups' at
                         // b * kCountersPerSeq + kSeqCounter; zero between calls
    float* p1_o;         // [slots][Hq][D]  chunk o / l
    float* p1_ml;        // [slots][Hq][2]  chunk (m, l), base-2 logits
    float* p2_o;         // [slots][Hq][D]  group o / l (group gi of b at slot first(b) + b + gi)
    float* p2_ml;        // [slots][Hq][2]
    int out_f32;
    int batch, n_q_heads, n_kv_heads, group;  // group = Hq / Hkv
    int max_pages;                // 16-token pages a block-table row addresses
    int bt_cols, page_shift;      // block-table columns; the page code of virtual_page (page_size = 16 m)
    int max_chunks, chunk_tiles;  // chunk mode: workgroup (b, chunk), b * max_chunks + chunk
    int segmented;                // balanced mode: workgroup w takes tiles [w T / W, (w + 1) T / W)
    int slots;                    // workgroups + B
    int seg_off;                  // LDS byte offset of the segment list
    float log2_scale;
};

// K operand: eight codes (one dword, low nibble first) -> fp16 subnormals in
// the order d0, d4, 16*d1, 16*d5, d2, d6, 16*d3, 16*d7 (units of 2^-24,
// codes offset by +8).  Each half is one v_bitop3 ((x ^ c) & m); masks
// mlo = 0x000F000F, mhi = 0x00F000F0 keep the codes, zero masks drop the
// lane from the product.
__device__ __forceinline__ half8_t k_operand(uint32_t x, uint32_t mlo, uint32_t mhi) {
    const uint32_t y = x >> 8;
    const u32x4_t r = {(x ^ 0x00080008u) & mlo, (x ^ 0x00800080u) & mhi, (y ^ 0x00080008u) & mlo,
                       (y ^ 0x00800080u) & mhi};
    return __builtin_bit_cast(half8_t, r);
}

// q (8 consecutive dims) in the order of k_operand, high-nibble dims / 16.
__device__ __forceinline__ half8_t q_operand(u32x4_t w) {
    const half2_t w0 = as_half2(w[0]), w1 = as_half2(w[1]), w2 = as_half2(w[2]), w3 = as_half2(w[3]);
    const half_t s16 = (half_t)0.0625f;
    return half8_t{w0.x, w2.x, w0.y * s16, w2.y * s16, w1.x, w3.x, w1.y * s16, w3.y * s16};
}

// V operands from the 8 bytes of one transposed read (byte k' = token k'):
// lo = low nibbles (even dim), hi = 16 * high nibbles (odd dim), both in the
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
constexpr int kVSlotByte[8] = {0, 2, 1, 3, 4, 6, 5, 7};

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// v_permlane32_swap / v_permlane16_swap as opaque instructions (the s_nop
// covers the VALU-write -> permlane-read hazard).
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// max / sum over the four 16-lane rows (lanes n, n+16, n+32, n+48).
__device__ __forceinline__ float row_max4(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    swap32(a, b);
    uint32_t c = __builtin_bit_cast(uint32_t, fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)));
    uint32_t d = c;
    swap16(c, d);
    return fmaxf(__builtin_bit_cast(float, c), __builtin_bit_cast(float, d));
}
__device__ __forceinline__ float row_sum4(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    swap32(a, b);
    uint32_t c = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b));
    uint32_t d = c;
    swap16(c, d);
    return __builtin_bit_cast(float, c) + __builtin_bit_cast(float, d);
}
// Sum over the GS adjacent lanes of a column group (DPP quad permutations).
template <int GS>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (GS >= 2)
        x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
    if constexpr (GS >= 4)
        x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
    return x;
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

// Buffer resource over `bytes` bytes at `base`; offsets past the end read 0
// (and write nothing) without a memory access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// K loads into registers (non-temporal, like every cache-page load) are
// inline assembly too, so that the compiler's
// wait analysis (which cannot follow registers loaded two loop iterations
// earlier and would wait for every load in flight) leaves them alone.  A
// register loaded this way may only be read after a wait that names it as an
// in/out operand (wait_vmcnt_k), which orders the reads after the wait and
// keeps the register from being reused while the load is in flight.
__device__ __forceinline__ u32x4_t rsrc_words(const void* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return u32x4_t{(uint32_t)p, (uint32_t)(p >> 32) & 0xFFFFu, bytes, 0x00020000u};
}
__device__ __forceinline__ void load_k(u32x4_t& out, uint32_t voff, u32x4_t rs) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen nt" : "=&v"(out) : "v"(voff), "s"(rs) : "memory");
}
__device__ __forceinline__ void load_k(u32x2_t& out, uint32_t voff, u32x4_t rs) {
    asm volatile("buffer_load_dwordx2 %0, %1, %2, 0 offen nt" : "=&v"(out) : "v"(voff), "s"(rs) : "memory");
}
template <int N, typename T>
__device__ __forceinline__ void wait_vmcnt_k(T (&k)[2]) {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(k[0]), "+v"(k[1]) : "n"(N) : "memory");
}
template <typename T>
__device__ __forceinline__ void wait_vmcnt0_k(T (&k0)[2], T (&k1)[2], T (&k2)[2]) {
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(k0[0]), "+v"(k0[1]), "+v"(k1[0]), "+v"(k1[1]), "+v"(k2[0]), "+v"(k2[1])
                 :
                 : "memory");
}

// Reads of stage data (written by direct-to-LDS loads) are inline assembly
// that waits for its own results: the compiler cannot relate them to the
// direct loads still in flight into the other stages and would wait for
// those too.  The stage's loads are complete when these run (a vmcnt wait
// and a workgroup barrier precede them).
//
// Eight 16-bit values: slot 4 r + i at addr + O + r * R + i * S.
template <int O, int R, int S>
__device__ __forceinline__ void lds_read8_u16(uint32_t addr, uint32_t (&x)[8]) {
    static_assert(O + R + 3 * S < 65536, "ds offset range");
    asm volatile(
        "ds_read_u16 %0, %8 offset:%9\n\t"
        "ds_read_u16 %1, %8 offset:%10\n\t"
        "ds_read_u16 %2, %8 offset:%11\n\t"
        "ds_read_u16 %3, %8 offset:%12\n\t"
        "ds_read_u16 %4, %8 offset:%13\n\t"
        "ds_read_u16 %5, %8 offset:%14\n\t"
        "ds_read_u16 %6, %8 offset:%15\n\t"
        "ds_read_u16 %7, %8 offset:%16\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7])
        : "v"(addr), "n"(O), "n"(O + S), "n"(O + 2 * S), "n"(O + 3 * S), "n"(O + R), "n"(O + R + S),
          "n"(O + R + 2 * S), "n"(O + R + 3 * S)
        : "memory");
}
// N transposed 8-byte reads (ds_read_b64_tr_b8).
template <int N>
__device__ __forceinline__ void lds_read_tr8(const uint32_t (&addr)[N], int2v_t (&w)[N]) {
    static_assert(N == 2 || N == 4, "two or four reads");
    if constexpr (N == 4) {
        asm volatile(
            "ds_read_b64_tr_b8 %0, %4\n\t"
            "ds_read_b64_tr_b8 %1, %5\n\t"
            "ds_read_b64_tr_b8 %2, %6\n\t"
            "ds_read_b64_tr_b8 %3, %7\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
            : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3])
            : "memory");
    } else {
        asm volatile(
            "ds_read_b64_tr_b8 %0, %2\n\t"
            "ds_read_b64_tr_b8 %1, %3\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w[0]), "=&v"(w[1])
            : "v"(addr[0]), "v"(addr[1])
            : "memory");
    }
}

// Position swizzle of a token's 16-byte V chunks (C chunks per row): the
// 16 rows of a page take 16 different positions, and the second page of a
// tile the other half of the positions (C >= 32), so a transposed read over
// tokens of both pages hits every bank once.
__device__ __forceinline__ int swz(int t, int C) { return ((t & 15) ^ (((t >> 4) & 1) * (C / 2))) & (C - 1); }

// Page geometry of a (Hkv, head_dim) cache, for the device template and the
// host.  All loads move 16 bytes per lane; a page's V slab (16 token rows of
// C 16-byte chunks) takes v_loads loads, each scale slab s_loads (loads of
// less than 64 lanes run with the lanes past the slab switched off).
struct PageGeom {
    int C, v_bytes, s_bytes, v_loads, s_loads, jpp, pb, ts, nw, jobs, jmax, stage;
};
constexpr PageGeom page_geom(int hkv, int d) {
    PageGeom g{};
    g.C = hkv * d / 32;
    g.v_bytes = 16 * hkv * d / 2;
    g.s_bytes = 16 * hkv * (d / 32) * 2;
    g.v_loads = (g.v_bytes + 1023) / 1024;
    g.s_loads = (g.s_bytes + 1023) / 1024;
    g.jpp = g.v_loads + 2 * g.s_loads;
    g.pb = g.v_bytes + 2 * g.s_bytes;  // LDS bytes per page: [V][K scales][V scales]
    int ts = kMaxWaves / hkv;
    while (ts > 1 && kStages * ts * 2 * g.pb > kLdsBudget) --ts;
    g.ts = ts;
    g.nw = ts * hkv;
    g.jobs = ts * 2 * g.jpp;  // LDS loads per stage
    g.jmax = (g.jobs + g.nw - 1) / g.nw;
    g.stage = ts * 2 * g.pb;
    return g;
}

// Device-coherent (sc1) 16- and 8-byte accesses of the split-KV partials:
// they bypass the non-coherent caches, so workgroups on other XCDs see them.
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

template <int D, int GS, int HKV>
__global__ __launch_bounds__(64 * kMaxWaves) void int4_decode_pages_kernel(Args a) {
    constexpr int G = D / 32;   // scale groups per head
    constexpr int NP = G / GS;  // passes (groups per column slot)
    static_assert(GS >= 1 && GS <= G && G % GS == 0, "scale slots must divide the groups");
    constexpr PageGeom L = page_geom(HKV, D);
    constexpr int C = L.C, TS = L.ts, NW = L.nw, PB = L.pb, VR = L.v_bytes, SR = L.s_bytes;
    constexpr int J = L.jmax;
    constexpr int ST = HKV * G * 2;  // scale bytes of one token (all heads)
    // Scale rows in LDS: token t at slot (t % 4) * 4 + t / 4 when a row is
    // whole 16-byte chunks, so the four tokens 4 jq + i a read instruction
    // fetches for jq = 0..3 sit in different banks; else in token order.
    constexpr bool kScalePerm = ST % 16 == 0;
    constexpr int SS = kScalePerm ? 4 * ST : ST;  // bytes between tokens 4 jq + i and 4 jq + i + 1
    using kvec_t = typename std::conditional<D == 128, u32x4_t, u32x2_t>::type;  // a lane's K of one page
    constexpr int BD = 64 * NW;  // threads per workgroup
    extern __shared__ __align__(16) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15;   // MFMA column (B/C) or row (A)
    const int jq = lane >> 4;  // MFMA k-chunk (A/B) or row quad (C)
    constexpr int hkv = HKV;
    const int hh = wave % HKV, slot = wave / HKV;

    const int wg = xcd_remap(blockIdx.x, gridDim.x);
    const int g = a.group;

    // ---- one segment: tiles [t_begin, t_end) of sequence b, chunk c of its
    // n_chunks, the first of which logical workgroup `first` does.  A
    // negative t_end / n_chunks (chunk mode) follows from the length.
    auto segment = [&](const int b, const int t_begin, const int t_end_in, const int c_in, const int nch_in,
                       const int first) __attribute__((always_inline)) {
    const int p0 = 2 * t_begin;

    const int32_t* bt = a.block_table + (int64_t)b * a.bt_cols;
    int pid0 = 0, pid1 = 0;
    if (p0 + lane < a.max_pages) pid0 = virtual_page(bt, p0 + lane, a.page_shift);
    if (p0 + 64 + lane < a.max_pages) pid1 = virtual_page(bt, p0 + 64 + lane, a.page_shift);

    // Column n = (query head h, scale slot gs); this lane's K quarter row
    // lies in group gl = jq * G / 4.  Pass p puts group p * GS + gs in the
    // columns of slot gs: the lane's q enters the columns of slot gl % GS,
    // its K only the pass gl / GS.
    const int h = n / GS, gs = n % GS;
    const bool col_valid = h < g;
    const half_t* qrow = a.q + ((int64_t)b * a.n_q_heads + hh * g + (col_valid ? h : 0)) * D;
    const int gl = jq * G / 4;
    half8_t qb[G];
#pragma unroll
    for (int m = 0; m < G; ++m) {
        u32x4_t raw = {0, 0, 0, 0};
        if (col_valid && gl % GS == gs) raw = *reinterpret_cast<const u32x4_t*>(qrow + jq * (D / 4) + 8 * m);
        qb[m] = q_operand(raw);
    }
    uint32_t kmlo[NP], kmhi[NP];
    float qinit[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        kmlo[p] = gl / GS == p ? 0x000F000Fu : 0u;
        kmhi[p] = gl / GS == p ? 0x00F000F0u : 0u;
        // -8 * 2^-24 * (sum of the column group's q as the B operand holds
        // it): removes the +8 code offset.
        float part = 0.0f;
        if (col_valid) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const half8_t qf = q_operand(*reinterpret_cast<const u32x4_t*>(qrow + (p * GS + gs) * 32 + 8 * c));
#pragma unroll
                for (int i = 0; i < 8; ++i) part += (float)qf[i] * ((i & 2) ? 16.0f : 1.0f);
            }
        }
        qinit[p] = -8.0f * 5.9604644775390625e-08f * part;
    }

    const int seq_len = a.seq_lens[b];
    const int n_tiles = (seq_len + kTile - 1) / kTile;
    if (t_begin >= n_tiles) return;  // uniform over the workgroup
    const int t_end = t_end_in >= 0 ? min(t_end_in, n_tiles) : min(t_begin + a.chunk_tiles, n_tiles);
    const int n_chunks = nch_in >= 0 ? nch_in : (n_tiles + a.chunk_tiles - 1) / a.chunk_tiles;
    const int chunk = c_in;
    const int n_stages = (t_end - t_begin + TS - 1) / TS;
    const int last_lp = (seq_len + kPageSize - 1) / kPageSize - 1;
    constexpr uint32_t page_data = (uint32_t)L.v_bytes;
    constexpr uint32_t page_scale = (uint32_t)L.s_bytes;

    // Physical page of logical page lp of this chunk (p0 <= lp < p0 + 128;
    // past the sequence, the last page stands in).
    auto page_of = [&](int lp) -> int64_t {
        const int rel = min(lp, last_lp) - p0;
        return (int64_t)__builtin_amdgcn_readlane(rel < 64 ? pid0 : pid1, rel & 63);
    };
    // Wait for the page ids here, on every path: a first use under a branch
    // would leave later uses waiting for every load in flight.
    pid0 = opaque(pid0);
    pid1 = opaque(pid1);

    // ---- LDS: kStages stages of TS tiles x 2 pages; per page
    // [V: VR][K scales: SR][V scales: SR], scales as in memory
    // ([token][kv head][G halves]).
    //
    // This wave's loads into LDS, the same for every stage: job
    // u = j * NW + wave < L.jobs of the stage's TS * 2 pages x jpp, packed as
    // (LDS offset in the stage << 14) | (active lanes << 7) | (page slot << 2)
    // | kind (0 V, 1 K scales, 2 V scales).
    const int my_jobs = (L.jobs - wave + NW - 1) / NW;  // J or J - 1
    int job_code[J];
    uint32_t job_voff[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int u = min(j * NW + wave, L.jobs - 1);
        const int pg_slot = u / L.jpp, jb = u - pg_slot * L.jpp;
        if (jb < L.v_loads) {
            // V rows: load jb covers LDS chunk positions 64 jb + lane; fetch
            // the chunk stored there.
            const int P = 64 * jb + lane;
            const int row = P / C, pos = P % C;
            const int lanes = min(64, L.v_bytes / 16 - 64 * jb);
            job_voff[j] = (uint32_t)(row * C + (pos ^ swz(16 * (pg_slot & 1) + row, C))) * 16;
            job_code[j] = ((pg_slot * PB + jb * 1024) << 14) | (lanes << 7) | (pg_slot << 2);
        } else {
            // Scales: a straight copy.
            const int js = jb - L.v_loads;
            const int is_v = js >= L.s_loads ? 1 : 0;
            const int i = js - is_v * L.s_loads;
            const int lanes = min(64, L.s_bytes / 16 - 64 * i);
            const int P = 64 * i + lane;  // 16-byte LDS chunk of the scale slab
            int chunk16 = P;
            if constexpr (kScalePerm) {
                const int slot = P / (ST / 16), w = P % (ST / 16);
                chunk16 = (4 * (slot % 4) + slot / 4) * (ST / 16) + w;
            }
            job_voff[j] = (uint32_t)(chunk16 * 16);
            job_code[j] = ((pg_slot * PB + VR + is_v * SR + i * 1024) << 14) | (lanes << 7) | (pg_slot << 2) | (1 + is_v);
        }
    }
    // This lane's K of a page: token row n, head hh, quarter jq.
    const uint32_t k_voff = (uint32_t)((n * hkv + hh) * (D / 2) + jq * (D / 8));

    // Stage `stage` into LDS stage buffer `buf`, and this wave's K of it into
    // kb: my_jobs + 2 loads per wave, past the chunk included.
    auto issue = [&](int stage, int buf, kvec_t (&kb)[2]) __attribute__((always_inline)) {
        uint8_t* const st = smem + buf * L.stage;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            if (j < my_jobs) {
                const int code = job_code[j];
                const uint32_t voff = job_voff[j];  // (an array element here drops the host launch stub)
                const int kind = code & 3, ts = (code >> 3) & 15, r = (code >> 2) & 1, lanes = (code >> 7) & 127;
                const int tile = t_begin + stage * TS + ts;
                const bool valid = tile < t_end;
                const int64_t pid = valid ? page_of(2 * tile + r) : 0;
                IRIS_LDS void* const dst = (IRIS_LDS void*)(st + (code >> 14));
                const uint8_t* const src = kind == 0 ? a.v_data + pid * page_data
                                                     : (kind == 1 ? a.k_scale : a.v_scale) + pid * page_scale;
                const auto rs = page_rsrc(src, valid ? (kind == 0 ? page_data : page_scale) : 0u);
                // Lanes past a slab that is not a whole number of loads are
                // switched off (an exec mask here costs throughput, so only
                // layouts with such slabs use it).
                constexpr bool kPartial = L.v_bytes % 1024 != 0 || L.s_bytes % 1024 != 0;
                if (!kPartial || lane < lanes)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, voff, 0, 0, kNT);
            }
        }
        const int tile = t_begin + stage * TS + slot;
        const bool valid = tile < t_end;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int64_t pid = valid ? page_of(2 * tile + r) : 0;
            load_k(kb[r], k_voff, rsrc_words(a.k_data + pid * page_data, valid ? page_data : 0u));
        }
    };

    // ---- per-lane LDS read offsets within a tile slot's two pages.
    // Transposed V reads: supplier row s = n reads token tau(jq, n >> 1),
    // half n & 1, of group grp.
    const int trk = n >> 1;
    const int tr_tok = 4 * jq + (trk & 3) + 16 * (trk >> 2);
    uint32_t tr_off[G];
#pragma unroll
    for (int grp = 0; grp < G; ++grp)
        tr_off[grp] = (uint32_t)((tr_tok >> 4) * PB + ((tr_tok & 15) * C + ((hh * G + grp) ^ swz(tr_tok, C))) * 16 +
                                 8 * (n & 1));
    // Scales of this lane's tokens 4 jq + i of page r, head hh, slot gs.
    const uint32_t sc_off = (uint32_t)(VR + (kScalePerm ? jq * ST : 4 * jq * ST) + hh * G * 2 + gs * 2);

    const float c24 = a.log2_scale * 16777216.0f;  // MFMA units -> base-2 logits
    const float lazy = 2.0f / c24;
    float m_run = -INFINITY;
    float l_part = 0.0f;
    float s_lo = INFINITY;  // lowest valid score seen
    float ps[NP];
    float4_t o[NP][2];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        ps[p] = 0.0f;
        o[p][0] = o[p][1] = float4_t{0, 0, 0, 0};
    }

    // ---- compute this wave's tile of a stage (its head, its slot).
    auto compute = [&](int stage, int buf, const kvec_t (&kb)[2]) __attribute__((always_inline)) {
        const int tile = t_begin + stage * TS + slot;
        if (tile >= t_end) return;  // uniform over the wave
        const uint32_t base = lds_addr(smem + buf * L.stage + slot * 2 * PB);
        const int tok0 = tile * kTile;
        const bool full = tok0 + kTile <= seq_len;
        const uint32_t sb = base + opaque(sc_off);
        // ---- QK: s[r][i] is token 16 r + 4 jq + i, column n (MFMA units)
        float s[2][4];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) s[r][i] = 0.0f;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            uint32_t ksr[8];  // K scales of the pass: slot 4 r + i = token 16 r + 4 jq + i
            lds_read8_u16<0, PB, SS>(sb + (uint32_t)(p * GS * 2), ksr);
            const uint32_t mlo = NP == 1 ? 0x000F000Fu : kmlo[p], mhi = NP == 1 ? 0x00F000F0u : kmhi[p];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                float4_t acc = {qinit[p], qinit[p], qinit[p], qinit[p]};
#pragma unroll
                for (int m = 0; m < G; ++m) acc = mfma16x16x32(k_operand(kb[r][m], mlo, mhi), qb[m], acc);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const half_t ks = __builtin_bit_cast(half_t, (uint16_t)ksr[4 * r + i]);
                    s[r][i] = __builtin_fmaf((float)ks, acc[i], s[r][i]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) s[r][i] = group_sum<GS>(s[r][i]);
        // ---- online softmax (base 2, lazy rescale)
        // lowest score of the valid tokens (-inf: a non-finite K scale or
        // query); v_minimum3 needs no canonicalised operands
        auto vmin = [](float x, float y) { return __builtin_elementwise_minimum(x, y); };
        if (full) {
            s_lo = vmin(vmin(s_lo, vmin(vmin(s[0][0], s[0][1]), vmin(s[0][2], s[0][3]))),
                        vmin(vmin(s[1][0], s[1][1]), vmin(s[1][2], s[1][3])));
        } else {
            const int sl = opaque_int(seq_len);  // (the compares stay in this branch)
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (tok0 + 16 * r + 4 * jq + i >= sl) s[r][i] = -INFINITY;
                    else s_lo = vmin(s_lo, s[r][i]);
                }
        }
        float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                         fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
        mx = row_max4(mx);  // finite: token tok0 < seq_len
        if (__ballot(mx > m_run + lazy) != 0) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c24);
            m_run = m_new;
            l_part *= alpha;
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                ps[p] *= alpha;
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[p][e][i] *= alpha;
            }
        }
        const float moff = -m_run * c24;
        float pr[2][4];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pr[r][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r][i], c24, moff));
                l_part += pr[r][i];
            }
        // ---- PV: V scales and the transposed V codes
        uint32_t tra[G];
#pragma unroll
        for (int grp = 0; grp < G; ++grp) tra[grp] = base + opaque(tr_off[grp]);
        int2v_t vw[G];
        lds_read_tr8<G>(tra, vw);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            uint32_t vsr[8];
            lds_read8_u16<SR, PB, SS>(sb + (uint32_t)(p * GS * 2), vsr);
            float vsv[2][4];
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) vsv[r][i] = (float)__builtin_bit_cast(half_t, (uint16_t)vsr[4 * r + i]);
            if (!full) {
                // Tokens past seq_len may hold any bytes: never let their
                // scale reach the product (0 * NaN).
#pragma unroll
                for (int r = 0; r < 2; ++r)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (tok0 + 16 * r + 4 * jq + i >= seq_len) vsv[r][i] = 0.0f;
            }
            half8_t bp;
#pragma unroll
            for (int sl = 0; sl < 8; ++sl) {
                const int r = kVSlotByte[sl] >> 2, i = kVSlotByte[sl] & 3;
                bp[sl] = (half_t)(pr[r][i] * vsv[r][i]);
            }
            const half2_t one2 = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
            for (int qq = 0; qq < 4; ++qq)
                ps[p] = __builtin_amdgcn_fdot2(half2_t{bp[2 * qq], bp[2 * qq + 1]}, one2, ps[p], false);
#pragma unroll
            for (int gg = 0; gg < GS; ++gg) {
                const half8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
                const half8_t bm = gs == gg ? bp : z;
                half8_t a0, a1;
                v_operands(vw[p * GS + gg], a0, a1);
                o[p][0] = mfma16x16x32(a0, bm, o[p][0]);
                o[p][1] = mfma16x16x32(a1, bm, o[p][1]);
            }
        }
    };

    // ---- the pipeline.  Step s: wait for this wave's loads of stage s (the
    // loads of stage s + 1 may stay in flight: my_jobs + 2 of them, at least
    // WAITN); the barrier makes every wave's stage-s loads visible and frees
    // the buffer of stage s - 1, which then receives stage s + 2; compute
    // stage s.  No branch separates a K load from its wait (a branch join
    // could copy a register whose load is still in flight): every iteration
    // runs its three steps, compute skips stages past the chunk.
    constexpr int WAITN = L.jobs % NW == 0 ? J + 2 : J + 1;
    kvec_t kb0[2], kb1[2], kb2[2];
    issue(0, 0, kb0);
    issue(1, 1, kb1);
    auto step = [&](int stage, int cur, kvec_t (&kc)[2], int nxt, kvec_t (&kn)[2]) __attribute__((always_inline)) {
        wait_vmcnt_k<WAITN>(kc);
        __builtin_amdgcn_s_barrier();
        issue(stage + 2, nxt, kn);
        compute(stage, cur, kc);
    };
    for (int sidx = 0; sidx < n_stages; sidx += kStages) {
        step(sidx, 0, kb0, 2, kb2);
        step(sidx + 1, 1, kb1, 0, kb0);
        step(sidx + 2, 2, kb2, 1, kb1);
    }
    // The loads past the chunk still write LDS and the K registers.
    wait_vmcnt0_k(kb0, kb1, kb2);
    __syncthreads();

    // ---- final per-lane values: undo the code offset and the 2^-24 units
    m_run *= c24;
    l_part = row_sum4(poison_if_neg_inf(s_lo, l_part));
#pragma unroll
    for (int p = 0; p < NP; ++p) ps[p] = 8.0f * row_sum4(ps[p]);

    // ---- this wave's (m, l, o) per query head (at most 16): [0, 16) m,
    // [16, 32) l, [32 + qh D, ...) o (unnormalised) in its area of LDS.
    const int area = (32 + (16 / GS) * D) * 4;
    float* const ep = reinterpret_cast<float*>(smem + wave * area);
    if (col_valid) {
        if (jq == 0 && gs == 0) {
            ep[h] = m_run;
            ep[16 + h] = l_part;
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int grp = p * GS + gs;
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ep[32 + h * D + grp * 32 + 2 * (4 * jq + i) + e] =
                        o[p][e][i] * (e ? 1048576.0f : 16777216.0f) - ps[p];
        }
    }
    __syncthreads();

    // ---- this chunk's result, 4 elements at a time: element idx = (kv head
    // j, query head qh, dim d) of this sequence's Hq x D output, merged over
    // the TS tile slots of head j.
    const int hq = a.n_q_heads;
    const int total = hq * D, n4 = total / 4;
    const int gD = g * D;
    auto chunk4 = [&](int e4, float& mstar, float& lsum) -> float4_t {
        const int idx = 4 * e4;
        const int j = idx / gD, rem = idx - j * gD, qh = rem / D, d = rem - qh * D;
        mstar = -INFINITY;
        for (int s = 0; s < TS; ++s)
            mstar = fmaxf(mstar, reinterpret_cast<const float*>(smem + (s * hkv + j) * area)[qh]);
        lsum = 0.0f;
        float4_t acc = {0, 0, 0, 0};
        for (int s = 0; s < TS; ++s) {
            const float* w = reinterpret_cast<const float*>(smem + (s * hkv + j) * area);
            const float f = __builtin_amdgcn_exp2f(w[qh] - mstar);  // 0 for idle slots
            lsum += w[16 + qh] * f;
            acc += *reinterpret_cast<const float4_t*>(w + 32 + qh * D + d) * f;
        }
        return acc * (1.0f / lsum);
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
            float mstar, lsum;
            store_out4(e4, chunk4(e4, mstar, lsum));
        }
        return;
    }

    // ---- split-KV.  Partials are written and read with device-coherent
    // (sc1) accesses; a writer waits for its stores before its arrival.
    const uint32_t part_o = (uint32_t)total * 4, part_ml = (uint32_t)hq * 8;  // bytes per partial
    {
        const int64_t row = (int64_t)first + b + chunk;
        const auto ro = page_rsrc(a.p1_o + row * total, part_o);
        const auto rm = page_rsrc(a.p1_ml + row * hq * 2, part_ml);
        for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
            float mstar, lsum;
            const float4_t v = chunk4(e4, mstar, lsum);
            store4_sc1(v, ro, (uint32_t)e4 * 16);
            if ((4 * e4) % D == 0) store2_sc1(float2v_t{mstar, lsum}, rm, (uint32_t)(4 * e4 / D) * 8);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();

    // Merge M partials (o at ro, (m, l) at rm; partial c at c * part_*) with
    // every load of a batch in flight, into the output (to_out) or into the
    // group partial at wo / wm (merged o / l and each query head's (m, l)).
    float* const wts = reinterpret_cast<float*>(smem);  // [M][hq] merge weights
    float* const hdr = wts + kMaxGroups * hq;          // [hq] (m*, l*)
    uint32_t* const ctl = reinterpret_cast<uint32_t*>(hdr + 2 * hq);
    constexpr int CB = 8;
    auto merge = [&](const __amdgpu_buffer_rsrc_t& ro, const __amdgpu_buffer_rsrc_t& rm, int M, bool to_out,
                     const __amdgpu_buffer_rsrc_t& wo, const __amdgpu_buffer_rsrc_t& wm) {
        // The first batch of this thread's partials is loaded before the
        // (m, l) round trip.
        // (Threads past the output and partials past M load nothing.)
        const int e_first = (int)threadIdx.x;
        float4_t first[CB];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            first[cb] = float4_t{0, 0, 0, 0};
            if (e_first < n4 && cb < M) first[cb] = load4_sc1(ro, (uint32_t)cb * part_o + (uint32_t)e_first * 16);
        }
        // Weights w_c = l_c 2^(m_c - m*) / L: a thread per (query head,
        // partial c), the MP >= M partials of a head in adjacent lanes, max
        // and sum by lane shuffles.
        const int MP = M <= 1 ? 1 : 1 << (32 - __builtin_clz(M - 1));  // <= 64
        for (int t0 = 0; t0 < hq * MP; t0 += blockDim.x) {  // the same trip count in every lane
            const int t = t0 + (int)threadIdx.x;
            const int qh = t / MP, c = t % MP;
            const bool ok = qh < hq && c < M;
            const float2v_t ml = ok ? load2_sc1(rm, (uint32_t)(c * hq + qh) * 8) : float2v_t{-INFINITY, 0.0f};
            float mstar = ml[0];
            for (int off = MP / 2; off > 0; off >>= 1) mstar = fmaxf(mstar, __shfl_xor(mstar, off, 64));
            const float w = ok ? ml[1] * __builtin_amdgcn_exp2f(ml[0] - mstar) : 0.0f;
            float lsum = w;
            for (int off = MP / 2; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off, 64);
            if (ok) wts[c * hq + qh] = w / lsum;
            if (ok && c == 0) {
                hdr[2 * qh] = mstar;
                hdr[2 * qh + 1] = lsum;
            }
        }
        __syncthreads();
        for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
            const int qh = 4 * e4 / D;
            float4_t acc = {0, 0, 0, 0};
            for (int c0 = 0; c0 < M; c0 += CB) {
                float4_t oc[CB];
                const bool pre = e4 == (int)threadIdx.x && c0 == 0;
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const int c = min(c0 + cb, M - 1);
                    oc[cb] = pre ? first[cb] : load4_sc1(ro, (uint32_t)c * part_o + (uint32_t)e4 * 16);
                }
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
                    if (c0 + cb < M) acc += oc[cb] * wts[(c0 + cb) * hq + qh];
            }
            if (to_out) {
                store_out4(e4, acc);
            } else {
                store4_sc1(acc, wo, (uint32_t)e4 * 16);
                if ((4 * e4) % D == 0) store2_sc1(float2v_t{hdr[2 * qh], hdr[2 * qh + 1]}, wm, (uint32_t)qh * 8);
            }
        }
    };
    // Arrival at a counter: true in the workgroup that completes `expect`
    // arrivals (which then resets the counter).
    auto arrive = [&](uint32_t* counter, int expect) -> bool {
        if (threadIdx.x == 0) ctl[0] = arrive_last(counter, (uint32_t)expect) ? 1u : 0u;
        __syncthreads();
        const bool last = ctl[0] != 0;
        __syncthreads();
        return last;
    };

    const int grp = chunk / kMergeGroup;
    const int n_groups = (n_chunks + kMergeGroup - 1) / kMergeGroup;
    const int members = min(kMergeGroup, n_chunks - grp * kMergeGroup);
    if (!arrive(a.counters + (int64_t)b * kCountersPerSeq + grp, members)) return;
    {
        const int64_t row = (int64_t)first + b + grp * kMergeGroup;
        const auto ro = page_rsrc(a.p1_o + row * total, part_o * members);
        const auto rm = page_rsrc(a.p1_ml + row * hq * 2, part_ml * members);
        const int64_t row2 = (int64_t)first + b + grp;
        const auto wo = page_rsrc(a.p2_o + row2 * total, n_groups > 1 ? part_o : 0u);
        const auto wm = page_rsrc(a.p2_ml + row2 * hq * 2, n_groups > 1 ? part_ml : 0u);
        merge(ro, rm, members, n_groups == 1, wo, wm);
        if (n_groups == 1) return;
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (!arrive(a.counters + (int64_t)b * kCountersPerSeq + kSeqCounter, n_groups)) return;
    {
        const int64_t row2 = (int64_t)first + b;
        const auto ro = page_rsrc(a.p2_o + row2 * total, part_o * n_groups);
        const auto rm = page_rsrc(a.p2_ml + row2 * hq * 2, part_ml * n_groups);
        merge(ro, rm, n_groups, true, ro, rm);
    }
    };  // segment

    // ---- this workgroup's segment.  Chunk mode: (wg / max_chunks,
    // wg % max_chunks).  Balanced mode: the sequences' tiles laid end to end
    // (T in all) are cut into W = max_chunks equal ranges, range w =
    // [w T / W, (w + 1) T / W); sequence b, tiles [P_b, P_b + n_b), meets
    // ranges first(b) .. last(b), wg_of(x) = ((x + 1) W - 1) / T being the
    // range that holds tile x, and its chunk c lies in range first(b) + c.
    // Workgroup w < W takes the segment holding its range's first tile;
    // workgroup W + b takes sequence b's first segment when b starts inside a
    // range (after that range's first tile).  So every segment has exactly
    // one workgroup, and each workgroup one segment.
    int sb, st0, st1, sc, snc, sfirst;
    if (!a.segmented) {
        sb = wg / a.max_chunks;
        sc = wg % a.max_chunks;
        st0 = sc * a.chunk_tiles;
        st1 = -1;
        snc = -1;
        sfirst = sb * a.max_chunks;
    } else {
        const int W = a.max_chunks;
        const int bid = blockIdx.x;
        // Ranges: consecutive ones (the chunks of a sequence) on one XCD;
        // the B sequence-start workgroups round-robin over the XCDs.
        const int w_self = bid < W ? xcd_remap(bid, W) : -1;
        const int b_self = bid < W ? -1 : bid - W;
        int* const seg = reinterpret_cast<int*>(smem + a.seg_off);  // [6]: the segment found
        long long* const red = reinterpret_cast<long long*>(seg + 8);  // [NW]
        auto tiles_of = [&](int bb) -> long long {
            const long long t = ((long long)a.seq_lens[bb] + kTile - 1) / kTile;
            return t > 0 ? t : 0;
        };
        long long part = 0;
        for (int bb = threadIdx.x; bb < a.batch; bb += BD) part += tiles_of(bb);
        for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
        if (lane == 0) red[wave] = part;
        if (threadIdx.x == 0) seg[0] = -1;
        __syncthreads();
        long long T = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) T += red[w];
        __syncthreads();
        // At most T ranges, so that none is empty and a sequence's chunks
        // are numbered without gaps (range workgroups past them have none).
        const long long Wl = (long long)W < T ? (long long)W : T;
        if (T > (long long)kMaxChunkTiles * Wl) {
            // The lengths outgrew the plan (a balanced plan made for fewer
            // tokens): a range would not fit the page-id window.  Every
            // workgroup sees the same T, so all of them take this branch and
            // write NaN into the whole output instead of a wrong result.
            const int64_t n_out = (int64_t)a.batch * a.n_q_heads * D;
            for (int64_t i = (int64_t)blockIdx.x * BD + threadIdx.x; i < n_out; i += (int64_t)gridDim.x * BD) {
                if (a.out_f32) reinterpret_cast<float*>(a.out)[i] = __builtin_nanf("");
                else reinterpret_cast<half_t*>(a.out)[i] = __builtin_bit_cast(half_t, (uint16_t)0x7E00);
            }
            return;
        }
        auto range_lo = [&](long long w) -> long long { return w * T / Wl; };
        auto range_hi = [&](long long w) -> long long { return (w + 1) * T / Wl; };
        long long carry = 0;
        for (int b0 = 0; b0 < a.batch; b0 += BD) {
            const int bb = b0 + (int)threadIdx.x;
            const long long nb = bb < a.batch ? tiles_of(bb) : 0;
            long long x = nb;  // inclusive scan over the wave
            for (int off = 1; off < 64; off <<= 1) {
                const long long y = __shfl_up(x, off, 64);
                if (lane >= off) x += y;
            }
            if (lane == 63) red[wave] = x;
            __syncthreads();
            long long before = 0, sum = 0;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const long long v = red[w];
                if (w < wave) before += v;
                sum += v;
            }
            const long long pb = carry + before + x - nb;  // P_b
            if (nb > 0) {
                long long w = -1;
                if (w_self >= 0 && w_self < Wl) {
                    const long long lo = range_lo(w_self);
                    if (pb <= lo && lo < pb + nb && lo < range_hi(w_self)) w = w_self;
                } else if (bb == b_self) {
                    const long long f = ((pb + 1) * Wl - 1) / T;
                    if (pb > range_lo(f) && pb < range_hi(f)) w = f;
                }
                if (w >= 0) {  // at most one thread of the workgroup
                    const long long f = ((pb + 1) * Wl - 1) / T, l = ((pb + nb) * Wl - 1) / T;
                    const long long lo = range_lo(w), hi = range_hi(w);
                    seg[0] = bb;
                    seg[1] = (int)((lo > pb ? lo : pb) - pb);
                    seg[2] = (int)((hi < pb + nb ? hi : pb + nb) - pb);
                    seg[3] = (int)(w - f);
                    seg[4] = (int)(l - f + 1);
                    seg[5] = (int)f;
                }
            }
            carry += sum;
            __syncthreads();
        }
        sb = __builtin_amdgcn_readfirstlane(seg[0]);
        if (sb < 0) return;  // no segment (uniform over the workgroup)
        st0 = __builtin_amdgcn_readfirstlane(seg[1]);
        st1 = __builtin_amdgcn_readfirstlane(seg[2]);
        sc = __builtin_amdgcn_readfirstlane(seg[3]);
        snc = __builtin_amdgcn_readfirstlane(seg[4]);
        sfirst = __builtin_amdgcn_readfirstlane(seg[5]);
    }
    segment(sb, st0, st1, sc, snc, sfirst);
}

}  // namespace pg

// ------------------------------------------------------------------ host side

namespace {

constexpr int kWaves = 16;  // every (Hkv, head_dim) layout runs 16 waves per workgroup

// Scale slots per query head: as many of the G groups as fit beside the
// group's query heads in the 16 MFMA columns.
int pick_gs(int g, int head_dim) {
    int gs = 4;
    while (gs > 1 && gs * g > 16) gs >>= 1;
    const int G = head_dim / 32;
    return gs < G ? gs : G;
}

int64_t groups_of(int64_t max_chunks) { return (max_chunks + pg::kMergeGroup - 1) / pg::kMergeGroup; }

// The balanced mode's segment record and scan scratch at the end of LDS.
constexpr int kSegBytes = 8 * 4 + pg::kMaxWaves * 8;

// Dynamic LDS: the larger of the stage ring, the epilogue's per-wave
// (m, l, o) areas and the merge's weights (a sequence in at most
// `max_chunks` chunks), then the segment list at *seg_off.
int lds_bytes(int hkv, int g, int head_dim, int64_t max_chunks, int* seg_off = nullptr) {
    if (groups_of(max_chunks) > pg::kMaxGroups) return pg::kLdsBudget + 1;
    const pg::PageGeom geo = pg::page_geom(hkv, head_dim);
    const int gs = pick_gs(g, head_dim);
    const int64_t hq = (int64_t)hkv * g;
    const int64_t area = (32 + (16 / gs) * head_dim) * 4;
    const int64_t stages = (int64_t)pg::kStages * geo.stage;
    const int64_t epi = (int64_t)geo.nw * area;
    const int64_t merge = max_chunks > 1 ? (pg::kMaxGroups * hq + 2 * hq) * 4 + 16 : 0;
    int64_t bytes = stages > epi ? stages : epi;
    if (merge > bytes) bytes = merge;
    bytes = (bytes + 15) / 16 * 16;
    if (seg_off != nullptr) *seg_off = (int)bytes;
    bytes += kSegBytes;
    return bytes > (int64_t)pg::kLdsBudget ? pg::kLdsBudget + 1 : (int)bytes;
}

struct WorkspaceLayout {
    int64_t counters, p1_o, p1_ml, p2_o, p2_ml, total;
};

int64_t round256(int64_t x) { return (x + 255) / 256 * 256; }

// [counters: counter_region_bytes(batch)][chunk partials: o, then (m, l)]
// [group partials: o, then (m, l); only when a sequence can have more than
// one group], each region 256-byte aligned.  Only the counters carry state
// from one call to the next.
WorkspaceLayout workspace_layout(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t slots, bool level2) {
    const int64_t s2 = level2 ? slots : 0;
    WorkspaceLayout w;
    w.counters = 0;
    w.p1_o = counter_region_bytes(batch);
    w.p1_ml = w.p1_o + round256(slots * num_q_heads * head_dim * 4);
    w.p2_o = w.p1_ml + round256(slots * num_q_heads * 2 * 4);
    w.p2_ml = w.p2_o + round256(s2 * num_q_heads * head_dim * 4);
    w.total = w.p2_ml + round256(s2 * num_q_heads * 2 * 4);
    return w;
}

template <int D, int GS, int HKV>
int launch(dim3 grid, int lds, hipStream_t s, const pg::Args& a) {
    static_assert(pg::page_geom(HKV, D).nw == kWaves, "16 waves per workgroup");
    static std::atomic<uint64_t> lds_raised{0};
    if (lds > 65536 &&
        allow_full_lds(reinterpret_cast<const void*>(&pg::int4_decode_pages_kernel<D, GS, HKV>), lds_raised) != kOk)
        return kLaunchError;
    hipLaunchKernelGGL((pg::int4_decode_pages_kernel<D, GS, HKV>), grid, dim3(64 * kWaves), lds, s, a);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}

// Instantiated (head_dim, scale slots): D = 128 with GS 4 or 2 (up to 8 query
// heads per kv head), D = 64 with GS 2 or 1 (up to 16); Hkv 1, 2, 4 or 8.
bool has_variant(int hkv, int head_dim, int gs) {
    if (hkv != 1 && hkv != 2 && hkv != 4 && hkv != 8) return false;
    if (head_dim == 128) return gs == 4 || gs == 2;
    return head_dim == 64 && (gs == 2 || gs == 1);
}

}  // namespace

bool pages_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_pages) {
    if (num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || num_q_heads / num_kv_heads > 16) return false;
    if (head_dim != 64 && head_dim != 128) return false;
    const int hkv = (int)num_kv_heads, g = (int)(num_q_heads / num_kv_heads);
    if (!has_variant(hkv, (int)head_dim, pick_gs(g, (int)head_dim))) return false;
    // The merge of the most chunks a sequence can need must fit in LDS.
    const int64_t max_tiles = (max_pages * pg::kPageSize + pg::kTile - 1) / pg::kTile;
    const int64_t min_chunks = (max_tiles + pg::kMaxChunkTiles - 1) / pg::kMaxChunkTiles;
    return lds_bytes(hkv, g, (int)head_dim, min_chunks) <= pg::kLdsBudget;
}

int pages_waves() { return kWaves; }

int pages_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_pages,
               int64_t total_tokens, int64_t max_tokens, int32_t tokens_per_split, bool allow_stream,
               int32_t* out_chunk_tiles, int32_t* out_max_chunks, int32_t* out_waves, int64_t* out_workspace_bytes) {
    const int hkv = (int)num_kv_heads, g = (int)(num_q_heads / num_kv_heads);
    const pg::PageGeom geo = pg::page_geom(hkv, (int)head_dim);
    const int64_t cap_tokens = max_pages * pg::kPageSize;
    const bool known = total_tokens >= 0 && max_tokens >= 0;
    if (max_tokens < 0 || max_tokens > cap_tokens) max_tokens = cap_tokens;
    if (total_tokens < 0) total_tokens = batch * max_tokens;
    const int64_t max_tiles = (cap_tokens + pg::kTile - 1) / pg::kTile;
    const int64_t longest_tiles = (max_tokens + pg::kTile - 1) / pg::kTile;
    // The streaming kernel's chunk mode at 8 query heads per kv head (it has
    // no balanced mode there): chunk plans only.
    const bool stream_chunks_only = allow_stream && stream_supported(num_q_heads, num_kv_heads, head_dim) &&
                                    !stream_balanced_supported(num_q_heads, num_kv_heads, head_dim);
    if (known && tokens_per_split <= 0 && total_tokens < batch * max_tokens && !stream_chunks_only) {
        // The streaming kernel's shape runs its own balanced mode (one range
        // a CU, a workgroup walking every piece of its range).
        if (allow_stream && stream_balanced_supported(num_q_heads, num_kv_heads, head_dim) &&
            stream_balanced_plan(batch, num_q_heads, head_dim, total_tokens, out_chunk_tiles, out_max_chunks,
                                 out_workspace_bytes) == kOk) {
            *out_waves = kWaves;
            return kOk;
        }
        // Ragged lengths (known): the balanced mode.  The tiles of all
        // sequences laid end to end, at most tiles_ub of them, in W equal
        // ranges of at least four stages, each within the page-id window.
        // With one workgroup per CU, the W ranges and the B sequence-start
        // workgroups fit the 256 CUs at once when W <= 256 - B.
        const int64_t tiles_ub = (total_tokens + pg::kTile - 1) / pg::kTile + batch;
        const int64_t room = batch < 128 ? 256 - batch : 128;
        int64_t per_wg = (tiles_ub + room - 1) / room;
        if (per_wg < 4 * geo.ts) per_wg = 4 * geo.ts;
        if (per_wg > pg::kMaxChunkTiles) per_wg = pg::kMaxChunkTiles;
        int64_t wgs = (tiles_ub + per_wg - 1) / per_wg;
        if (wgs < 1) wgs = 1;
        const int64_t share = (tiles_ub + wgs - 1) / wgs;
        if (share <= pg::kMaxChunkTiles && wgs <= 8 * pg::kMaxGroups &&
            lds_bytes(hkv, g, (int)head_dim, wgs) <= pg::kLdsBudget) {
            *out_chunk_tiles = -(int32_t)share;  // negative: the balanced mode
            *out_max_chunks = (int32_t)wgs;
            *out_waves = kWaves;
            *out_workspace_bytes =
                wgs > 1 ? workspace_layout(batch, num_q_heads, head_dim, wgs + batch, wgs > pg::kMergeGroup).total : 0;
            return kOk;
        }
    }
    // Chunk mode.  The grid covers every tile block_table can address (the
    // kernel cannot see a length it was not planned for); the lengths steer
    // the chunk size.
    int64_t chunk_tiles;
    if (tokens_per_split > 0) {
        chunk_tiles = (tokens_per_split + pg::kTile - 1) / pg::kTile;
    } else {
        // About one workgroup per CU (256 CUs), each with at least four
        // stages, and the longest sequence cut into equal chunks.
        const int64_t tiles = (total_tokens + pg::kTile - 1) / pg::kTile + batch;
        int64_t per_wg = (tiles + 255) / 256;
        if (per_wg < 4 * geo.ts) per_wg = 4 * geo.ts;
        const int64_t pieces = (longest_tiles + per_wg - 1) / per_wg;
        chunk_tiles = pieces > 0 ? (longest_tiles + pieces - 1) / pieces : per_wg;
        chunk_tiles = (chunk_tiles + geo.ts - 1) / geo.ts * geo.ts;
    }
    if (chunk_tiles < 1) chunk_tiles = 1;
    // The streaming kernel's chunks at 8 query heads per kv head: at most
    // stream_max_chunks() a sequence.
    if (stream_chunks_only) {
        const int64_t min_tiles = (max_tiles + stream_max_chunks() - 1) / stream_max_chunks();
        if (chunk_tiles < min_tiles) chunk_tiles = min_tiles;
    }
    if (chunk_tiles > pg::kMaxChunkTiles) chunk_tiles = pg::kMaxChunkTiles;
    // One chunk per sequence when the longest one fits in a chunk.
    if (chunk_tiles >= longest_tiles && max_tiles <= pg::kMaxChunkTiles) chunk_tiles = max_tiles;
    // Fewer, longer chunks while the merge does not fit.
    while (chunk_tiles < pg::kMaxChunkTiles &&
           lds_bytes(hkv, g, (int)head_dim, (max_tiles + chunk_tiles - 1) / chunk_tiles) > pg::kLdsBudget)
        ++chunk_tiles;
    const int64_t max_chunks = (max_tiles + chunk_tiles - 1) / chunk_tiles;
    if (lds_bytes(hkv, g, (int)head_dim, max_chunks) > pg::kLdsBudget) return kInvalidArgument;
    *out_chunk_tiles = (int32_t)chunk_tiles;
    *out_max_chunks = (int32_t)max_chunks;
    *out_waves = kWaves;
    int64_t ws = max_chunks > 1 ? pages_workspace_bytes(batch, num_q_heads, head_dim, max_chunks) : 0;
    if (max_chunks > 1 && allow_stream && stream_supported(num_q_heads, num_kv_heads, head_dim) &&
        max_chunks <= stream_max_chunks()) {
        const int64_t sw = stream_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, max_chunks);
        if (sw > ws) ws = sw;
    }
    *out_workspace_bytes = ws;
    return kOk;
}

// Workspace of a chunk-mode plan (slots: batch x max_chunks workgroups +
// batch).
int64_t pages_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t max_chunks) {
    return workspace_layout(batch, num_q_heads, head_dim, batch * max_chunks + batch, max_chunks > pg::kMergeGroup)
        .total;
}

int pages_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale, const void* v_scale,
                 const int32_t* block_table, const int32_t* seq_lens, void* output, int32_t output_is_f32,
                 void* workspace, int64_t workspace_bytes_avail, int64_t batch, int64_t num_q_heads,
                 int64_t num_kv_heads, int64_t head_dim, int64_t max_pages, int64_t bt_cols, int32_t page_shift,
                 float softmax_scale, int32_t chunk_tiles, int32_t max_chunks, bool allow_stream, void* stream) {
    const int hkv = (int)num_kv_heads;
    // chunk_tiles > 0: chunk mode, batch x max_chunks workgroups of
    // chunk_tiles tiles; < 0: the balanced mode, max_chunks workgroups
    // sharing every sequence's tiles (-chunk_tiles bounds a share).
    const bool balanced = chunk_tiles < 0;
    const int64_t share = balanced ? -(int64_t)chunk_tiles : chunk_tiles;
    if (share <= 0 || share > pg::kMaxChunkTiles || max_chunks <= 0) return kInvalidArgument;
    // The shapes the streaming kernel has (decode_stream.hip), in either
    // mode: it runs them instead (allow_stream false keeps this kernel, for
    // A/B measurements).  Its workspace layout is this kernel's.
    if (allow_stream &&
        (balanced ? stream_balanced_supported(num_q_heads, num_kv_heads, head_dim) && max_chunks <= 8 * pg::kMaxGroups
                  : stream_supported(num_q_heads, num_kv_heads, head_dim) && max_chunks <= stream_max_chunks()))
        return stream_launch(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output, output_is_f32,
                             workspace, workspace_bytes_avail, batch, num_q_heads, num_kv_heads, head_dim, max_pages,
                             bt_cols, page_shift, softmax_scale, chunk_tiles, max_chunks, stream);
    if (!balanced && share * max_chunks * 2 < max_pages) return kInvalidArgument;
    if (balanced && max_chunks > 8 * pg::kMaxGroups) return kInvalidArgument;
    const int g = (int)(num_q_heads / num_kv_heads);
    const int gs = pick_gs(g, (int)head_dim);
    if (!has_variant(hkv, (int)head_dim, gs)) return kInvalidArgument;
    int seg_off = 0;
    const int lds = lds_bytes(hkv, g, (int)head_dim, max_chunks, &seg_off);
    if (lds > pg::kLdsBudget) return kInvalidArgument;
    // Balanced mode: W range workgroups and B sequence-start workgroups.
    const int64_t nblocks = balanced ? (int64_t)max_chunks + batch : batch * (int64_t)max_chunks;
    if (nblocks > 0x7FFFFFFF - batch) return kInvalidArgument;
    pg::Args a;
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
    a.n_kv_heads = hkv;
    a.group = g;
    a.max_pages = (int)max_pages;
    a.bt_cols = (int)bt_cols;
    a.page_shift = page_shift;
    a.max_chunks = max_chunks;
    a.chunk_tiles = (int)share;
    a.segmented = balanced ? 1 : 0;
    a.slots = (int)((balanced ? (int64_t)max_chunks : nblocks) + batch);  // ranges (or workgroups) + B
    a.seg_off = seg_off;
    a.log2_scale = softmax_scale * 1.4426950408889634f;
    a.counters = nullptr;
    a.p1_o = a.p1_ml = a.p2_o = a.p2_ml = nullptr;
    if (max_chunks > 1) {
        const WorkspaceLayout w = workspace_layout(batch, num_q_heads, head_dim, a.slots, max_chunks > pg::kMergeGroup);
        if (workspace == nullptr || workspace_bytes_avail < w.total) return kWorkspaceTooSmall;
        uint8_t* const ws = (uint8_t*)workspace;
        a.counters = (uint32_t*)(ws + w.counters);
        a.p1_o = (float*)(ws + w.p1_o);
        a.p1_ml = (float*)(ws + w.p1_ml);
        a.p2_o = (float*)(ws + w.p2_o);
        a.p2_ml = (float*)(ws + w.p2_ml);
    }
    const dim3 grid((unsigned)nblocks);
    hipStream_t s = (hipStream_t)stream;
#define IRIS_PAGES_CASE(D_, GS_, HKV_) \
    if (head_dim == D_ && gs == GS_ && hkv == HKV_) return launch<D_, GS_, HKV_>(grid, lds, s, a)
    IRIS_PAGES_CASE(128, 4, 1);
    IRIS_PAGES_CASE(128, 4, 2);
    IRIS_PAGES_CASE(128, 4, 4);
    IRIS_PAGES_CASE(128, 4, 8);
    IRIS_PAGES_CASE(128, 2, 1);
    IRIS_PAGES_CASE(128, 2, 2);
    IRIS_PAGES_CASE(128, 2, 4);
    IRIS_PAGES_CASE(128, 2, 8);
    IRIS_PAGES_CASE(64, 2, 1);
    IRIS_PAGES_CASE(64, 2, 2);
    IRIS_PAGES_CASE(64, 2, 4);
    IRIS_PAGES_CASE(64, 2, 8);
    IRIS_PAGES_CASE(64, 1, 1);
    IRIS_PAGES_CASE(64, 1, 2);
    IRIS_PAGES_CASE(64, 1, 4);
    IRIS_PAGES_CASE(64, 1, 8);
#undef IRIS_PAGES_CASE
    return kInvalidArgument;
}

}  // namespace iris
