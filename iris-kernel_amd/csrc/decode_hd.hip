// INT4 paged decode attention for gfx950 (MI355X): the MFMA kernel for the
// head dims between the fast kernels' 64, 128 and 256, and, in its
// token-page mode, for every page size.
//
// Replaces the TileLang kernel `_int4_paged_decode_attention`
// (src/iris_kernel/fused_attention.py:11-220 in Hunter2030ZeRo/Iris-Kernel)
// for head_dim 96, 160, 192 and 224 (G = 3, 5, 6, 7 scale groups of 32
// dims), any number of kv heads and of query heads per kv head, pages of
// 16 m tokens; in token-page mode (TOK) for head_dim 64 to 256 (G = 2-8)
// and pages of any size, each token's page looked up through the block
// table (ODD: the scale shifts per token, where G x Hkv is odd).  It computes the result of
// `torch_eager_int4_paged_decode_attention`
// (src/iris_kernel/torch_eager_attention.py:154-239), which takes any head
// dim that is a multiple of the group size (:93) and any page size (:72)
// where the reference's fused path takes 64 and 128 and pages of 16
// (fused_attention.py:390-403).
//
// Streaming: a workgroup of W waves (16 at G = 2, 12 at 3, 8 above) owns (sequence,
// kv head, block of up to 16 of its query heads, chunk of 32-token tiles);
// the kv heads of one (sequence, query block, chunk) run on one XCD, one
// after another, so the cache lines their rows share are fetched into one
// L2.  Wave w streams tiles w, w + W, ... of the chunk through two LDS slots
// of its own, with no workgroup barrier in the loop.  Per tile a wave
// * issues the loads of the next tile into the slot the previous tile
//   used, waits for this tile's (vmcnt) and computes it, reading the
//   slot in two phases (K codes and scales before QK, V codes and scales
//   before PV) so that only half of a tile's operands are live in registers
//   at once;
// * loads straight into LDS: the kv head's K and V rows of the tile's 32
//   tokens (16 G bytes a token, one 16-byte piece a lane and load, the
//   pieces token-major) and, per token, the aligned dwords that cover its
//   2 G bytes of each scale tensor (a kv head's scales start on an odd half
//   when kv head * G or the row is odd; the dword count covers the shift);
// * keeps its page ids in lanes of one register (v_readlane); in token-page
//   mode it loads the block-table entries of a tile's 32 tokens into LDS one
//   tile ahead of the data, and each load lane takes its token's slot in the
//   pool with ds_bpermute.
//
// Compute, the query heads of the block as the 16 MFMA columns
// (v_mfma_f32_16x16x32_f16):
// * QK as S^T: per group g and 16-token half, A = the K codes (exact fp16
//   subnormals, nibble + 8; the offset removed by the accumulator's start),
//   B = q; the K scale per (token, group) on the fp32 result;
// * fp32 online softmax in base 2 with lazy rescaling; a head's 32 scores in
//   the four 16-lane rows of its column; the lowest valid score tracked so a
//   non-finite K scale or query gives NaN heads as the eager path does;
// * PV as O^T: A = the V codes transposed (ds_read_b64_tr_b8), B = p *
//   v_scale rounded once to fp16 (the C layout of S^T is the B layout of
//   PV); the V codes' +8 offset removed through the sum of those weights.
// The waves' states are combined through LDS at the end.
//
// Split-KV: chunks publish (o / l, m, l) per query head with device-coherent
// stores; the last to arrive merges them (arrive_last in common.h).
#include "common.h"
#include "decode_hd.h"
#include "iris_hip.h"

namespace iris {
namespace hd {

constexpr int kTile = 32;
constexpr int kMaxTilesPerWave = 32;  // a wave's page ids (two a tile) fill its 64 lanes
constexpr int kMaxChunks = 64;
constexpr int kMergeBatch = 8;
constexpr int kHeads = 16;  // query heads of a workgroup (a block of its kv head's)

typedef int int2v_t __attribute__((ext_vector_type(2)));
#define IRIS_LDS __attribute__((address_space(3)))

template <int G_>
struct Geo {
    static constexpr int G = G_, D = 32 * G_, HB = 16 * G_;  // groups, head_dim, code bytes of a head row
    // waves a workgroup and LDS slots a wave (one tile in flight while one is computed)
    static constexpr int W = G_ <= 2 ? 16 : G_ <= 3 ? 12 : 8;
    static constexpr int R = 2;
    static constexpr int NK = (32 * G_ + 63) / 64;  // 16-byte loads a tensor a tile
    static constexpr int KA = 512 * G_;             // code area of a slot, per tensor (32 G pieces)
    // scale dwords a token needs (at most): G halves from its first one, which
    // is the second half of a dword only where G is odd
    static constexpr int SD = (G_ + (G_ & 1)) / 2;
    static constexpr int SP = SD <= 1 ? 1 : SD <= 2 ? 2 : 4;  // scale dwords a token occupies in LDS
    static constexpr int NS = (32 * SP + 63) / 64;           // 4-byte loads a scale tensor a tile
    static constexpr int NSR = SP == 1 ? 1 : SP == 2 ? 2 : 4;  // 16-byte scale reads a half tile
    static constexpr int NA = (G_ + 1) / 2;                  // aligned scale dwords a token
    // Slot: [K pieces 32 G x 16 B (area KA)][V pieces (KA)][K scales 32 x SP dwords][V scales]
    static constexpr int K_OFF = 0, V_OFF = KA, KS_OFF = 2 * KA, VS_OFF = 2 * KA + 128 * SP;
    static constexpr int SLOT = 2 * KA + 256 * SP;
    static constexpr int RING_BYTES = W * R * SLOT;
    // Epilogue over the ring: per wave [m 16][l 16][o 16 heads x (D + 1)] fp32.
    static constexpr int EPI_ROW = D + 1, EPI_FLOATS = 32 + kHeads * EPI_ROW;
    static constexpr int CTL_OFF = W * EPI_FLOATS * 4;
    static constexpr int MAIN_BYTES = RING_BYTES > CTL_OFF + 16 ? RING_BYTES : CTL_OFF + 16;
    // Token-page mode: a wave's block-table entries of two tiles (32 a tile)
    // past the ring and the epilogue.
    static constexpr int ID_OFF = (MAIN_BYTES + 15) / 16 * 16, ID_BYTES = 2 * 32 * 4;
    static constexpr int LDS_BYTES = MAIN_BYTES;
    static constexpr int LDS_BYTES_TOK = ID_OFF + W * ID_BYTES;
    static_assert(R == 2, "ring depth (the pipeline alternates two slots)");
    static_assert(NA <= SP && SD <= SP, "scale dwords of a token");
    static_assert(LDS_BYTES_TOK <= 160 * 1024, "LDS of a CU");
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
    uint32_t* counters;  // sequence b's at b * kCountersPerSeq: one per (kv head, query block); zero between calls
    float* part_o;       // [B][max_chunks][Hq][D] o / l of each chunk
    float* part_ml;      // [B][max_chunks][Hq][2] (m, l), base-2 logits
    int out_f32;
    int n_q_heads, n_kv_heads, group, q_blocks;
    int n_units;         // batch x max_chunks
    int seq_units;       // batch: the units of one chunk index
    int n_heads_blocks;  // n_kv_heads x q_blocks: the workgroups of a unit
    int max_chunks, chunk_tiles;
    int max_pages;            // 16-token pages a block-table row addresses
    int bt_cols, page_code;   // block-table columns; the page code of virtual_page (page_size = 16 m)
    int page_size;            // tokens a page (token-page mode)
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
// One dword of LDS that a direct-to-LDS load wrote, read as inline assembly
// that waits for its own result (see Reads below).
__device__ __forceinline__ uint32_t lds_read_b32(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    return v;
}
__device__ __forceinline__ void store_sc1(float v, float* p) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_sc1(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS reads of a tile, as inline assembly that waits for its own results:
// the compiler cannot tell them from the loads still streaming into the
// other slot and would wait for those too.  The wave's vmcnt wait for the
// tile precedes them.
// Phase 1, before QK: the K code dwords of (e, g) at kb[e] + 16 g, and the K
// scales of the lane's tokens: 16-byte reads at sb + 16 (16 e + i) (4 scale
// dwords a token) or sb + 8 (16 e + i) for token pairs i, i + 1 (2 a token).
// Phase 2, before PV: the transposed V reads of group g at tb + 16 g and
// the V scales, as the K scales.
#define IRIS_R32(o, b, off) "ds_read_b32 %" #o ", %[" #b "] offset:" #off "\n\t"
#define IRIS_R128(o, off) "ds_read_b128 %" #o ", %[sb] offset:" #off "\n\t"
#define IRIS_TR(o, off) "ds_read_b64_tr_b8 %" #o ", %[tb] offset:" #off "\n\t"
#define IRIS_WAIT "s_waitcnt lgkmcnt(0)"
#define IRIS_S4(o0, o1, o2, o3, o4, o5, o6, o7)                                                              \
    IRIS_R128(o0, 0) IRIS_R128(o1, 16) IRIS_R128(o2, 32) IRIS_R128(o3, 48) IRIS_R128(o4, 256) IRIS_R128(o5, 272) \
        IRIS_R128(o6, 288) IRIS_R128(o7, 304)
#define IRIS_S2(o0, o1, o2, o3) IRIS_R128(o0, 0) IRIS_R128(o1, 16) IRIS_R128(o2, 128) IRIS_R128(o3, 144)
#define IRIS_S4_OUT(x) \
    "=&v"(x[0][0]), "=&v"(x[0][1]), "=&v"(x[0][2]), "=&v"(x[0][3]), "=&v"(x[1][0]), "=&v"(x[1][1]), \
        "=&v"(x[1][2]), "=&v"(x[1][3])
#define IRIS_S2_OUT(x) "=&v"(x[0][0]), "=&v"(x[0][1]), "=&v"(x[1][0]), "=&v"(x[1][1])

template <int G>
struct Reads;
template <>
struct Reads<2> {  // one scale dword a token: tokens 16 e + 4 jq .. + 3 in one 16-byte read at sb + 64 e
    static __device__ __forceinline__ void k(uint32_t kb0, uint32_t kb1, uint32_t sb, uint32_t (&k)[2][2],
                                             u32x4_t (&s)[2][1]) {
        asm volatile(IRIS_R32(0, kb0, 0) IRIS_R32(1, kb0, 16) IRIS_R32(2, kb1, 0) IRIS_R32(3, kb1, 16)
                         IRIS_R128(4, 0) IRIS_R128(5, 64) IRIS_WAIT
                     : "=&v"(k[0][0]), "=&v"(k[0][1]), "=&v"(k[1][0]), "=&v"(k[1][1]), "=&v"(s[0][0]), "=&v"(s[1][0])
                     : [kb0] "v"(kb0), [kb1] "v"(kb1), [sb] "v"(sb)
                     : "memory");
    }
    static __device__ __forceinline__ void v(uint32_t tb, uint32_t sb, int2v_t (&v)[2], u32x4_t (&s)[2][1]) {
        asm volatile(IRIS_TR(0, 0) IRIS_TR(1, 16) IRIS_R128(2, 0) IRIS_R128(3, 64) IRIS_WAIT
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(s[0][0]), "=&v"(s[1][0])
                     : [tb] "v"(tb), [sb] "v"(sb)
                     : "memory");
    }
};
template <>
struct Reads<4> {
    static __device__ __forceinline__ void k(uint32_t kb0, uint32_t kb1, uint32_t sb, uint32_t (&k)[2][4],
                                             u32x4_t (&s)[2][2]) {
        asm volatile(IRIS_R32(0, kb0, 0) IRIS_R32(1, kb0, 16) IRIS_R32(2, kb0, 32) IRIS_R32(3, kb0, 48)
                         IRIS_R32(4, kb1, 0) IRIS_R32(5, kb1, 16) IRIS_R32(6, kb1, 32) IRIS_R32(7, kb1, 48)
                             IRIS_S2(8, 9, 10, 11) IRIS_WAIT
                     : "=&v"(k[0][0]), "=&v"(k[0][1]), "=&v"(k[0][2]), "=&v"(k[0][3]), "=&v"(k[1][0]),
                       "=&v"(k[1][1]), "=&v"(k[1][2]), "=&v"(k[1][3]), IRIS_S2_OUT(s)
                     : [kb0] "v"(kb0), [kb1] "v"(kb1), [sb] "v"(sb)
                     : "memory");
    }
    static __device__ __forceinline__ void v(uint32_t tb, uint32_t sb, int2v_t (&v)[4], u32x4_t (&s)[2][2]) {
        asm volatile(IRIS_TR(0, 0) IRIS_TR(1, 16) IRIS_TR(2, 32) IRIS_TR(3, 48) IRIS_S2(4, 5, 6, 7) IRIS_WAIT
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), IRIS_S2_OUT(s)
                     : [tb] "v"(tb), [sb] "v"(sb)
                     : "memory");
    }
};
template <>
struct Reads<3> {
    static __device__ __forceinline__ void k(uint32_t kb0, uint32_t kb1, uint32_t sb, uint32_t (&k)[2][3],
                                             u32x4_t (&s)[2][2]) {
        asm volatile(IRIS_R32(0, kb0, 0) IRIS_R32(1, kb0, 16) IRIS_R32(2, kb0, 32) IRIS_R32(3, kb1, 0)
                         IRIS_R32(4, kb1, 16) IRIS_R32(5, kb1, 32) IRIS_S2(6, 7, 8, 9) IRIS_WAIT
                     : "=&v"(k[0][0]), "=&v"(k[0][1]), "=&v"(k[0][2]), "=&v"(k[1][0]), "=&v"(k[1][1]),
                       "=&v"(k[1][2]), IRIS_S2_OUT(s)
                     : [kb0] "v"(kb0), [kb1] "v"(kb1), [sb] "v"(sb)
                     : "memory");
    }
    static __device__ __forceinline__ void v(uint32_t tb, uint32_t sb, int2v_t (&v)[3], u32x4_t (&s)[2][2]) {
        asm volatile(IRIS_TR(0, 0) IRIS_TR(1, 16) IRIS_TR(2, 32) IRIS_S2(3, 4, 5, 6) IRIS_WAIT
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), IRIS_S2_OUT(s)
                     : [tb] "v"(tb), [sb] "v"(sb)
                     : "memory");
    }
};
template <>
struct Reads<5> {
    static __device__ __forceinline__ void k(uint32_t kb0, uint32_t kb1, uint32_t sb, uint32_t (&k)[2][5],
                                             u32x4_t (&s)[2][4]) {
        asm volatile(IRIS_R32(0, kb0, 0) IRIS_R32(1, kb0, 16) IRIS_R32(2, kb0, 32) IRIS_R32(3, kb0, 48)
                         IRIS_R32(4, kb0, 64) IRIS_R32(5, kb1, 0) IRIS_R32(6, kb1, 16) IRIS_R32(7, kb1, 32)
                             IRIS_R32(8, kb1, 48) IRIS_R32(9, kb1, 64) IRIS_S4(10, 11, 12, 13, 14, 15, 16, 17) IRIS_WAIT
                     : "=&v"(k[0][0]), "=&v"(k[0][1]), "=&v"(k[0][2]), "=&v"(k[0][3]), "=&v"(k[0][4]),
                       "=&v"(k[1][0]), "=&v"(k[1][1]), "=&v"(k[1][2]), "=&v"(k[1][3]), "=&v"(k[1][4]), IRIS_S4_OUT(s)
                     : [kb0] "v"(kb0), [kb1] "v"(kb1), [sb] "v"(sb)
                     : "memory");
    }
    static __device__ __forceinline__ void v(uint32_t tb, uint32_t sb, int2v_t (&v)[5], u32x4_t (&s)[2][4]) {
        asm volatile(IRIS_TR(0, 0) IRIS_TR(1, 16) IRIS_TR(2, 32) IRIS_TR(3, 48) IRIS_TR(4, 64)
                         IRIS_S4(5, 6, 7, 8, 9, 10, 11, 12) IRIS_WAIT
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), IRIS_S4_OUT(s)
                     : [tb] "v"(tb), [sb] "v"(sb)
                     : "memory");
    }
};
template <>
struct Reads<6> {
    static __device__ __forceinline__ void k(uint32_t kb0, uint32_t kb1, uint32_t sb, uint32_t (&k)[2][6],
                                             u32x4_t (&s)[2][4]) {
        asm volatile(IRIS_R32(0, kb0, 0) IRIS_R32(1, kb0, 16) IRIS_R32(2, kb0, 32) IRIS_R32(3, kb0, 48)
                         IRIS_R32(4, kb0, 64) IRIS_R32(5, kb0, 80) IRIS_R32(6, kb1, 0) IRIS_R32(7, kb1, 16)
                             IRIS_R32(8, kb1, 32) IRIS_R32(9, kb1, 48) IRIS_R32(10, kb1, 64) IRIS_R32(11, kb1, 80)
                                 IRIS_S4(12, 13, 14, 15, 16, 17, 18, 19) IRIS_WAIT
                     : "=&v"(k[0][0]), "=&v"(k[0][1]), "=&v"(k[0][2]), "=&v"(k[0][3]), "=&v"(k[0][4]),
                       "=&v"(k[0][5]), "=&v"(k[1][0]), "=&v"(k[1][1]), "=&v"(k[1][2]), "=&v"(k[1][3]),
                       "=&v"(k[1][4]), "=&v"(k[1][5]), IRIS_S4_OUT(s)
                     : [kb0] "v"(kb0), [kb1] "v"(kb1), [sb] "v"(sb)
                     : "memory");
    }
    static __device__ __forceinline__ void v(uint32_t tb, uint32_t sb, int2v_t (&v)[6], u32x4_t (&s)[2][4]) {
        asm volatile(IRIS_TR(0, 0) IRIS_TR(1, 16) IRIS_TR(2, 32) IRIS_TR(3, 48) IRIS_TR(4, 64) IRIS_TR(5, 80)
                         IRIS_S4(6, 7, 8, 9, 10, 11, 12, 13) IRIS_WAIT
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), IRIS_S4_OUT(s)
                     : [tb] "v"(tb), [sb] "v"(sb)
                     : "memory");
    }
};
template <>
struct Reads<7> {
    static __device__ __forceinline__ void k(uint32_t kb0, uint32_t kb1, uint32_t sb, uint32_t (&k)[2][7],
                                             u32x4_t (&s)[2][4]) {
        asm volatile(IRIS_R32(0, kb0, 0) IRIS_R32(1, kb0, 16) IRIS_R32(2, kb0, 32) IRIS_R32(3, kb0, 48)
                         IRIS_R32(4, kb0, 64) IRIS_R32(5, kb0, 80) IRIS_R32(6, kb0, 96) IRIS_R32(7, kb1, 0)
                             IRIS_R32(8, kb1, 16) IRIS_R32(9, kb1, 32) IRIS_R32(10, kb1, 48) IRIS_R32(11, kb1, 64)
                                 IRIS_R32(12, kb1, 80) IRIS_R32(13, kb1, 96)
                                     IRIS_S4(14, 15, 16, 17, 18, 19, 20, 21) IRIS_WAIT
                     : "=&v"(k[0][0]), "=&v"(k[0][1]), "=&v"(k[0][2]), "=&v"(k[0][3]), "=&v"(k[0][4]),
                       "=&v"(k[0][5]), "=&v"(k[0][6]), "=&v"(k[1][0]), "=&v"(k[1][1]), "=&v"(k[1][2]),
                       "=&v"(k[1][3]), "=&v"(k[1][4]), "=&v"(k[1][5]), "=&v"(k[1][6]), IRIS_S4_OUT(s)
                     : [kb0] "v"(kb0), [kb1] "v"(kb1), [sb] "v"(sb)
                     : "memory");
    }
    static __device__ __forceinline__ void v(uint32_t tb, uint32_t sb, int2v_t (&v)[7], u32x4_t (&s)[2][4]) {
        asm volatile(IRIS_TR(0, 0) IRIS_TR(1, 16) IRIS_TR(2, 32) IRIS_TR(3, 48) IRIS_TR(4, 64) IRIS_TR(5, 80)
                         IRIS_TR(6, 96) IRIS_S4(7, 8, 9, 10, 11, 12, 13, 14) IRIS_WAIT
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                       IRIS_S4_OUT(s)
                     : [tb] "v"(tb), [sb] "v"(sb)
                     : "memory");
    }
};
template <>
struct Reads<8> {
    static __device__ __forceinline__ void k(uint32_t kb0, uint32_t kb1, uint32_t sb, uint32_t (&k)[2][8],
                                             u32x4_t (&s)[2][4]) {
        asm volatile(IRIS_R32(0, kb0, 0) IRIS_R32(1, kb0, 16) IRIS_R32(2, kb0, 32) IRIS_R32(3, kb0, 48)
                         IRIS_R32(4, kb0, 64) IRIS_R32(5, kb0, 80) IRIS_R32(6, kb0, 96) IRIS_R32(7, kb0, 112)
                             IRIS_R32(8, kb1, 0) IRIS_R32(9, kb1, 16) IRIS_R32(10, kb1, 32) IRIS_R32(11, kb1, 48)
                                 IRIS_R32(12, kb1, 64) IRIS_R32(13, kb1, 80) IRIS_R32(14, kb1, 96)
                                     IRIS_R32(15, kb1, 112) IRIS_S4(16, 17, 18, 19, 20, 21, 22, 23) IRIS_WAIT
                     : "=&v"(k[0][0]), "=&v"(k[0][1]), "=&v"(k[0][2]), "=&v"(k[0][3]), "=&v"(k[0][4]),
                       "=&v"(k[0][5]), "=&v"(k[0][6]), "=&v"(k[0][7]), "=&v"(k[1][0]), "=&v"(k[1][1]),
                       "=&v"(k[1][2]), "=&v"(k[1][3]), "=&v"(k[1][4]), "=&v"(k[1][5]), "=&v"(k[1][6]),
                       "=&v"(k[1][7]), IRIS_S4_OUT(s)
                     : [kb0] "v"(kb0), [kb1] "v"(kb1), [sb] "v"(sb)
                     : "memory");
    }
    static __device__ __forceinline__ void v(uint32_t tb, uint32_t sb, int2v_t (&v)[8], u32x4_t (&s)[2][4]) {
        asm volatile(IRIS_TR(0, 0) IRIS_TR(1, 16) IRIS_TR(2, 32) IRIS_TR(3, 48) IRIS_TR(4, 64) IRIS_TR(5, 80)
                         IRIS_TR(6, 96) IRIS_TR(7, 112) IRIS_S4(8, 9, 10, 11, 12, 13, 14, 15) IRIS_WAIT
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                       "=&v"(v[7]), IRIS_S4_OUT(s)
                     : [tb] "v"(tb), [sb] "v"(sb)
                     : "memory");
    }
};
#undef IRIS_R32
#undef IRIS_R128
#undef IRIS_TR
#undef IRIS_WAIT
#undef IRIS_S4
#undef IRIS_S2
#undef IRIS_S4_OUT
#undef IRIS_S2_OUT

// The scale dwords of the lane's token 16 e + 4 jq + i from a phase's
// 16-byte reads, aligned to its kv head's first half (v_alignbit by 0 or 16
// bits): half c & 1 of dword c / 2 is group c.  Dwords past the loaded ones
// reach only halves that are never used.
template <int G>
__device__ __forceinline__ void aligned_scales(const u32x4_t (&raw)[2][Geo<G>::NSR], int e, int i,
                                               uint32_t shift, uint32_t (&out)[Geo<G>::NA]) {
    constexpr int SP = Geo<G>::SP;
    uint32_t w[SP];
#pragma unroll
    for (int j = 0; j < SP; ++j) {
        if constexpr (SP == 4) w[j] = raw[e][i][j];
        else if constexpr (SP == 2) w[j] = raw[e][i >> 1][2 * (i & 1) + j];
        else w[j] = raw[e][0][i];
    }
#pragma unroll
    for (int c = 0; c < Geo<G>::NA; ++c) out[c] = __builtin_amdgcn_alignbit(c + 1 < SP ? w[c + 1] : 0u, w[c], shift);
}

// TOK: token-page mode (any page size; a tile's tokens looked up one by one
// through the block table); otherwise pages of 16 m tokens.  ODD (token
// pages only): Hkv x G odd, so a kv head's scales start on either half of a
// dword depending on the token's slot; the shift is then taken per token.
template <int G, bool TOK, bool ODD>
__global__ __launch_bounds__(64 * Geo<G>::W) void int4_decode_hd_kernel(Args a) {
    static_assert(TOK || !ODD, "per-token scale shifts are a token-page mode");
    using L = Geo<G>;
    constexpr int D = L::D, HB = L::HB, W = L::W, NK = L::NK, NS = L::NS, SP = L::SP, SLOT = L::SLOT;
    // G = 8 in token-page mode: a kv head's 8 scales are one 16-byte-aligned
    // 16 bytes, so one 16-byte load a token covers both scale tensors (K
    // scales in lanes 0-31, V scales in lanes 32-63)
    constexpr bool S16 = TOK && G == 8;
    static_assert(!S16 || (SP == 4 && L::VS_OFF == L::KS_OFF + 512), "the 16-byte scale load's LDS layout");
    // G = 2 (one scale dword a kv head, token pages only): one 4-byte load a
    // token covers both tensors the same way (K at KS_OFF + 4 t, V at
    // VS_OFF + 4 t = KS_OFF + 128 + 4 t)
    constexpr bool S4 = TOK && G == 2;
    static_assert(TOK || SP > 1, "one-dword scale rows: token-page mode only");
    static_assert(!S4 || (SP == 1 && L::VS_OFF == L::KS_OFF + 128), "the 4-byte scale load's LDS layout");
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15;   // MFMA row (A) or column (B, C): token or query head
    const int jq = lane >> 4;  // MFMA k-chunk (A, B) or row quad (C)

    // ---- ((kv head, query block), unit = (chunk, sequence b), chunk
    // slowest).  Workgroups are dispatched to the 8 XCDs in turn (workgroup
    // i to XCD i % 8), and a kv head's rows are only 16 G of each token's
    // Hkv 16 G bytes, which every query block of the kv head reads: the
    // (kv head, query block) pairs of one unit run on one XCD, one after
    // another (k = i / 8, unit (k / (Hkv Q)) 8 + i % 8, pair k % (Hkv Q)),
    // so the cache lines they share are fetched into one L2.  With the
    // chunk index slowest, each XCD gets its share of every chunk index
    // (chunks past a sequence's end, which return at once, would otherwise
    // leave whole XCDs idle when the table is wider than the sequences);
    // within chunk c the sequence index is rotated by c, so a sequence's
    // chunks run on different XCDs (a long sequence of a ragged batch would
    // otherwise load one XCD's share of the bandwidth).  The grid is padded
    // to whole groups of 8 units; padding workgroups return at once.  The
    // divisions run on the VALU; readfirstlane keeps the results, and all
    // that derives from them (the loop bounds among it), scalar.
    const int k_x = blockIdx.x >> 3;
    const int hb = __builtin_amdgcn_readfirstlane(k_x % a.n_heads_blocks);  // (kv head, query block)
    const int kvh = __builtin_amdgcn_readfirstlane(hb / a.q_blocks);
    const int qb = __builtin_amdgcn_readfirstlane(hb - kvh * a.q_blocks);
    const int unit = __builtin_amdgcn_readfirstlane((k_x / a.n_heads_blocks) * 8 + (blockIdx.x & 7));
    if (unit >= a.n_units) return;
    const int chunk = __builtin_amdgcn_readfirstlane(unit / a.seq_units);
    const int b = __builtin_amdgcn_readfirstlane(rotate_back(unit - chunk * a.seq_units, chunk, a.seq_units));
    const int t_begin = chunk * a.chunk_tiles;
    const int p0 = 2 * t_begin;  // first 16-token page of the chunk
    const int32_t* bt = a.block_table + (int64_t)b * a.bt_cols;
    const int h_first = qb * kHeads;
    const int nh = min(a.group - h_first, kHeads);  // query heads of the block
    const int hq0 = kvh * a.group + h_first;        // its first query head

    // ---- this wave's page ids (lane l: chunk page 2 (W (l >> 1) + wave) +
    // (l & 1), i.e. page l & 1 of its tile l >> 1, up to 32 tiles, clamped
    // into the table row), q and the length, in flight together
    int my_pid = 0;
    if constexpr (!TOK)
        my_pid = virtual_page(bt, min(p0 + 2 * (W * (lane >> 1) + wave) + (lane & 1), a.max_pages - 1), a.page_code);
    // q as the QK B operand: lane (head n, k-chunk jq) holds dims 32 g + 8 jq
    // .. + 7 of head n (zero for columns past the block's heads)
    const bool col_valid = n < nh;
    u32x4_t qraw[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        qraw[g] = u32x4_t{0, 0, 0, 0};
        if (col_valid)
            qraw[g] = *reinterpret_cast<const u32x4_t*>(a.q + ((int64_t)b * a.n_q_heads + hq0 + n) * D + 32 * g + 8 * jq);
    }
    const int seq_len = __builtin_amdgcn_readfirstlane(a.seq_lens[b]);
    asm volatile("" ::: "memory");  // keeps the loads above issued before the early return below

    const int n_tiles = (seq_len + kTile - 1) / kTile;
    if (t_begin >= n_tiles) return;  // uniform over the workgroup
    const int t_end = min(t_begin + a.chunk_tiles, n_tiles);
    const int n_ct = t_end - t_begin;
    const int n_chunks = (n_tiles + a.chunk_tiles - 1) / a.chunk_tiles;
    const int last_lp = (seq_len + 15) / 16 - 1;
    // Table entries past jlim (pages past the sequence or the chunk) are
    // never read: a tile's second page past it is read as its first.
    const int jlim = min(last_lp - p0, 2 * n_ct - 1);

    // ---- loads of this wave's tile s into slot `slot` of its ring.
    // Codes: piece p = 64 i + lane (p < 32 G) is token p / G, group p % G of
    // the tile, at 16 p in the tensor's area.
    // Scales: piece p = 64 i + lane is dword j = p % SP of token t = p / SP,
    // at 4 p; token t's dwords start at the dword holding its kv head's first
    // scale (byte o_t = ((page * 16 + m) * Hkv + kvh) * 2 G, m = t & 15), and
    // only those that hold some of its 2 G bytes are loaded (the tensor's end
    // is a multiple of 32 bytes, so none of them passes it).
    // Per-lane offsets within a page (32-bit: a page is 16 token rows of
    // Hkv kv heads) and per-tile uniform page bases; code load i reads page b
    // from lane 16 G - 64 i on, scale load i from token 16 (p >= 16 SP).
    const int64_t page_bytes = (int64_t)16 * a.n_kv_heads * HB;     // a page of a code tensor
    const int64_t spage_bytes = (int64_t)16 * a.n_kv_heads * G * 2;  // a page of a scale tensor
    uint32_t code_off[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const int p = 64 * i + lane;
        const int m = p / G, c = p - m * G;
        code_off[i] = (uint32_t)(((m & 15) * a.n_kv_heads + kvh) * HB + 16 * c);
    }
    uint32_t sc_off[NS];
    bool sc_ok[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        const int p = 64 * i + lane;
        const int t = p / SP, j = p % SP;
        const int h0 = ((t & 15) * a.n_kv_heads + kvh) * G;  // first half, less the page's (an even count)
        const int sh = h0 & 1;
        sc_ok[i] = 2 * j < G + sh;  // the dword holds some of the kv head's halves
        sc_off[i] = (uint32_t)((h0 - sh) * 2 + 4 * j);
    }
    uint8_t* const ring = smem + wave * L::R * SLOT;
    const int n_my = n_ct > wave ? (n_ct - wave + W - 1) / W : 0;
    auto issue = [&](int s, int slot) __attribute__((always_inline)) {
        uint8_t* const dst = ring + slot * SLOT;
        const int t = W * s + wave;  // chunk-relative tile
        const int pa = __builtin_amdgcn_readlane(my_pid, 2 * s);
        const int pb = 2 * t + 1 > jlim ? pa : __builtin_amdgcn_readlane(my_pid, 2 * s + 1);
        const uint8_t* const ka = a.k_data + pa * page_bytes;
        const uint8_t* const kb = a.k_data + pb * page_bytes;
        const uint8_t* const va = a.v_data + pa * page_bytes;
        const uint8_t* const vb = a.v_data + pb * page_bytes;
#pragma unroll
        for (int i = 0; i < NK; ++i) {
            if (NK * 64 == 32 * G || 64 * i + lane < 32 * G) {
                const bool second = lane >= 16 * G - 64 * i;
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>((second ? kb : ka) + code_off[i]),
                                                 (IRIS_LDS void*)(dst + L::K_OFF + 1024 * i), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>((second ? vb : va) + code_off[i]),
                                                 (IRIS_LDS void*)(dst + L::V_OFF + 1024 * i), 16, 0, 0);
            }
        }
        const uint8_t* const ksa = a.k_scale + pa * spage_bytes;
        const uint8_t* const ksb = a.k_scale + pb * spage_bytes;
        const uint8_t* const vsa = a.v_scale + pa * spage_bytes;
        const uint8_t* const vsb = a.v_scale + pb * spage_bytes;
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if (sc_ok[i]) {
                const bool second = 64 * i + lane >= 16 * SP;
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>((second ? ksb : ksa) + sc_off[i]),
                                                 (IRIS_LDS void*)(dst + L::KS_OFF + 256 * i), 4, 0, 0);
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>((second ? vsb : vsa) + sc_off[i]),
                                                 (IRIS_LDS void*)(dst + L::VS_OFF + 256 * i), 4, 0, 0);
            }
        }
    };

    // ---- token-page mode: a tile's 32 tokens (the last valid one for those
    // past the sequence) are looked up one by one.  Lane l < 32 loads the
    // block-table entry of token l into the wave's entry slot (tile & 1),
    // one tile before the tile's data loads; then each lane turns its entry
    // into the token's slot in the pool (entry * page_size + token %
    // page_size) and every load lane takes its token's slot with
    // ds_bpermute.  With Hkv * G even every token's kv head starts on the
    // same half of a scale dword ((kvh G) & 1); with it odd (ODD) the half is
    // the parity of slot Hkv G + kvh G, taken per token: for the loads, and,
    // as a 32-bit mask of the tile's tokens (a ballot at the slot lookup),
    // for the reads.
    uint8_t* const ent_base = smem + L::ID_OFF + wave * L::ID_BYTES;
    const int psz = a.page_size;
    auto issue_entries = [&](int s) __attribute__((always_inline)) {
        const int tg = min((t_begin + W * s + wave) * kTile + lane, seq_len - 1);
        if (lane < 32)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(bt + min(tg / psz, a.bt_cols - 1)),
                                             (IRIS_LDS void*)(ent_base + (s & 1) * 128), 4, 0, 0);
    };
    const int64_t row_bytes = (int64_t)a.n_kv_heads * HB;       // a token row of a code tensor
    const int64_t srow_halves = (int64_t)a.n_kv_heads * G;      // a token row of a scale tensor
    const int tok_sh = (kvh * G) & 1;                           // (Hkv * G even)
    auto slots_of = [&](int s, uint32_t& odd_mask) __attribute__((always_inline)) -> uint32_t {
        const uint32_t e = lds_read_b32(lds_addr(ent_base + (s & 1) * 128) + 4 * (lane & 31));
        const int tg = min((t_begin + W * s + wave) * kTile + (lane & 31), seq_len - 1);
        const uint32_t slot = e * (uint32_t)psz + (uint32_t)(tg % psz);  // a pool of at most 2^32 token slots
        if constexpr (ODD)  // bit t: token t's kv head starts on the second half of a dword
            odd_mask = (uint32_t)__ballot(((slot * (uint32_t)srow_halves + (uint32_t)(kvh * G)) & 1u) != 0);
        return slot;
    };
    auto issue_tok = [&](int slot, uint32_t slots) __attribute__((always_inline)) {
        uint8_t* const dst = ring + slot * SLOT;
#pragma unroll
        for (int i = 0; i < NK; ++i) {
            const int p = 64 * i + lane;
            const int m = (p < 32 * G ? p : 0) / G, c = p - (p / G) * G;
            const uint32_t sm = __builtin_amdgcn_ds_bpermute(4 * m, (int)slots);  // every lane, outside the branch
            if (NK * 64 == 32 * G || p < 32 * G) {
                const int64_t off = (int64_t)sm * row_bytes + kvh * HB + 16 * c;
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(a.k_data + off),
                                                 (IRIS_LDS void*)(dst + L::K_OFF + 1024 * i), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(a.v_data + off),
                                                 (IRIS_LDS void*)(dst + L::V_OFF + 1024 * i), 16, 0, 0);
            }
        }
        if constexpr (S16 || S4) {
            // G = 8 or 2: a kv head's scales are one aligned 16 or 4 bytes,
            // so one load covers both tensors: lane t < 32 the K scales of
            // token t, lane 32 + t its V scales (right after the K area)
            const uint32_t st = __builtin_amdgcn_ds_bpermute(4 * (lane & 31), (int)slots);
            const int64_t off = ((int64_t)st * srow_halves + kvh * G) * 2;
            const void* const src = reinterpret_cast<const void*>((lane < 32 ? a.k_scale : a.v_scale) + off);
            if constexpr (S16) __builtin_amdgcn_global_load_lds(src, (IRIS_LDS void*)(dst + L::KS_OFF), 16, 0, 0);
            else __builtin_amdgcn_global_load_lds(src, (IRIS_LDS void*)(dst + L::KS_OFF), 4, 0, 0);
            return;
        }
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int p = 64 * i + lane;
            const int t = p / SP, j = p % SP;
            const uint32_t st = __builtin_amdgcn_ds_bpermute(4 * t, (int)slots);
            int sh = tok_sh;
            bool ok = sc_ok[i];
            if constexpr (ODD) {
                sh = (int)((st * (uint32_t)srow_halves + (uint32_t)(kvh * G)) & 1u);
                ok = 2 * j < G + sh;  // (j = 0 in every token: each load has a lane)
            }
            if (ok) {
                const int64_t off = (((int64_t)st * srow_halves + kvh * G) - sh) * 2 + 4 * j;
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(a.k_scale + off),
                                                 (IRIS_LDS void*)(dst + L::KS_OFF + 256 * i), 4, 0, 0);
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(a.v_scale + off),
                                                 (IRIS_LDS void*)(dst + L::VS_OFF + 256 * i), 4, 0, 0);
            }
        }
    };

    // ---- q operands (in the order of k_operand; high-nibble dims / 16) and
    // the accumulator start that removes the +8 of the K codes: C row (token)
    // of column n starts at -8 * 2^-24 * (sum of q over the group).
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

    // ---- per-lane LDS offsets within a slot, and the half shift of the
    // lane's tokens' scales: token 16 e + 4 jq + i starts on half
    // ((i Hkv + kvh) G) & 1 of its first dword (the page and 4 jq terms are even)
    const uint32_t k_rd = (uint32_t)(L::K_OFF + (n * G) * 16 + 4 * jq);  // + 256 G e + 16 g
    // K scales of token 16 e + 4 jq + i at + 16 (16 e + i) (four dwords a
    // token), or of the token pair i, i + 1 at + 8 (16 e + i) (two)
    const uint32_t s_rd = (uint32_t)(L::KS_OFF + 4 * SP * (4 * jq));
    constexpr uint32_t kVsDelta = L::VS_OFF - L::KS_OFF;
    // Transposed V reads: lane (n, jq) supplies the 8-byte half (n & 1) of
    // token tr_tok's piece of group g; after the 8 x 8 byte transpose it holds
    // byte column n (dims 2 n, 2 n + 1 of the group) of tokens
    // 16 (k' >> 2) + 4 jq + (k' & 3), k' the byte index.
    const int trk = n >> 1;
    const int tr_tok = 4 * jq + (trk & 3) + 16 * (trk >> 2);
    const uint32_t tr_rd = (uint32_t)(L::V_OFF + (tr_tok * G) * 16 + 8 * (n & 1));  // + 16 g
    uint32_t shift[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) shift[i] = (uint32_t)((((i * a.n_kv_heads + kvh) * G) & 1) * 16);
    constexpr int NSR = L::NSR;  // 16-byte scale reads a half tile

    const float c24 = a.log2_scale * 16777216.0f;  // MFMA units -> base-2 logits
    const float lazy = 2.0f / c24;                 // rescale when a maximum grows by more (base 2)
    float m_run = -INFINITY;                       // MFMA units
    float l_part = 0.0f;
    float s_lo = INFINITY;                         // lowest valid score seen
    // wsum[g]: the lane's share of the sum of group g's PV weights (the fp16
    // B operand), for the V codes' +8 offset (a v_dot2 with ones a pair).
    float wsum[G];
    float4_t o[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        wsum[g] = 0.0f;
        o[g][0] = o[g][1] = float4_t{0, 0, 0, 0};
    }
    const half2_t ones = {(half_t)1.0f, (half_t)1.0f};

    // One tile whose slot has landed: s[e][i] is token 16 e + 4 jq + i,
    // query head n.
    // odd_mask: the tile's per-token scale shifts (ODD; see slots_of)
    auto compute = [&](int tile, uint32_t base, uint32_t odd_mask) __attribute__((always_inline)) {
        // the half shift of the scales of token 16 e + 4 jq + i
        auto shift_of = [&](int e, int i) -> uint32_t {
            if constexpr (ODD) return ((odd_mask >> (16 * e + 4 * jq + i)) & 1u) * 16u;
            else return shift[i];
        };
        const int tok0 = tile * kTile;
        const bool full = tok0 + kTile <= seq_len;
        uint32_t kw[2][G];
        u32x4_t sraw[2][NSR];
        Reads<G>::k(base + k_rd, base + k_rd + 256 * G, base + s_rd, kw, sraw);
        float s[2][4];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            float4_t acc[G];
#pragma unroll
            for (int g = 0; g < G; ++g)
                acc[g] = mfma16x16x32(k_operand(kw[e][g]), qm[g], float4_t{qinit[g], qinit[g], qinit[g], qinit[g]});
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t ks[L::NA];
                aligned_scales<G>(sraw, e, i, shift_of(e, i), ks);
                float sc = 0.0f;
#pragma unroll
                for (int g = 0; g < G; ++g) sc = __builtin_fmaf((float)as_half2(ks[g >> 1])[g & 1], acc[g][i], sc);
                s[e][i] = sc;
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
        mx = row_max4(mx);  // finite (token tok0 < seq_len) unless a score is NaN
        if (__ballot(mx > m_run + lazy) != 0) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c24);
            m_run = m_new;
            l_part *= alpha;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                wsum[g] *= alpha;
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
        int2v_t vw[G];
        Reads<G>::v(base + tr_rd, base + s_rd + kVsDelta, vw, sraw);
        uint32_t vs[2][4][L::NA];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) aligned_scales<G>(sraw, e, i, shift_of(e, i), vs[e][i]);
        if (!full) {
            // Tokens past seq_len may hold any bytes: never let their scale
            // reach the product (0 * NaN).  A real branch.
            const int nv = opaque_int(nval);
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (16 * e + i >= nv)
#pragma unroll
                        for (int c = 0; c < L::NA; ++c) vs[e][i][c] = 0u;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            half8_t bp;
#pragma unroll
            for (int sl = 0; sl < 8; ++sl) {
                const int e = kVSlotByte[sl] >> 2, i = kVSlotByte[sl] & 3;
                bp[sl] = (half_t)__builtin_fmaf(p[e][i], (float)as_half2(vs[e][i][g >> 1])[g & 1], 0.0f);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                wsum[g] = __builtin_amdgcn_fdot2(half2_t{bp[2 * j], bp[2 * j + 1]}, ones, wsum[g], false);
            half8_t lo, hi;
            v_operands(vw[g], lo, hi);
            o[g][0] = mfma16x16x32(lo, bp, o[g][0]);
            o[g][1] = mfma16x16x32(hi, bp, o[g][1]);
        }
    };

    // ---- the pipeline, per wave (no workgroup barrier), two LDS slots: tile
    // s is computed from slot s & 1 once this wave's loads of it have landed
    // (vmcnt counts in order; every load instruction of a tile has a lane
    // that issues it, so a tile is always JOBS of them), with tile s + 1 in
    // flight into the other slot, whose reads by tile s - 1 have returned.
    // (Three slots, two tiles in flight, measured 1-7% slower at G = 3, 4
    // and 5 on MI355X.)
    //
    // Token-page mode: per tile one more load (its block-table entries), one
    // tile ahead of the data: iteration s reads the entries of tile s + 1
    // (loaded at s - 1, before the data of tile s), issues the entries of
    // tile s + 2, then the data of tile s + 1.
    constexpr int JOBS = 2 * NK + (S16 || S4 ? 1 : 2 * NS);
    static_assert(JOBS + 2 < 64, "vmcnt range");
    const uint32_t ring_addr = lds_addr(ring);
    uint32_t odd_cur = 0, odd_next = 0;  // (ODD) the scale shifts of tiles s and s + 1
    if constexpr (TOK) {
        // entries of tiles 0 and 1, then the data of tile 0
        if (n_my > 0) issue_entries(0);
        if (n_my > 1) issue_entries(1);
        wait_vmcnt<0>();
        if (n_my > 0) issue_tok(0, slots_of(0, odd_cur));
    } else {
        if (n_my > 0) issue(0, 0);
    }
    for (int s = 0; s < n_my; ++s) {
        const int next = (s + 1) & 1;  // slot of tile s + 1
        if (s + 1 < n_my) {
            if constexpr (!TOK) {
                issue(s + 1, next);
                wait_vmcnt<JOBS>();  // tile s
            } else {
                wait_vmcnt<JOBS>();  // the entries of tile s + 1 (tile s's data may fly)
                const uint32_t sl = slots_of(s + 1, odd_next);
                if (s + 2 < n_my) {
                    issue_entries(s + 2);
                    issue_tok(next, sl);
                    wait_vmcnt<JOBS + 1>();  // tile s
                } else {
                    issue_tok(next, sl);
                    wait_vmcnt<JOBS>();  // tile s
                }
            }
        } else {
            wait_vmcnt<0>();
        }
        compute(t_begin + W * s + wave, ring_addr + (uint32_t)((s & 1) * SLOT), odd_cur);
        odd_cur = odd_next;
    }
    wait_vmcnt<0>();
    __syncthreads();

    // ---- each wave's (m, l, o) in LDS area `wave`: [0, 16) m (base-2
    // logits), [16, 32) l, [32 + h EPI_ROW + d] o (code offset removed).
    {
        l_part = row_sum4(poison_if_neg_inf(s_lo, l_part));
        float* const ep = reinterpret_cast<float*>(smem) + wave * L::EPI_FLOATS;
        if (jq == 0) {
            ep[n] = m_run * c24;
            ep[16 + n] = l_part;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float psr = 8.0f * row_sum4(wsum[g]);
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ep[32 + n * L::EPI_ROW + 32 * g + 2 * (4 * jq + i) + e] =
                        o[g][e][i] * (e ? 1048576.0f : 16777216.0f) - psr;
        }
    }
    __syncthreads();

    // ---- the chunk's result for element idx = (query head h of the block,
    // dim d): the W waves' states combined (a wave without tiles has
    // m = -inf, l = 0, o = 0 and weight 0)
    const float* const ep0 = reinterpret_cast<const float*>(smem);
    const int hq = a.n_q_heads;
    const int n_el = nh * D;
    auto combine = [&](int idx, float& mc, float& lc) -> float {
        const int h = idx / D, d = idx - h * D;
        mc = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) mc = fmaxf(mc, ep0[w * L::EPI_FLOATS + h]);
        lc = 0.0f;
        float oc = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float* const ep = ep0 + w * L::EPI_FLOATS;
            const float f = __builtin_amdgcn_exp2f(ep[h] - mc);
            lc += ep[16 + h] * f;
            oc += ep[32 + h * L::EPI_ROW + d] * f;
        }
        return oc * (1.0f / lc);
    };
    const int64_t out0 = ((int64_t)b * hq + hq0) * D;  // the block's first output element
    auto store_out = [&](int idx, float v) {
        if (a.out_f32) reinterpret_cast<float*>(a.out)[out0 + idx] = v;
        else reinterpret_cast<half_t*>(a.out)[out0 + idx] = (half_t)v;
    };
    if (n_chunks == 1) {
        for (int idx = threadIdx.x; idx < n_el; idx += blockDim.x) {
            float mc, lc;
            store_out(idx, combine(idx, mc, lc));
        }
        return;
    }

    // ---- split-KV: publish (o / l, m, l) with device-coherent stores; the
    // last chunk of this (sequence, kv head, query block) to arrive merges.
    auto part_row = [&](int c) -> int64_t { return ((int64_t)b * a.max_chunks + c) * hq + hq0; };
    for (int idx = threadIdx.x; idx < n_el; idx += blockDim.x) {
        float mc, lc;
        const float oc = combine(idx, mc, lc);
        store_sc1(oc, a.part_o + part_row(chunk) * D + idx);
        const int h = idx / D;
        if (idx - h * D == 0) {
            store_sc1(mc, a.part_ml + (part_row(chunk) + h) * 2);
            store_sc1(lc, a.part_ml + (part_row(chunk) + h) * 2 + 1);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    uint32_t* const ctl = reinterpret_cast<uint32_t*>(smem + L::CTL_OFF);
    if (threadIdx.x == 0)
        ctl[0] = arrive_last(a.counters + (int64_t)b * kCountersPerSeq + kvh * a.q_blocks + qb,
                             (uint32_t)n_chunks)
                     ? 1u
                     : 0u;
    __syncthreads();
    if (ctl[0] == 0) return;

    // Merge: o = sum_c w_c (o / l)_c / sum_c w_c, w_c = l_c 2^(m_c - m*),
    // kMergeBatch partials in flight, m* the running maximum.
    for (int idx = threadIdx.x; idx < n_el; idx += blockDim.x) {
        const int h = idx / D;
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
                } else {
                    ov[cb] = load_sc1(a.part_o + part_row(c) * D + idx);
                    mv[cb] = load_sc1(a.part_ml + (part_row(c) + h) * 2);
                    lv[cb] = load_sc1(a.part_ml + (part_row(c) + h) * 2 + 1);
                }
            }
            float mb = mstar;
#pragma unroll
            for (int cb = 0; cb < kMergeBatch; ++cb) mb = fmaxf(mb, mv[cb]);
            const float rr = __builtin_amdgcn_exp2f(mstar - mb);  // 0 on the first batch
            acc *= rr;
            lsum *= rr;
#pragma unroll
            for (int cb = 0; cb < kMergeBatch; ++cb) {
                const float w = lv[cb] * __builtin_amdgcn_exp2f(mv[cb] - mb);
                acc += ov[cb] * w;
                lsum += w;
            }
            mstar = mb;
        }
        store_out(idx, acc * (1.0f / lsum));
    }
}

}  // namespace hd

// ------------------------------------------------------------------ host side

bool hd_supported(int64_t head_dim) {
    return head_dim == 96 || head_dim == 160 || head_dim == 192 || head_dim == 224;
}

bool hd_tok_supported(int64_t head_dim, int64_t num_kv_heads) {
    return head_dim % 32 == 0 && head_dim >= 64 && head_dim <= 256 && num_kv_heads > 0;
}

int hd_waves(int64_t head_dim) {
    switch (head_dim) {
        case 64: return hd::Geo<2>::W;
        case 96: return hd::Geo<3>::W;
        case 128: return hd::Geo<4>::W;
        case 160: return hd::Geo<5>::W;
        case 192: return hd::Geo<6>::W;
        case 256: return hd::Geo<8>::W;
        default: return hd::Geo<7>::W;
    }
}

// Tiles a chunk may hold: a wave's page ids, two a tile, fill its 64 lanes.
static int64_t hd_max_chunk_tiles(int W) { return (int64_t)hd::kMaxTilesPerWave * W; }

static int64_t hd_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t max_chunks) {
    const int64_t rows = batch * max_chunks * num_q_heads;
    const int64_t o = rows * head_dim * 4;
    return counter_region_bytes(batch) + (o + 255) / 256 * 256 + rows * 2 * 4;
}

int hd_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_pages,
            int64_t total_tokens, int64_t max_tokens, int32_t tokens_per_split, bool token_pages,
            int32_t* out_chunk_tiles, int32_t* out_max_chunks, int32_t* out_waves, int64_t* out_workspace_bytes) {
    const bool ok = token_pages ? hd_tok_supported(head_dim, num_kv_heads) : hd_supported(head_dim);
    if (!ok || batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || max_pages <= 0)
        return kInvalidArgument;
    const int64_t q_blocks = (num_q_heads / num_kv_heads + hd::kHeads - 1) / hd::kHeads;
    const int W = hd_waves(head_dim);
    const int64_t cap_tokens = max_pages * 16;
    if (max_tokens < 0 || max_tokens > cap_tokens) max_tokens = cap_tokens;
    if (total_tokens < 0 || total_tokens > batch * max_tokens) total_tokens = batch * max_tokens;
    // The grid covers every tile block_table can address; the lengths steer
    // the chunk size: one CU's share (256 CUs on MI355X) of the tiles of all
    // (sequence, kv head, query block) units, so that no workgroup holds
    // more than its CU's share (a ragged batch's long sequences are split,
    // the short ones take one chunk each; the tiles of a batch: about
    // total / 32 + batch / 2, at most batch x the longest); but no less than
    // the longest sequence over the units a CU gets, up to 8 tiles a wave
    // (below that a workgroup's fixed costs, and the split's, outweigh the
    // balance: MI355X, B=128, Hq=16, Hkv=1, D=96, lengths in [128, 8192]:
    // 39.6 us with chunks of 3 tiles a wave against 34.2 with 11).
    const int64_t max_tiles = (cap_tokens + hd::kTile - 1) / hd::kTile;
    const int64_t longest = (max_tokens + hd::kTile - 1) / hd::kTile;
    int64_t chunk_tiles;
    if (tokens_per_split > 0) {
        chunk_tiles = (tokens_per_split + hd::kTile - 1) / hd::kTile;
    } else {
        int64_t tiles = total_tokens / hd::kTile + batch / 2;
        if (tiles > batch * longest) tiles = batch * longest;
        const int64_t share = (tiles * num_kv_heads * q_blocks + 255) / 256;
        int64_t per_unit = 256 / (batch * num_kv_heads * q_blocks);
        if (per_unit < 1) per_unit = 1;
        int64_t floor_tiles = (longest + per_unit - 1) / per_unit;
        if (floor_tiles > 8 * W) floor_tiles = 8 * W;
        chunk_tiles = share > floor_tiles ? share : floor_tiles;
        // The merging workgroup reads every chunk's partial of its block of
        // query heads, kMergeBatch chunks a round: at most 64 partial
        // elements a thread (MI355X, B=1, Hq=16, Hkv=1, D=128, L=16384: 64
        // chunks 36.3 us, 16 chunks 22.2).
        const int64_t nh = num_q_heads / num_kv_heads < hd::kHeads ? num_q_heads / num_kv_heads : hd::kHeads;
        const int64_t per_thread = (nh * head_dim + 64 * W - 1) / (64 * W);
        const int64_t most = 64 / per_thread > 1 ? 64 / per_thread : 1;
        const int64_t fewest_tiles = (longest + most - 1) / most;
        if (chunk_tiles < fewest_tiles) chunk_tiles = fewest_tiles;
        if (chunk_tiles > longest) chunk_tiles = longest;
    }
    const int64_t cap = hd_max_chunk_tiles(W);
    chunk_tiles = (chunk_tiles + W - 1) / W * W;
    if (chunk_tiles < W) chunk_tiles = W;
    if (chunk_tiles > cap) chunk_tiles = cap;
    int64_t max_chunks = (max_tiles + chunk_tiles - 1) / chunk_tiles;
    if (max_chunks > hd::kMaxChunks) {
        chunk_tiles = ((max_tiles + hd::kMaxChunks - 1) / hd::kMaxChunks + W - 1) / W * W;
        if (chunk_tiles > cap) return kInvalidArgument;
        max_chunks = (max_tiles + chunk_tiles - 1) / chunk_tiles;
    }
    if (max_chunks > 1 && num_kv_heads * q_blocks > kCountersPerSeq) return kInvalidArgument;
    *out_chunk_tiles = (int32_t)chunk_tiles;
    *out_max_chunks = (int32_t)max_chunks;
    *out_waves = W;
    *out_workspace_bytes = max_chunks > 1 ? hd_workspace_bytes(batch, num_q_heads, head_dim, max_chunks) : 0;
    return kOk;
}

namespace {
template <int G, bool TOK, bool ODD = false>
int launch_hd(dim3 grid, hipStream_t s, const hd::Args& a) {
    using L = hd::Geo<G>;
    static std::atomic<uint64_t> lds_raised{0};
    if (allow_full_lds(reinterpret_cast<const void*>(&hd::int4_decode_hd_kernel<G, TOK, ODD>), lds_raised) != kOk)
        return kLaunchError;
    hipLaunchKernelGGL((hd::int4_decode_hd_kernel<G, TOK, ODD>), grid, dim3(64 * L::W),
                       TOK ? L::LDS_BYTES_TOK : L::LDS_BYTES, s, a);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}
}  // namespace

int hd_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale, const void* v_scale,
              const int32_t* block_table, const int32_t* seq_lens, void* output, int32_t output_is_f32,
              void* workspace, int64_t workspace_bytes_avail, int64_t batch, int64_t num_q_heads,
              int64_t num_kv_heads, int64_t head_dim, int64_t max_pages, int64_t bt_cols, int32_t page_code,
              int64_t page_size, bool token_pages, float softmax_scale, int32_t chunk_tiles, int32_t max_chunks,
              int32_t waves, void* stream) {
    const bool ok = token_pages ? hd_tok_supported(head_dim, num_kv_heads) && page_size >= 1 && bt_cols > 0 &&
                                      bt_cols * page_size <= 0x3FFFFFFF
                                : hd_supported(head_dim);
    if (!ok || batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || max_pages <= 0)
        return kInvalidArgument;
    const int W = hd_waves(head_dim);
    if (waves != W || chunk_tiles <= 0 || chunk_tiles > hd_max_chunk_tiles(W) || max_chunks <= 0 ||
        max_chunks > hd::kMaxChunks)
        return kInvalidArgument;
    // the grid covers every token (every 16-token page) the table addresses
    if (token_pages ? (int64_t)chunk_tiles * max_chunks * hd::kTile < bt_cols * page_size
                    : (int64_t)chunk_tiles * max_chunks * 2 < max_pages)
        return kInvalidArgument;
    const int64_t g = num_q_heads / num_kv_heads;
    const int64_t q_blocks = (g + hd::kHeads - 1) / hd::kHeads;
    if (max_chunks > 1 && num_kv_heads * q_blocks > kCountersPerSeq) return kInvalidArgument;
    const int64_t units = batch * (int64_t)max_chunks;
    const int64_t nblocks = (units + 7) / 8 * 8 * num_kv_heads * q_blocks;  // whole groups of 8 units (XCD order)
    if (nblocks > 0x7FFFFFFF || num_q_heads > 0x7FFFFFFF) return kInvalidArgument;
    hd::Args a;
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
    a.n_kv_heads = (int)num_kv_heads;
    a.group = (int)g;
    a.q_blocks = (int)q_blocks;
    a.n_units = (int)units;
    a.seq_units = (int)batch;
    a.n_heads_blocks = (int)(num_kv_heads * q_blocks);
    a.max_chunks = max_chunks;
    a.chunk_tiles = chunk_tiles;
    a.max_pages = (int)max_pages;
    a.bt_cols = (int)bt_cols;
    a.page_code = page_code;
    a.page_size = (int)page_size;
    a.log2_scale = softmax_scale * 1.4426950408889634f;
    a.counters = nullptr;
    a.part_o = a.part_ml = nullptr;
    if (max_chunks > 1) {
        const int64_t need = hd_workspace_bytes(batch, num_q_heads, head_dim, max_chunks);
        if (workspace == nullptr || workspace_bytes_avail < need) return kWorkspaceTooSmall;
        uint8_t* const ws = (uint8_t*)workspace;
        const int64_t o = batch * max_chunks * num_q_heads * head_dim * 4;
        a.counters = (uint32_t*)ws;
        a.part_o = (float*)(ws + counter_region_bytes(batch));
        a.part_ml = (float*)(ws + counter_region_bytes(batch) + (o + 255) / 256 * 256);
    }
    const dim3 grid((unsigned)nblocks);
    hipStream_t s = (hipStream_t)stream;
    if (token_pages) {
        // Hkv x G odd: the scale shifts per token (G odd and Hkv odd)
        const bool odd = (head_dim / 32 * num_kv_heads) % 2 != 0;
        switch (head_dim) {
            case 64: return launch_hd<2, true>(grid, s, a);
            case 96: return odd ? launch_hd<3, true, true>(grid, s, a) : launch_hd<3, true>(grid, s, a);
            case 128: return launch_hd<4, true>(grid, s, a);
            case 160: return odd ? launch_hd<5, true, true>(grid, s, a) : launch_hd<5, true>(grid, s, a);
            case 192: return launch_hd<6, true>(grid, s, a);
            case 256: return launch_hd<8, true>(grid, s, a);
            default: return odd ? launch_hd<7, true, true>(grid, s, a) : launch_hd<7, true>(grid, s, a);
        }
    }
    switch (head_dim) {
        case 96: return launch_hd<3, false>(grid, s, a);
        case 160: return launch_hd<5, false>(grid, s, a);
        case 192: return launch_hd<6, false>(grid, s, a);
        default: return launch_hd<7, false>(grid, s, a);
    }
}

}  // namespace iris
