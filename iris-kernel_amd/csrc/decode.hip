// INT4 paged decode attention for gfx950: split-KV with the combine fused
// into the same launch.
//
// Replaces the TileLang kernel `_int4_paged_decode_attention`
// (src/iris_kernel/fused_attention.py:11-220 in Hunter2030ZeRo/Iris-Kernel)
// and computes the result of `torch_eager_int4_paged_decode_attention`
// (src/iris_kernel/torch_eager_attention.py:154-239): per sequence b and
// query head h, softmax(q . K^T * scale) . V over the first seq_lens[b]
// tokens of the paged INT4 cache, with kv head h / g.
//
// Schedule
// --------
// * Tile = 32 tokens = two 16-token pages.  A wavefront owns KVW kv heads
//   (KVW * g <= 16) and walks tiles; the 16 columns of every MFMA are the
//   (kv head, query head) pairs of those KVW heads, so at g = 4 the GQA tile
//   has no padding.
// * A workgroup of NW waves owns one (sequence, kv block, chunk of tiles);
//   wave w takes tiles w, w + NW, ... of the chunk (a fixed split keeps the
//   result bit-identical from run to run).  The waves' partial softmax
//   states are merged through LDS at the end.
// * Sequences longer than one chunk (flash-decoding split-KV; the reference
//   has no split): every chunk writes (m, l, o / l) to the workspace and
//   bumps an arrival counter of its (sequence, kv block); the workgroup that
//   arrives last merges all chunks of that pair, writes the output and
//   resets the counter to zero for the next call.  One launch, no combine
//   kernel.
// * Software pipeline per wave: while tile i is computed, the wave's next
//   tile is in flight -- K codes into registers (one dword per MFMA operand,
//   so no lane shuffles are needed), V codes and both scale tensors straight
//   into a double-buffered LDS stage (global_load_lds_dwordx4 / _dword).  V
//   is read back transposed with ds_read_b64_tr_b8 (one instruction gives
//   each lane byte m of 8 tokens).  The chunk's physical page ids are loaded
//   once per wave (two VGPRs) and picked with v_readlane.
//
// Arithmetic
// ----------
// Codes enter the MFMAs as fp16 subnormals: after flipping bit 3 a nibble
// is u = n + 8 in [0, 15], and the 16-bit pattern u (or 16u, for a high
// nibble left in place) is exactly u * 2^-24 (16u * 2^-24); the MFMA keeps
// subnormal inputs exact.  The +8 offset is removed with one per-group
// correction term, the 2^24 (and 16) factors are folded into the scales.
// QK: S^T[t][n] = sum_grp ks[t][grp] * (sum_{d in grp} k[t][d] * q[n][d]) with
//     v_mfma_f32_16x16x32_f16: A = K codes of 16 tokens x one 32-dim group,
//     B = q (fp16; high-nibble dims divided by 16, exactly), fp32 accumulate;
//     one MFMA per (group, kv head) with B masked to that head's columns,
//     then the fp32 tile is scaled per (token, group):
//     s += ks * (acc * 2^24 * c - 8 * c * sum_grp q).
// Softmax: fp32 online softmax in base 2 (c = scale * log2 e), running max
//     per column, per-lane partial sums.
// PV: O^T[d][n] += sum_t V[t][d] * (p[t][n] * vs[t][grp(d)]), A = V codes
//     transposed (rows = 16 dims of one group, k = 32 tokens), B = p * vs
//     rounded once to fp16.  The MFMA C layout of S^T is, register for
//     register, the B layout needed here, so p never moves between lanes.
//     The +8 offset: o = acc * 2^24 (2^20 for high nibbles) - 8 * sum_t B.
//
// MFMA operand layouts (v_mfma_f32_16x16x32_f16, lane l, i = 0..7 / 0..3):
//   A[l % 16][8 * (l / 16) + i],  B[8 * (l / 16) + i][l % 16],
//   C[4 * (l / 16) + i][l % 16].
// ds_read_b64_tr_b8 (per 16-lane group, lane i, byte k): the byte at offset
//   i % 8 of the 8-byte row addressed by lane 2k + i / 8.
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "common.h"
#include "decode_any.h"
#include "decode_hd.h"
#include "decode_mqa.h"
#include "decode_pages.h"
#include "decode_stream.h"
#include "iris_hip.h"

namespace iris {

constexpr int kTile = 32;
constexpr int kPageSize = 16;
constexpr int kMaxChunkTiles = 64;  // a chunk's 2 * 64 page ids fill two VGPRs
#ifndef IRIS_STREAM_AUX
#define IRIS_STREAM_AUX 0
#endif
// Cache-policy bits of the streaming K / V / scale loads.
constexpr int kStreamAux = IRIS_STREAM_AUX;

typedef int int2v_t __attribute__((ext_vector_type(2)));
#define IRIS_LDS __attribute__((address_space(3)))
#define IRIS_GLOBAL __attribute__((address_space(1)))

struct DecodeArgs {
    const half_t* q;
    const uint8_t* k_data;
    const uint8_t* v_data;
    const half_t* k_scale;
    const half_t* v_scale;
    const int32_t* block_table;
    const int32_t* seq_lens;
    void* out;
    uint32_t* counters;  // counter kvb of sequence b at b * kCountersPerSeq + kvb; zero between calls
    float* ws_o;         // [B][max_chunks][n_kv_blocks][16 * D]  o / l, MFMA C order
    float* ws_ml;        // [B][max_chunks][n_kv_blocks][16][2]   (m, l), base-2 logits
    int out_f32;
    int batch, n_q_heads, n_kv_heads, group;  // group = Hq / Hkv
    int max_pages;            // 16-token pages a block-table row addresses
    int bt_cols, page_shift;  // block-table columns; the page code of virtual_page (page_size = 16 m)
    // kv blocks: (KVW kv heads) x (q_blocks blocks of 16 of a kv head's
    // query heads; q_blocks > 1 only for group > 16, with KVW = 1)
    int n_kv_blocks, q_blocks, max_chunks, chunk_tiles;
    float log2_scale;  // softmax_scale * log2(e)
};

// K operand: eight codes (one dword, low nibble first) -> fp16 subnormals
// in the order d0, d4, 16*d1, 16*d5, d2, d6, 16*d3, 16*d7 (units of 2^-24,
// codes offset by +8).  Each half is one v_bitop3 ((x ^ c) & m).
__device__ __forceinline__ half8_t k_operand(uint32_t x) {
    const uint32_t y = x >> 8;
    const u32x4_t r = {(x ^ 0x00080008u) & 0x000F000Fu, (x ^ 0x00800080u) & 0x00F000F0u,
                       (y ^ 0x00080008u) & 0x000F000Fu, (y ^ 0x00800080u) & 0x00F000F0u};
    return __builtin_bit_cast(half8_t, r);
}

// V operands from the 8 bytes of one transposed read (byte k' = token k'):
// lo = low nibbles (even dim), hi = 16 * high nibbles (odd dim), both in the
// slot order k' = 0, 2, 1, 3, 4, 6, 5, 7 (bytes 0 and 2 of a dword share a
// mask, so no byte shuffles are needed).
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
// Byte (token) index k' held by each slot of the V operands.
constexpr int kVSlotByte[8] = {0, 2, 1, 3, 4, 6, 5, 7};

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// v_permlane32_swap / v_permlane16_swap as opaque instructions.  (Through
// the builtins, the compiler folds the two results of a swap whose operands
// are the same value into one, which breaks the reductions below.)  The
// s_nop covers the VALU-write -> permlane-read hazard.
//   swap32: a[32 + i] <-> b[i]            (i = 0..31)
//   swap16: a[16 * (2r + 1) + i] <-> b[16 * 2r + i]   (r = 0, 1; i = 0..15)
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// max / sum over the four 16-lane rows (lanes n, n+16, n+32, n+48).
__device__ __forceinline__ float row_max4(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    swap32(a, b);  // a = low half on both halves, b = high half on both halves
    uint32_t c = __builtin_bit_cast(uint32_t, __builtin_elementwise_maximum(as_f32(a), as_f32(b)));
    uint32_t d = c;
    swap16(c, d);  // c = even rows on both rows of a pair, d = odd rows
    return __builtin_elementwise_maximum(as_f32(c), as_f32(d));
}

__device__ __forceinline__ float row_sum4(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    swap32(a, b);
    uint32_t c = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b));
    uint32_t d = c;
    swap16(c, d);
    return __builtin_bit_cast(float, c) + __builtin_bit_cast(float, d);
}

// 4x4 dword transpose across the four 16-lane rows: on return, register g
// of a lane in row q holds what register q of the same lane position in row
// g held.
__device__ __forceinline__ void transpose_rows4(u32x4_t& x) {
    uint32_t x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
    swap32(x0, x2);
    swap32(x1, x3);
    swap16(x0, x1);
    swap16(x2, x3);
    x = u32x4_t{x0, x1, x2, x3};
}

// ---- VALU tile: v_dot2c_f32_f16 with DPP row broadcasts (no MFMA)
//
// The alternative to the MFMA tile, selected per launch (the
// IRIS_DECODE_VALU_TILE bit of waves_per_block) for the layouts KVW * g = 16 with g = 4 or 16.  Every dot product
// is a chain of v_dot2c_f32_f16 whose first operand is broadcast from one
// lane of the 16-lane row (DPP row_newbcast), so each fp16 pair is unpacked
// or computed once and no operand is replicated in registers:
//   QK: the K codes stay in the MFMA A layout (lane = token n of the
//       16-token half, row jq = 8-dim chunk of each group); the q pairs of
//       the row's chunk sit one per lane (lane 4b + p: pair p of column
//       4a + b, register a), and the partial sums of the four chunks are
//       added across the rows with a 4 x 4 transpose;
//   softmax / PV: lane (n, row rho) holds token n (and 16 + n) of columns
//       col(rho, w), w = 0..3; PV broadcasts p * v_scale of token pair
//       (t, t + 16) from lane t to the 16 lanes of the row, each of which
//       accumulates the two dims of one V byte.
// Instruction counts per 32-token tile and kv head equal the minimum g * D / 4
// dot2 per product (QK and PV each) plus the unpacking and the reductions.

// QK of column quad A over this lane's code pairs kp (the four pairs of one
// k_operand dword): acc[b] = offset term of column 4A + b (broadcast from lane
// 4A + b of qc) + sum_p kp[p] . (q pair broadcast from lane 4b + p of qv).
// A VGPR a VALU instruction wrote is read through DPP two wait states later
// (the leading s_nop).
template <int A>
__device__ __forceinline__ void qk_valu(float (&acc)[4], uint32_t qv, uint32_t qc, const u32x4_t kp) {
    asm volatile(
        "s_nop 1\n\t"
        "v_mov_b32_dpp %0, %5 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b32_dpp %1, %5 row_newbcast:%11 row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b32_dpp %2, %5 row_newbcast:%12 row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b32_dpp %3, %5 row_newbcast:%13 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %4, %6 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %1, %4, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %2, %4, %6 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %3, %4, %6 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %4, %7 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %1, %4, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %2, %4, %7 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %3, %4, %7 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %4, %8 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %1, %4, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %2, %4, %8 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %3, %4, %8 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %4, %9 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %1, %4, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %2, %4, %9 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %3, %4, %9 row_newbcast:15 row_mask:0xf bank_mask:0xf"
        : "=&v"(acc[0]), "=&v"(acc[1]), "=&v"(acc[2]), "=&v"(acc[3])
        : "v"(qv), "v"(qc), "v"(kp[0]), "v"(kp[1]), "v"(kp[2]), "v"(kp[3]), "n"(4 * A), "n"(4 * A + 1),
          "n"(4 * A + 2), "n"(4 * A + 3));
}
__device__ __forceinline__ void qk_valu_quad(int a, float (&acc)[4], uint32_t qv, uint32_t qc, const u32x4_t kp) {
    switch (a) {  // a is a constant in every unrolled use
        case 0: qk_valu<0>(acc, qv, qc, kp); break;
        case 1: qk_valu<1>(acc, qv, qc, kp); break;
        case 2: qk_valu<2>(acc, qv, qc, kp); break;
        default: qk_valu<3>(acc, qv, qc, kp); break;
    }
}

// PV of token pairs T0 .. T0 + 3: o[w][e] += vl / vh[tt] . (p pair of column
// w broadcast from lane T0 + tt), e = 0 the byte's low-nibble dim, 1 its
// high-nibble dim (16x codes).
template <int T0>
__device__ __forceinline__ void pv_valu(float (&o)[4][2], const uint32_t (&pv)[4], const uint32_t (&vl)[4],
                                        const uint32_t (&vh)[4]) {
    asm volatile(
        "s_nop 1\n\t"
        "v_dot2c_f32_f16_dpp %0, %8, %12 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %1, %8, %16 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %2, %9, %12 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %3, %9, %16 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %4, %10, %12 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %5, %10, %16 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %6, %11, %12 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %7, %11, %16 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %8, %13 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %1, %8, %17 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %2, %9, %13 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %3, %9, %17 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %4, %10, %13 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %5, %10, %17 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %6, %11, %13 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %7, %11, %17 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %8, %14 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %1, %8, %18 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %2, %9, %14 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %3, %9, %18 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %4, %10, %14 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %5, %10, %18 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %6, %11, %14 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %7, %11, %18 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %8, %15 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %1, %8, %19 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %2, %9, %15 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %3, %9, %19 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %4, %10, %15 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %5, %10, %19 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %6, %11, %15 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %7, %11, %19 row_newbcast:%23 row_mask:0xf bank_mask:0xf"
        : "+v"(o[0][0]), "+v"(o[0][1]), "+v"(o[1][0]), "+v"(o[1][1]), "+v"(o[2][0]), "+v"(o[2][1]),
          "+v"(o[3][0]), "+v"(o[3][1])
        : "v"(pv[0]), "v"(pv[1]), "v"(pv[2]), "v"(pv[3]), "v"(vl[0]), "v"(vl[1]), "v"(vl[2]), "v"(vl[3]),
          "v"(vh[0]), "v"(vh[1]), "v"(vh[2]), "v"(vh[3]), "n"(T0), "n"(T0 + 1), "n"(T0 + 2), "n"(T0 + 3));
}

// Four transposed 8-byte LDS reads at addr + OFF + k * STRIDE (k = 0..3) that
// wait for their own results (as lds_tr8).
template <int OFF, int STRIDE>
__device__ __forceinline__ void lds_tr8_x4(uint32_t addr, int2v_t (&w)[4]) {
    static_assert(OFF >= 0 && OFF + 3 * STRIDE < 65536, "ds offset range");
    asm volatile(
        "ds_read_b64_tr_b8 %0, %4 offset:%5\n\t"
        "ds_read_b64_tr_b8 %1, %4 offset:%6\n\t"
        "ds_read_b64_tr_b8 %2, %4 offset:%7\n\t"
        "ds_read_b64_tr_b8 %3, %4 offset:%8\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
        : "v"(addr), "n"(OFF), "n"(OFF + STRIDE), "n"(OFF + 2 * STRIDE), "n"(OFF + 3 * STRIDE)
        : "memory");
}

// Workgroups are dispatched round-robin over the 8 XCDs; renumber them so
// that consecutive logical ids (the kv blocks and chunks of one sequence,
// which share scale lines and block-table rows) run on the same XCD and L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    constexpr int kXcds = 8;
    if (nblocks % kXcds != 0) return bid;
    return (bid % kXcds) * (nblocks / kXcds) + bid / kXcds;
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt at their maxima: 0x0F70 on gfx9),
// as the builtin: the compiler knows every load has landed after it, so it
// adds no wait of its own before the first use of a loaded register.
__device__ __forceinline__ void wait_vmem_all() {
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// An opaque copy of a per-lane value.  Used on loop-invariant address bases
// inside the tile loop, so the compiler folds each per-load constant into
// the instruction's offset field instead of keeping one precomputed
// base + constant VGPR per load alive across the loop.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Buffer resource over one page of a cache tensor (raw, stride 0, 32-bit
// data format: word 3 = 0x00020000 on gfx9-family parts).  Loads address
// base + voffset + soffset + imm, so a per-lane offset is computed once and
// every load of a page adds only constants; offsets past `bytes` read 0.
// Every caller passes wave-uniform values; reading them from the first lane
// says so to the compiler, which otherwise may keep a descriptor word in a
// VGPR and wrap each load in a loop over the distinct values of the lanes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0, (int)n,
                                             0x00020000);
}

// N transposed 8-byte LDS reads (ds_read_b64_tr_b8) that wait for their own
// results.  Written as assembly because the compiler cannot tell these reads
// from the direct-to-LDS loads of the next tile, still in flight into the
// other stage buffer, and would wait for those too; the data read here has
// landed (the tile loop's vmcnt(0) precedes it).
// Each reads addr[k] + OFF (OFF an immediate: the stage buffer's offset).
template <int N, int OFF>
__device__ __forceinline__ void lds_tr8(const uint32_t (&addr)[N], int2v_t (&w)[N]) {
    static_assert(N == 1 || N == 2 || N == 4, "one, two or four reads");
    static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
    if constexpr (N == 4) {
        asm volatile(
            "ds_read_b64_tr_b8 %0, %4 offset:%8\n\t"
            "ds_read_b64_tr_b8 %1, %5 offset:%8\n\t"
            "ds_read_b64_tr_b8 %2, %6 offset:%8\n\t"
            "ds_read_b64_tr_b8 %3, %7 offset:%8\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
            : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "n"(OFF)
            : "memory");
    } else if constexpr (N == 2) {
        asm volatile(
            "ds_read_b64_tr_b8 %0, %2 offset:%4\n\t"
            "ds_read_b64_tr_b8 %1, %3 offset:%4\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w[0]), "=&v"(w[1])
            : "v"(addr[0]), "v"(addr[1]), "n"(OFF)
            : "memory");
    } else {
        asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(w[0])
                     : "v"(addr[0]), "n"(OFF)
                     : "memory");
    }
}

// Head dimension of element `idx` of a 16 x D tile stored in MFMA C order:
// idx = ((grp * 2 + e) * 4 + i) * 64 + lane, lane = 16 * jq + column, and
// element (grp, e, i) of lane (column, jq) is dim grp * 32 + 2 * (4 jq + i) + e.
__device__ __forceinline__ int c_order_dim(int idx) {
    const int reg = idx >> 6, jq = (idx >> 4) & 3;
    return (reg >> 3) * 32 + 2 * (4 * jq + (reg & 3)) + ((reg >> 2) & 1);
}

template <int D, int KVW>
struct DecodeLayout {
    static constexpr int G = D / 32;          // scale groups per head
    static constexpr int HB = D / 2;          // packed bytes per (token, head)
    static constexpr int SEG = KVW * HB;      // V bytes per token for the KVW heads
    static constexpr int C = SEG / 16;        // 16-byte chunks per token
    static constexpr int SSEG = KVW * G * 2;  // scale bytes per token
    static constexpr int VBUF = kTile * SEG;
    static constexpr int SBUF = kTile * SSEG;
    static constexpr int BUF = VBUF + 2 * SBUF;
    static constexpr int STAGE = 2 * BUF;     // double buffered
    static constexpr int MERGE = (16 * D + 32) * 4;  // o in C order + (m, l) per column
    static constexpr int WAVE_LDS = ((STAGE > MERGE ? STAGE : MERGE) + 15) / 16 * 16;
    static constexpr int NV = kTile * C / 64;          // 16-byte V loads per lane per tile
    static constexpr int SDW = SBUF / 4;               // scale dwords per tensor per tile
    static constexpr int NS = (SDW + 63) / 64;         // 4-byte scale loads per lane per tile
    static constexpr int KREGS = KVW * G;              // K dwords per lane per 16-token half
    // Loads that cover both pages of a tile at once (more than 16 tokens a
    // load): their lane offsets are kept in NVO / NSO registers.
    static constexpr int NVO = 64 / C > 16 ? NV : 1;
    static constexpr int NSO = 64 / (SSEG / 4) > 16 ? NS : 1;
};

// The kernel body; VALU selects the v_dot2c tile instead of the MFMA tile
// (the loads, the split and the merges are the same).
template <int D, int KVW, bool VALU>
__device__ __forceinline__ void decode_body(const DecodeArgs& a) {
    using L = DecodeLayout<D, KVW>;
    static_assert(!VALU || ((KVW == 4 || KVW == 1) && D != 256), "VALU tile: g = 4 (KVW 4) or g = 16 (KVW 1)");
    constexpr int G = L::G, HB = L::HB, C = L::C, SSEG = L::SSEG;
    static_assert(C >= 2 && (C & (C - 1)) == 0, "chunks per token must be a power of two >= 2");
    extern __shared__ __align__(16) uint8_t smem[];

    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;   // MFMA column (B/C) or row (A)
    const int jq = lane >> 4;  // MFMA k-chunk (A/B) or row quad (C)

    const int wg = xcd_remap(blockIdx.x, gridDim.x);
    const int kvb = wg % a.n_kv_blocks;
    const int rest = wg / a.n_kv_blocks;
    const int chunk = rest % a.max_chunks;
    const int b = rest / a.max_chunks;
    const int kv0 = (kvb / a.q_blocks) * KVW;
    const int g = a.group;
    const int qoff = (kvb % a.q_blocks) * 16;  // first query head of the block (within the kv head)
    const int hkv = a.n_kv_heads;
    const int t_begin = chunk * a.chunk_tiles;
    const int p0 = 2 * t_begin;  // first logical page of the chunk

    // ---- loads that depend on nothing else go first: the chunk's page ids
    // (lane i holds logical pages p0 + i and p0 + 64 + i) and q.
    const int32_t* bt = a.block_table + (int64_t)b * a.bt_cols;
    int pid0 = 0, pid1 = 0;
    if (p0 + lane < a.max_pages) pid0 = virtual_page(bt, p0 + lane, a.page_shift);
    if (p0 + 64 + lane < a.max_pages) pid1 = virtual_page(bt, p0 + 64 + lane, a.page_shift);

    // Column n of the MFMA tiles = (kv head kv0 + n / g, query head n % g),
    // or, for g > 16, query head qoff + n of kv head kv0.
    const int n_cols = a.q_blocks > 1 ? min(16, g - qoff) : KVW * g;
    const bool col_valid = n < n_cols;
    const int col_kv = col_valid && a.q_blocks == 1 ? n / g : 0;
    const int hq = kv0 * g + qoff + n;
    u32x4_t qraw[G];
#pragma unroll
    for (int grp = 0; grp < G; ++grp) {
        qraw[grp] = u32x4_t{0, 0, 0, 0};
        if (col_valid)
            qraw[grp] = *reinterpret_cast<const u32x4_t*>(a.q + ((int64_t)b * a.n_q_heads + hq) * D + grp * 32 + jq * 8);
    }

    const int seq_len = a.seq_lens[b];
    const int n_tiles = (seq_len + kTile - 1) / kTile;
    if (t_begin >= n_tiles) return;  // uniform over the workgroup
    const int t_end = min(t_begin + a.chunk_tiles, n_tiles);
    const int n_chunks = (n_tiles + a.chunk_tiles - 1) / a.chunk_tiles;
    const int last_lp = (seq_len + kPageSize - 1) / kPageSize - 1;
    const int64_t page_data = (int64_t)kPageSize * hkv * HB;     // bytes per page, K or V
    const int64_t page_scale = (int64_t)kPageSize * hkv * G * 2;  // bytes per page, one scale tensor

    // Physical page of logical page lp (clamped to the sequence's last page;
    // tokens past seq_len are masked).  p0 <= lp' < p0 + 2 * chunk_tiles.
    // Call it in uniform control flow only: the lane it reads belongs to a
    // VGPR select, which lanes masked off by a divergent branch leave stale.
    auto page_of = [&](int lp) -> int64_t {
        const int rel = min(lp, last_lp) - p0;
        return (int64_t)__builtin_amdgcn_readlane(rel < 64 ? pid0 : pid1, rel & 63);
    };

    const float c = a.log2_scale;
    // Scores are kept in MFMA units (s' = s / c24); c24 = scale * log2(e) *
    // 2^24 converts them to base-2 logits inside the exponent.
    const float c24 = c * 16777216.0f;
    // Lazy rescaling: the running max moves only when a column's max grows
    // by more than 2 (base 2), so p <= 4 and p * v_scale stays inside fp16.
    const float lazy = 2.0f / c24;

    // Per-lane, tile-invariant parts of the load addresses.
    // K (registers): lane (t, jq) of 16-token half r needs, per (kv j, group),
    // the dword of dims grp * 32 + 8 jq .. + 7 of token t (the A operand).
    // D = 128: one 16-byte load per kv head gives lane (t, jq) all of group
    // jq, and a 4 x 4 dword transpose across the four 16-lane rows turns that
    // into dword jq of every group (16 separate 4-byte loads would cost four
    // times the cache-line lookups).  D = 64: two 4-byte loads per head.
    const uint32_t k_off = (uint32_t)(n * hkv + kv0) * HB + jq * (D == 128 ? 16 : 4);
    // V (LDS, 16-byte chunks): 1 KB per load = TPI tokens of one page when
    // C <= 16; chunk p of token tau lands at LDS position p and is fetched
    // from chunk p ^ f(tau), f(tau) = ((tau & 3) | ((tau >> 4) << 2)) & (C - 1).
    constexpr int TPI = 64 / C;
    const int v_tok = lane / C, v_p = lane % C;
    uint32_t v_lane[2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
        v_lane[r] = (uint32_t)(v_tok * hkv + kv0) * HB +
                    (uint32_t)((v_p ^ (((v_tok & 3) | (r << 2)) & (C - 1))) * 16);
    // Scales (LDS, 4-byte loads): dword w of token tau's KVW * G scales.
    constexpr int SW = SSEG / 4;        // dwords per token
    constexpr int STPI = 64 / SW;       // tokens per load
    const int s_tok = lane / SW, s_w = lane % SW;
    const uint32_t s_lane = ((uint32_t)(s_tok * hkv + kv0) * G + 2 * s_w) * 2;
    // Lane offsets inside a page of the loads that cover both pages of a
    // tile in one instruction (V when TPI > 16, scales when STPI > 16):
    // V chunk p of token tau at row (tau & 15) * hkv + kv0, chunk p ^ f;
    // scale dword w of token tau.
    // (Literal bounds: with a template-dependent bound the host pass of
    // hipcc dropped the <64, 1> kernel's instantiation without a diagnostic.)
    static_assert(L::NVO <= 1 && L::NSO <= 2, "lane-offset registers");
    uint32_t v_loff[1], s_loff[2];
#pragma unroll
    for (int it = 0; it < L::NVO; ++it) {
        const int qi = it * 64 + lane;
        const int tau = qi / C, p = qi % C;
        const int f = ((tau & 3) | ((tau >> 4) << 2)) & (C - 1);
        v_loff[it] = (uint32_t)(((tau & 15) * hkv + kv0) * HB + (p ^ f) * 16);
    }
#pragma unroll
    for (int it = 0; it < L::NSO; ++it) {
        const int qi = it * 64 + lane;
        const int tau = qi / SW, w = qi % SW;
        s_loff[it] = (uint32_t)((((tau & 15) * hkv + kv0) * G + 2 * w) * 2);
    }
    // The same as addresses from the tensor bases: a load's lane address is
    // then (the lane's page) * (page bytes) + base, one v_mad_u64_u32 with
    // no per-page 64-bit scalar arithmetic.
    uint64_t v_lbase[1], ks_lbase[2], vs_lbase[2];
#pragma unroll
    for (int it = 0; it < L::NVO; ++it) v_lbase[it] = (uint64_t)(uintptr_t)a.v_data + v_loff[it];
#pragma unroll
    for (int it = 0; it < L::NSO; ++it) {
        ks_lbase[it] = (uint64_t)(uintptr_t)a.k_scale + s_loff[it];
        vs_lbase[it] = (uint64_t)(uintptr_t)a.v_scale + s_loff[it];
    }
    // tr8 reads: supplier row s = n reads token tau(jq, k = n >> 1), half
    // n & 1; the chunk of (kv j, group grp) sits at position (j G + grp) ^ f.
    const int trk = n >> 1;
    const int tr_tok = 4 * jq + (trk & 3) + 16 * (trk >> 2);
    const uint32_t tr_base = (uint32_t)tr_tok * (C * 16) + 8 * (n & 1) + ((uint32_t)(trk & (C - 1)) << 4);
    // Byte offset of this lane's scales in a stage's scale block: token
    // 4 jq (+ 16 r + i), kv head col_kv.
    const uint32_t s_col = (uint32_t)((4 * jq * KVW + col_kv) * G) * 2;

    uint8_t* const stage = smem + wave * L::WAVE_LDS;

    // ---- loads of one tile: K codes into registers `kw` ...
    // (Lane address = page id * page bytes + this lane's address from the
    // tensor base: one v_mad_u64_u32 per page, the per-load constants in the
    // loads' offset fields.)
    const uint64_t k_lbase = (uint64_t)(uintptr_t)a.k_data + k_off;
    // D = 64, one kv head a wave: one 16-byte load a lane covers the tile.
    // Lane (n, jq) reads row n of page jq >> 1, bytes 16 (jq & 1) .. + 15
    // (group jq & 1); a 4 x 4 transpose across the rows at use turns that
    // into dword jq of every (page, group), the MFMA A layout.
    const uint64_t k64_lbase = (uint64_t)(uintptr_t)a.k_data + (uint32_t)(n * hkv + kv0) * HB + 16 * (jq & 1);
    auto issue_k = [&](int tile, uint32_t (&kw)[2][L::KREGS]) {
        if constexpr (D == 64 && KVW == 1) {
            // (both page ids first, in uniform control flow: page_of reads a
            // lane of a VGPR select, which a divergent branch would leave
            // unwritten in its inactive lanes)
            const uint32_t pa = (uint32_t)page_of(2 * tile), pb = (uint32_t)page_of(2 * tile + 1);
            const uint32_t pk = (jq >> 1) ? pb : pa;
            const u32x4_t x =
                *reinterpret_cast<const IRIS_GLOBAL u32x4_t*>((uint64_t)pk * (uint32_t)page_data + k64_lbase);
            kw[0][0] = x[0];
            kw[0][1] = x[1];
            kw[1][0] = x[2];
            kw[1][1] = x[3];
            return;
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            // (a global-address-space pointer: global_load, not flat_load, whose
            // pending count would also hold back the tile's LDS reads)
            const IRIS_GLOBAL uint8_t* const kp = reinterpret_cast<const IRIS_GLOBAL uint8_t*>(
                (uint64_t)(uint32_t)page_of(2 * tile + r) * (uint32_t)page_data + k_lbase);
#pragma unroll
            for (int j = 0; j < KVW; ++j) {
                if constexpr (D == 128) {
                    const u32x4_t x = *reinterpret_cast<const IRIS_GLOBAL u32x4_t*>(kp + j * HB);
#pragma unroll
                    for (int q = 0; q < 4; ++q) kw[r][j * G + q] = x[q];
                } else {
#pragma unroll
                    for (int grp = 0; grp < G; ++grp)
                        kw[r][j * G + grp] = *reinterpret_cast<const IRIS_GLOBAL uint32_t*>(kp + j * HB + grp * 16);
                }
            }
        }
    };
    // ... and V codes + both scale tensors straight into stage buffer `buf`.
    auto issue_v = [&](int tile, int buf) {
        const int64_t pg[2] = {page_of(2 * tile), page_of(2 * tile + 1)};
        uint8_t* const vb = stage + buf * L::BUF;
        if constexpr (TPI <= 16) {
            // one page per load: per-page resources, the token offset in soffset
            const __amdgpu_buffer_rsrc_t vr[2] = {page_rsrc(a.v_data + pg[0] * page_data, (uint32_t)page_data),
                                                  page_rsrc(a.v_data + pg[1] * page_data, (uint32_t)page_data)};
#pragma unroll
            for (int it = 0; it < L::NV; ++it) {
                const int tau0 = it * TPI, r = tau0 >> 4;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vr[r], (IRIS_LDS void*)(vb + it * 1024), 16, v_lane[r],
                                                         (tau0 & 15) * hkv * HB, 0, kStreamAux);
            }
        } else {
            // lanes of both pages in one load: the lane's page id (one of the
            // two, uniform) times the page size, plus its address from the base
            const uint32_t p0 = (uint32_t)pg[0], p1 = (uint32_t)pg[1];
#pragma unroll
            for (int it = 0; it < L::NV; ++it) {
                const int tau = (it * 64 + lane) / C;
                const uint64_t ad = (uint64_t)((tau >> 4) ? p1 : p0) * (uint32_t)page_data + v_lbase[it];
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(ad), (IRIS_LDS void*)(vb + it * 1024),
                                                 16, 0, kStreamAux);
            }
        }
        if constexpr (STPI <= 16) {
            const uint8_t* const ksb = reinterpret_cast<const uint8_t*>(a.k_scale);
            const uint8_t* const vsb = reinterpret_cast<const uint8_t*>(a.v_scale);
            const __amdgpu_buffer_rsrc_t kr[2] = {page_rsrc(ksb + pg[0] * page_scale, (uint32_t)page_scale),
                                                  page_rsrc(ksb + pg[1] * page_scale, (uint32_t)page_scale)};
            const __amdgpu_buffer_rsrc_t vr[2] = {page_rsrc(vsb + pg[0] * page_scale, (uint32_t)page_scale),
                                                  page_rsrc(vsb + pg[1] * page_scale, (uint32_t)page_scale)};
#pragma unroll
            for (int it = 0; it < L::NS; ++it) {
                const int tau0 = it * STPI, r = tau0 >> 4;
                const int soff = (tau0 & 15) * hkv * G * 2;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(kr[r], (IRIS_LDS void*)(vb + L::VBUF + it * 256), 4, s_lane,
                                                         soff, 0, kStreamAux);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vr[r], (IRIS_LDS void*)(vb + L::VBUF + L::SBUF + it * 256), 4,
                                                         s_lane, soff, 0, kStreamAux);
            }
        } else if (D == 64 && KVW == 1 && hkv == 1) {
            // One kv head in the cache: a page's scales of one tensor are 64
            // contiguous bytes, so lanes 0-15 bring both tensors of both pages
            // in one 16-byte-a-lane load (lane l: tensor l >> 3, page
            // (l >> 2) & 1, piece l & 3), landing as the two scale blocks.
            if (lane < 16) {
                const uint64_t pb = (uint64_t)(uint32_t)(((lane >> 2) & 1) ? pg[1] : pg[0]) * (uint32_t)page_scale;
                const uint64_t tb = (uint64_t)(uintptr_t)((lane >> 3) ? (const void*)a.v_scale : (const void*)a.k_scale);
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(tb + pb + 16 * (lane & 3)),
                                                 (IRIS_LDS void*)(vb + L::VBUF), 16, 0, kStreamAux);
            }
        } else {
            const uint32_t p0 = (uint32_t)pg[0], p1 = (uint32_t)pg[1];
#pragma unroll
            for (int it = 0; it < L::NS; ++it) {
                const int qi = it * 64 + lane;
                if (L::SDW % 64 == 0 || qi < L::SDW) {
                    const uint64_t po = (uint64_t)(((qi / SW) >> 4) ? p1 : p0) * (uint32_t)page_scale;
                    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(po + ks_lbase[it]),
                                                     (IRIS_LDS void*)(vb + L::VBUF + it * 256), 4, 0, kStreamAux);
                    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(po + vs_lbase[it]),
                                                     (IRIS_LDS void*)(vb + L::VBUF + L::SBUF + it * 256), 4, 0, kStreamAux);
                }
            }
        }
    };

    // ---- the first tile's loads fly while q is turned into MFMA operands.
    uint32_t kw[2][L::KREGS];
    int tile = t_begin + wave;
    if (tile < t_end) {
        issue_v(tile, 0);
        issue_k(tile, kw);
    }

    // q as the QK B operand (k order of k_operand; high-nibble dims / 16),
    // one copy per kv head with the other heads' columns zeroed.  The +8
    // code offset contributes 8 * 2^-24 * sum_grp q to each group's MFMA
    // result; the accumulator starts at minus that.
    half8_t qm[KVW][G];
    float qinit[G];
#pragma unroll
    for (int grp = 0; grp < G; ++grp) {
        const u32x4_t w = qraw[grp];
        const half2_t w0 = as_half2(w[0]), w1 = as_half2(w[1]);
        const half2_t w2 = as_half2(w[2]), w3 = as_half2(w[3]);
        const half_t s16 = (half_t)0.0625f;
        const half8_t qf = {w0.x, w2.x, w0.y * s16, w2.y * s16, w1.x, w3.x, w1.y * s16, w3.y * s16};
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) part += (float)qf[i] * ((i & 2) ? 16.0f : 1.0f);
        qinit[grp] = -8.0f * 5.9604644775390625e-08f * row_sum4(part);
#pragma unroll
        for (int j = 0; j < KVW; ++j) {
            const half8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
            qm[j][grp] = (col_valid && col_kv == j) ? qf : z;
        }
    }

    float m_run = -INFINITY;  // MFMA units
    float l_part = 0.0f;
    float s_lo = INFINITY;  // lowest valid score seen
    float ps[G];
    float4_t o[G][2];
#pragma unroll
    for (int grp = 0; grp < G; ++grp) {
        ps[grp] = 0.0f;
        o[grp][0] = o[grp][1] = float4_t{0, 0, 0, 0};
    }

    // ---- VALU tile operands and state (VALU only).  The 16 columns are
    // 4a + b; with KVW = 4 (g = 4) column 4a + b is query head b of kv head
    // kv0 + a, with KVW = 1 (g = 16) query head 4a + b of kv head kv0.
    //   qv[a][grp]: lane (n, row jq) holds q pair n & 3 (k_operand order) of
    //     column 4a + (n >> 2), dims grp * 32 + 8 jq .. + 7;
    //   qc[grp]: the +8 code offset term of column n over the same dims,
    //     -8 * 2^-24 * sum q (the chain's start; the rows' partial sums add
    //     up to qinit).
    //   After QK, lane (n, row rho) holds tokens n and 16 + n of the columns
    //   col(rho, w) = 4 rho + w (KVW = 4: the row is a kv head) or 4 w + rho
    //   (KVW = 1), w = 0..3; softmax and PV keep that layout.
    uint32_t qv[4][G], qc[G];
    float vm[4], vl[4], vlo[4], vps[G][4], vo[G][4][2];
    if constexpr (VALU) {
        const half_t s16 = (half_t)0.0625f;
#pragma unroll
        for (int grp = 0; grp < G; ++grp) {
            const u32x4_t w = qraw[grp];
            const half2_t w0 = as_half2(w[0]), w1 = as_half2(w[1]), w2 = as_half2(w[2]), w3 = as_half2(w[3]);
            const float part = (float)w0.x + (float)w2.x + (float)(w0.y * s16) * 16.0f + (float)(w2.y * s16) * 16.0f +
                               (float)w1.x + (float)w3.x + (float)(w1.y * s16) * 16.0f + (float)(w3.y * s16) * 16.0f;
            qc[grp] = as_u32(-8.0f * 5.9604644775390625e-08f * part);
#pragma unroll
            for (int qa = 0; qa < 4; ++qa) {
                const int hqa = kv0 * g + 4 * qa + (n >> 2);
                const u32x4_t x = *reinterpret_cast<const u32x4_t*>(a.q + ((int64_t)b * a.n_q_heads + hqa) * D + grp * 32 + jq * 8);
                const half2_t x0 = as_half2(x[0]), x1 = as_half2(x[1]), x2 = as_half2(x[2]), x3 = as_half2(x[3]);
                const half2_t pr[4] = {half2_t{x0.x, x2.x}, half2_t{x0.y * s16, x2.y * s16}, half2_t{x1.x, x3.x},
                                       half2_t{x1.y * s16, x3.y * s16}};
                const uint32_t lo = (n & 1) ? as_u32(pr[1]) : as_u32(pr[0]);
                const uint32_t hi = (n & 1) ? as_u32(pr[3]) : as_u32(pr[2]);
                qv[qa][grp] = (n & 2) ? hi : lo;
            }
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            vm[w] = -INFINITY;
            vl[w] = 0.0f;
            vlo[w] = INFINITY;
#pragma unroll
            for (int grp = 0; grp < G; ++grp) {
                vps[grp][w] = 0.0f;
                vo[grp][w][0] = vo[grp][w][1] = 0.0f;
            }
        }
    }

    // ---- compute one tile whose loads have landed.  The K registers are
    // consumed by QK; the next tile's K loads are issued right after, so they
    // fly during softmax and PV.
    // (bufc: std::integral_constant of the stage buffer, 0 or 1.)
    auto compute = [&](int tile, auto bufc, uint32_t (&kw)[2][L::KREGS], int next) {
        constexpr int kBufOff = decltype(bufc)::value * L::BUF;
        const uint8_t* const vb = stage + kBufOff;
        // scale of (token tok, this lane's kv head, grp) at [(tok * KVW) * G + grp]
        const uint32_t s_base = opaque(s_col);
        const half_t* const ks_lds = reinterpret_cast<const half_t*>(vb + L::VBUF + s_base);
        const half_t* const vs_lds = reinterpret_cast<const half_t*>(vb + L::VBUF + L::SBUF + s_base);
        const int tok_base = tile * kTile;
        const bool full = tok_base + kTile <= seq_len;
        if constexpr (D == 128) {
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int j = 0; j < KVW; ++j) {
                    u32x4_t x = {kw[r][j * G], kw[r][j * G + 1], kw[r][j * G + 2], kw[r][j * G + 3]};
                    transpose_rows4(x);
#pragma unroll
                    for (int q = 0; q < 4; ++q) kw[r][j * G + q] = x[q];
                }
        } else if constexpr (D == 64 && KVW == 1) {
            u32x4_t x = {kw[0][0], kw[0][1], kw[1][0], kw[1][1]};
            transpose_rows4(x);
            kw[0][0] = x[0];
            kw[0][1] = x[1];
            kw[1][0] = x[2];
            kw[1][1] = x[3];
        }
        // ---- QK: s[r][i] is token 16r + 4jq + i, column n (MFMA units)
        float s[2][4];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
#pragma unroll
            for (int i = 0; i < 4; ++i) s[r][i] = 0.0f;
#pragma unroll
            for (int grp = 0; grp < G; ++grp) {
                float4_t acc = {qinit[grp], qinit[grp], qinit[grp], qinit[grp]};
#pragma unroll
                for (int j = 0; j < KVW; ++j) acc = mfma16x16x32(k_operand(kw[r][j * G + grp]), qm[j][grp], acc);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    s[r][i] = __builtin_fmaf((float)ks_lds[(16 * r + i) * KVW * G + grp], acc[i], s[r][i]);
            }
        }
        if (next < t_end) issue_k(next, kw);
        // ---- online softmax (base 2, lazy rescale).  Token 16 r + 4 jq + i
        // of the tile is valid iff 16 r + i < nval.  (Maxima as
        // __builtin_elementwise_maximum: v_maximum3, which needs no
        // canonicalised operands after the masking selects; the scores are
        // finite or -inf.)
        const int nval = seq_len - tok_base - 4 * jq;
        // lowest score of the valid tokens (-inf: a non-finite K scale or
        // query); v_minimum3 needs no canonicalised operands
        auto vmin = [](float x, float y) { return __builtin_elementwise_minimum(x, y); };
        if (full) {
            s_lo = vmin(vmin(s_lo, vmin(vmin(s[0][0], s[0][1]), vmin(s[0][2], s[0][3]))),
                        vmin(vmin(s[1][0], s[1][1]), vmin(s[1][2], s[1][3])));
        } else {
            const int nv = opaque_int(nval);  // (the compares stay in this branch)
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (16 * r + i >= nv) s[r][i] = -INFINITY;
                    else s_lo = vmin(s_lo, s[r][i]);
                }
        }
        auto vmax = [](float x, float y) { return __builtin_elementwise_maximum(x, y); };
        float mx = vmax(vmax(vmax(s[0][0], s[0][1]), vmax(s[0][2], s[0][3])),
                        vmax(vmax(s[1][0], s[1][1]), vmax(s[1][2], s[1][3])));
        mx = row_max4(mx);  // finite: token tile*32 < seq_len
        if (__ballot(mx > m_run + lazy) != 0) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c24);
            m_run = m_new;
            l_part *= alpha;
#pragma unroll
            for (int grp = 0; grp < G; ++grp) {
                ps[grp] *= alpha;
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[grp][e][i] *= alpha;
            }
        }
        const float moff = -m_run * c24;
        float p[2][4];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[r][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r][i], c24, moff));
                l_part += p[r][i];
            }
        // ---- PV.  V scales as dwords (groups 2h, 2h + 1 of a token), so a
        // masked token clears whole dwords and each half feeds its product
        // directly.
        uint32_t vsd[2][4][G / 2];
        const uint32_t* const vs_w = reinterpret_cast<const uint32_t*>(vs_lds);
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int h = 0; h < G / 2; ++h) vsd[r][i][h] = vs_w[(16 * r + i) * KVW * G / 2 + h];
        if (!full) {
            // Tokens past seq_len may hold any bytes: never let their scale
            // reach the product (0 * NaN).  A real branch: the asm keeps the
            // compiler from turning it into selects that every tile executes.
            asm volatile("");
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (16 * r + i >= nval) {
#pragma unroll
                        for (int h = 0; h < G / 2; ++h) vsd[r][i][h] = 0u;
                    }
        }
        // V operands: the chunk of (kv j, group grp) sits at tr_base ^
        // ((j G + grp) << 4).  They are read in batches of NB, in the order
        // y = grp * KVW + j of the loop below, each batch when the loop
        // reaches its first chunk.
        constexpr int NB = G * KVW < 4 ? G * KVW : 4;
        const uint32_t stage_lds = (uint32_t)(uintptr_t)(const IRIS_LDS void*)stage;
        int2v_t wv[NB];
        auto read_v = [&](int y0) {
            uint32_t ad[NB];
#pragma unroll
            for (int k = 0; k < NB; ++k) {
                const int y = y0 + k, x = (y % KVW) * G + y / KVW;
                ad[k] = stage_lds + (tr_base ^ ((uint32_t)x << 4));
            }
            lds_tr8<NB, kBufOff>(ad, wv);
        };
#pragma unroll
        for (int grp = 0; grp < G; ++grp) {
            // B operand in the V slot order: slot -> token 16r + 4jq + i with
            // (r, i) = (k' >> 2, k' & 3), k' = kVSlotByte[slot].
            half8_t bp;
#pragma unroll
            for (int sl = 0; sl < 8; ++sl) {
                const int r = kVSlotByte[sl] >> 2, i = kVSlotByte[sl] & 3;
                bp[sl] = (half_t)__builtin_fmaf(p[r][i], (float)as_half2(vsd[r][i][grp >> 1])[grp & 1], 0.0f);
            }
            const half2_t one2 = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
            for (int qq = 0; qq < 4; ++qq)
                ps[grp] = __builtin_amdgcn_fdot2(half2_t{bp[2 * qq], bp[2 * qq + 1]}, one2, ps[grp], false);
#pragma unroll
            for (int j = 0; j < KVW; ++j) {
                const int y = grp * KVW + j;
                if (y % NB == 0) read_v(y);
                const half8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
                // Columns of other kv heads are zeroed; with one kv head per
                // wave only unused columns (n >= g) would be, and nothing of
                // theirs is ever stored.
                const half8_t bj = (KVW == 1 || (col_valid && col_kv == j)) ? bp : z;
                const int2v_t w = wv[y % NB];
                half8_t a0, a1;
                v_operands(w, a0, a1);
                o[grp][0] = mfma16x16x32(a0, bj, o[grp][0]);
                o[grp][1] = mfma16x16x32(a1, bj, o[grp][1]);
            }
        }
    };

    // ---- the VALU tile (VALU only; the layouts above the q setup).
    // V reads: supplier lane n of a row gives token T = (k & 1) + 16 ((k >> 1)
    // & 1) + 2 (k >> 2), k = n >> 1 (plus 4 per read), half n & 1, so each
    // dword of a read holds tokens (t, t + 1, t + 16, t + 17) and the code
    // masks pair t with t + 16.  The chunk of (kv head x / G, group x % G)
    // sits at position x ^ f(T) (f as for the loads above).
    const int kv_row = KVW == 4 ? jq : 0;
    const int vt_tok = ((n >> 1) & 1) + 16 * ((n >> 2) & 1) + 2 * (n >> 3);
    const uint32_t vt_base = (uint32_t)vt_tok * (C * 16) +
                             ((uint32_t)(((vt_tok & 3) | ((vt_tok >> 4) << 2)) & (C - 1)) << 4) + 8 * (n & 1);
    const uint32_t valu_s_tok = (uint32_t)(n * KVW * G) * 2;  // token n's scales in a stage's scale block
    auto compute_valu = [&](int tile, auto bufc, uint32_t (&kw)[2][L::KREGS], int next) {
        constexpr int kBufOff = decltype(bufc)::value * L::BUF;
        const uint8_t* const vb = stage + kBufOff;
        const uint32_t sb = opaque(valu_s_tok);
        const half_t* const ks_lds = reinterpret_cast<const half_t*>(vb + L::VBUF + sb);
        const half_t* const vs_lds = reinterpret_cast<const half_t*>(vb + L::VBUF + L::SBUF + sb) + kv_row * G;
        const int tok_base = tile * kTile;
        const bool full = tok_base + kTile <= seq_len;
        if constexpr (D == 128) {
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int j = 0; j < KVW; ++j) {
                    u32x4_t x = {kw[r][j * G], kw[r][j * G + 1], kw[r][j * G + 2], kw[r][j * G + 3]};
                    transpose_rows4(x);
#pragma unroll
                    for (int q = 0; q < 4; ++q) kw[r][j * G + q] = x[q];
                }
        } else if constexpr (D == 64 && KVW == 1) {
            u32x4_t x = {kw[0][0], kw[0][1], kw[1][0], kw[1][1]};
            transpose_rows4(x);
            kw[0][0] = x[0];
            kw[0][1] = x[1];
            kw[1][0] = x[2];
            kw[1][1] = x[3];
        }
        // ---- QK per 16-token half: partial sums over this row's chunk,
        // scaled per (token, group), then the four rows' partial sums added:
        // sc[r][w] = score of token 16 r + n, column col(rho, w)
        float sc[2][4];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            float sacc[4][4];
#pragma unroll
            for (int qa = 0; qa < 4; ++qa)
#pragma unroll
                for (int qb = 0; qb < 4; ++qb) sacc[qa][qb] = 0.0f;
#pragma unroll
            for (int grp = 0; grp < G; ++grp) {
                u32x4_t kp1 = {0, 0, 0, 0};
                if constexpr (KVW == 1) kp1 = __builtin_bit_cast(u32x4_t, k_operand(kw[r][grp]));
#pragma unroll
                for (int qa = 0; qa < 4; ++qa) {
                    const int j = KVW == 4 ? qa : 0;
                    const u32x4_t kp = KVW == 4 ? __builtin_bit_cast(u32x4_t, k_operand(kw[r][j * G + grp])) : kp1;
                    float acc[4];
                    qk_valu_quad(qa, acc, qv[qa][grp], qc[grp], kp);
                    const float ks = (float)ks_lds[16 * r * KVW * G + j * G + grp];
#pragma unroll
                    for (int qb = 0; qb < 4; ++qb) sacc[qa][qb] = __builtin_fmaf(ks, acc[qb], sacc[qa][qb]);
                    // in program order: unpacking every dword ahead of its
                    // chain would hold 4 VGPRs per dword
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                u32x4_t x;
#pragma unroll
                for (int k = 0; k < 4; ++k) x[k] = as_u32(KVW == 4 ? sacc[k][f] : sacc[f][k]);
                transpose_rows4(x);
                sc[r][f] = (as_f32(x[0]) + as_f32(x[1])) + (as_f32(x[2]) + as_f32(x[3]));
            }
        }
        if (next < t_end) issue_k(next, kw);
        {
            // lowest score of the valid tokens per column (-inf: a non-finite
            // K scale or query)
            const bool v0 = full || tok_base + n < seq_len, v1 = full || tok_base + 16 + n < seq_len;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                vlo[w] = __builtin_elementwise_minimum(
                    vlo[w], __builtin_elementwise_minimum(v0 ? sc[0][w] : INFINITY, v1 ? sc[1][w] : INFINITY));
        }
        if (!full) {
#pragma unroll
            for (int r = 0; r < 2; ++r)
                if (tok_base + 16 * r + n >= seq_len) {
#pragma unroll
                    for (int w = 0; w < 4; ++w) sc[r][w] = -INFINITY;
                }
        }
        // ---- online softmax per column (base 2, lazy rescale)
        float mx[4];
        bool grow = false;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            mx[w] = row16_max(fmaxf(sc[0][w], sc[1][w]));  // finite: token tile*32 < seq_len
            grow = grow || mx[w] > vm[w] + lazy;
        }
        if (__ballot(grow) != 0) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float m_new = fmaxf(vm[w], mx[w]);
                const float alpha = __builtin_amdgcn_exp2f((vm[w] - m_new) * c24);
                vm[w] = m_new;
                vl[w] *= alpha;
#pragma unroll
                for (int grp = 0; grp < G; ++grp) {
                    vps[grp][w] *= alpha;
                    vo[grp][w][0] *= alpha;
                    vo[grp][w][1] *= alpha;
                }
            }
        }
        float p[2][4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float moff = -vm[w] * c24;
#pragma unroll
            for (int r = 0; r < 2; ++r) p[r][w] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r][w], c24, moff));
            vl[w] += p[0][w] + p[1][w];
        }
        // ---- PV: B pairs p * v_scale of tokens (n, 16 + n), rounded once to fp16
        float vs0[G], vs1[G];
#pragma unroll
        for (int grp = 0; grp < G; ++grp) {
            vs0[grp] = (float)vs_lds[grp];
            vs1[grp] = (float)vs_lds[16 * KVW * G + grp];
        }
        if (!full) {
            asm volatile("");  // a real branch (see compute)
            if (tok_base + n >= seq_len) {
#pragma unroll
                for (int grp = 0; grp < G; ++grp) vs0[grp] = 0.0f;
            }
            if (tok_base + 16 + n >= seq_len) {
#pragma unroll
                for (int grp = 0; grp < G; ++grp) vs1[grp] = 0.0f;
            }
        }
        const uint32_t stage_lds = (uint32_t)(uintptr_t)(const IRIS_LDS void*)stage;
        const half2_t one2 = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
        for (int grp = 0; grp < G; ++grp) {
            uint32_t pv[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const half2_t h = {(half_t)(p[0][w] * vs0[grp]), (half_t)(p[1][w] * vs1[grp])};
                pv[w] = as_u32(h);
                vps[grp][w] = __builtin_amdgcn_fdot2(h, one2, vps[grp][w], false);
            }
            int2v_t rd[4];
            lds_tr8_x4<kBufOff, 4 * L::SEG>(stage_lds + (vt_base ^ ((uint32_t)(kv_row * G + grp) << 4)), rd);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t a0 = (uint32_t)rd[k][0], a8 = a0 >> 8, b0 = (uint32_t)rd[k][1], b8 = b0 >> 8;
                const uint32_t vlo[4] = {(a0 ^ 0x00080008u) & 0x000F000Fu, (a8 ^ 0x00080008u) & 0x000F000Fu,
                                         (b0 ^ 0x00080008u) & 0x000F000Fu, (b8 ^ 0x00080008u) & 0x000F000Fu};
                const uint32_t vhi[4] = {(a0 ^ 0x00800080u) & 0x00F000F0u, (a8 ^ 0x00800080u) & 0x00F000F0u,
                                         (b0 ^ 0x00800080u) & 0x00F000F0u, (b8 ^ 0x00800080u) & 0x00F000F0u};
                switch (k) {  // k is a constant in every unrolled use
                    case 0: pv_valu<0>(vo[grp], pv, vlo, vhi); break;
                    case 1: pv_valu<4>(vo[grp], pv, vlo, vhi); break;
                    case 2: pv_valu<8>(vo[grp], pv, vlo, vhi); break;
                    default: pv_valu<12>(vo[grp], pv, vlo, vhi); break;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    auto run_tile = [&](int tile, auto bufc, uint32_t (&kw)[2][L::KREGS], int next) {
        if constexpr (VALU) compute_valu(tile, bufc, kw, next);
        else compute(tile, bufc, kw, next);
    };

    // Wave w takes tiles t_begin + w, + nw, ...: a fixed split, so every
    // run (and every HIP-graph replay) adds the same terms in the same order.
    // Two stage buffers with compile-time bases: the loop is unrolled by two.
    while (tile < t_end) {
        int next = tile + nw;
        wait_vmem_all();  // this tile's V, scales (LDS) and K (registers) have landed
        if (next < t_end) issue_v(next, 1);
        run_tile(tile, std::integral_constant<int, 0>(), kw, next);
        tile = next;
        if (tile >= t_end) break;
        next = tile + nw;
        wait_vmem_all();
        if (next < t_end) issue_v(next, 0);
        run_tile(tile, std::integral_constant<int, 1>(), kw, next);
        tile = next;
    }
    // ---- final per-lane values: undo the code offset and the 2^-24 units,
    // back to base-2 logits for the merges
    if constexpr (VALU) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            vm[w] *= c24;
            vl[w] = row16_sum(poison_if_neg_inf(vlo[w], vl[w]));
#pragma unroll
            for (int grp = 0; grp < G; ++grp) vps[grp][w] = 8.0f * row16_sum(vps[grp][w]);
        }
    } else {
        m_run *= c24;
        l_part = row_sum4(poison_if_neg_inf(s_lo, l_part));
#pragma unroll
        for (int grp = 0; grp < G; ++grp) ps[grp] = 8.0f * row_sum4(ps[grp]);
    }

    // ---- merge the waves of this workgroup (LDS, MFMA C order: lane-major,
    // so stores and loads are free of bank conflicts)
    __syncthreads();  // every wave is done with its stage
    float* const mo = reinterpret_cast<float*>(smem + wave * L::WAVE_LDS);
    if constexpr (VALU) {
        // dim grp * 32 + 2 n + e of column col(jq, w), in C order
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int cw = KVW == 4 ? 4 * jq + w : 4 * w + jq;
#pragma unroll
            for (int grp = 0; grp < G; ++grp)
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    mo[((grp * 2 + e) * 4 + (n & 3)) * 64 + 16 * (n >> 2) + cw] =
                        vo[grp][w][e] * (e ? 1048576.0f : 16777216.0f) - vps[grp][w];
            if (n == 0) {
                mo[16 * D + cw] = vm[w];
                mo[16 * D + 16 + cw] = vl[w];
            }
        }
    } else {
#pragma unroll
        for (int grp = 0; grp < G; ++grp)
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    mo[((grp * 2 + e) * 4 + i) * 64 + lane] = o[grp][e][i] * (e ? 1048576.0f : 16777216.0f) - ps[grp];
        if (jq == 0) {
            mo[16 * D + n] = m_run;
            mo[16 * D + 16 + n] = l_part;
        }
    }
    __syncthreads();
    // Every thread serves one column (threadIdx % 16) for all its elements.
    const int col = threadIdx.x & 15;
    float fw[4];
    float mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w)
        if (w < nw) mstar = fmaxf(mstar, reinterpret_cast<const float*>(smem + w * L::WAVE_LDS)[16 * D + col]);
    float lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        fw[w] = 0.0f;
        if (w < nw) {
            const float* mw = reinterpret_cast<const float*>(smem + w * L::WAVE_LDS);
            fw[w] = __builtin_amdgcn_exp2f(mw[16 * D + col] - mstar);  // 0 for idle waves
            lsum += mw[16 * D + 16 + col] * fw[w];
        }
    }
    const float inv_l = 1.0f / lsum;
    auto merged = [&](int idx) {
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w)
            if (w < nw) acc += reinterpret_cast<const float*>(smem + w * L::WAVE_LDS)[idx] * fw[w];
        return acc * inv_l;
    };
    auto store_out = [&](int idx, float val) {
        const int64_t oi = ((int64_t)b * a.n_q_heads + kv0 * g + qoff + col) * D + c_order_dim(idx);
        if (a.out_f32) reinterpret_cast<float*>(a.out)[oi] = val;
        else reinterpret_cast<half_t*>(a.out)[oi] = (half_t)val;
    };
    if (n_chunks == 1) {
        if (col < n_cols)
            for (int idx = threadIdx.x; idx < 16 * D; idx += blockDim.x) store_out(idx, merged(idx));
        return;
    }

    // ---- split-KV: publish this chunk, and merge all chunks if it is the last.
    // The partials are written and read with agent-scope accesses (sc1: kept
    // coherent across the XCDs' L2 caches), and every wave waits for its
    // stores to complete before the barrier that precedes the arrival
    // increment, so the workgroup that sees the final count reads every
    // chunk's partial -- without a cache-wide writeback or invalidate.
    const int64_t n_kvb = a.n_kv_blocks;
    const int64_t slot = ((int64_t)b * a.max_chunks + chunk) * n_kvb + kvb;
    for (int idx = threadIdx.x; idx < 16 * D; idx += blockDim.x)
        __hip_atomic_store(a.ws_o + slot * 16 * D + idx, merged(idx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x < 16) {
        __hip_atomic_store(a.ws_ml + (slot * 16 + col) * 2, mstar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.ws_ml + (slot * 16 + col) * 2 + 1, lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_vmem_all();
    __syncthreads();
    uint32_t* const counter = a.counters + (int64_t)b * kCountersPerSeq + kvb;
    uint32_t* const ctl = reinterpret_cast<uint32_t*>(smem);  // wave 0's merge area is free now
    if (threadIdx.x == 0) ctl[1] = arrive_last(counter, (uint32_t)n_chunks) ? 1u : 0u;
    __syncthreads();
    if (ctl[1] == 0) return;

    // Partials are read with plain buffer loads carrying the sc1 cache bit
    // (coherent across the XCDs' L2 caches, like the stores), which the
    // compiler may issue together, unlike atomic loads.
    constexpr int kSC1 = 16;
    const int64_t slot0 = (int64_t)b * a.max_chunks * n_kvb + kvb;  // chunk c: slot0 + c * n_kvb
    const uint32_t o_stride = (uint32_t)(n_kvb * 16 * D * 4);        // bytes between chunks
    const uint32_t ml_stride = (uint32_t)(n_kvb * 32 * 4);
    const auto ro = page_rsrc(a.ws_o + slot0 * 16 * D, o_stride * (uint32_t)n_chunks);
    const auto rm = page_rsrc(a.ws_ml + slot0 * 32, ml_stride * (uint32_t)n_chunks);
    auto ld = [&](const __amdgpu_buffer_rsrc_t& rs, uint32_t off) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, kSC1));
    };
    // Chunks are merged in batches of CB with an online softmax; all loads of
    // a batch are issued together (indices clamped, surplus weights zeroed),
    // so up to CB chunks cost one memory round trip.
    // (8 at D = 64: the batch's registers set the kernel's VGPR count, and
    // there the tile loop needs fewer, so a smaller batch keeps more waves
    // resident; MI355X, configuration 4: 30.7 -> 29.4 us.  8 at D = 256,
    // whose tile loop holds twice the accumulators.)
    constexpr int CB = D == 128 ? 16 : 8;
    for (int base = threadIdx.x; base < 16 * D; base += 8 * (int)blockDim.x) {
        float acc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
        float m_acc = -INFINITY, l_acc = 0.0f;
        for (int c0 = 0; c0 < n_chunks; c0 += CB) {
            float mc[CB], lc[CB], oc[CB][8];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const uint32_t ch = (uint32_t)min(c0 + cb, n_chunks - 1);
                mc[cb] = ld(rm, ch * ml_stride + col * 8);
                lc[cb] = ld(rm, ch * ml_stride + col * 8 + 4);
#pragma unroll
                for (int k = 0; k < 8; ++k) oc[cb][k] = ld(ro, ch * o_stride + (uint32_t)min(base + k * (int)blockDim.x, 16 * D - 1) * 4);
            }
            float mb = m_acc;
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) mb = fmaxf(mb, mc[cb]);
            const float sc = __builtin_amdgcn_exp2f(m_acc - mb);  // 0 on the first batch
            l_acc *= sc;
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] *= sc;
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const float w = c0 + cb < n_chunks ? lc[cb] * __builtin_amdgcn_exp2f(mc[cb] - mb) : 0.0f;
                l_acc += w;
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] += w * oc[cb][k];
            }
            m_acc = mb;
        }
        const float inv2 = 1.0f / l_acc;
        if (col < n_cols) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int idx = base + k * (int)blockDim.x;
                if (idx < 16 * D) store_out(idx, acc[k] * inv2);
            }
        }
    }
}

template <int D, int KVW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2))) void int4_decode_kernel(DecodeArgs a) {
    decode_body<D, KVW, false>(a);
}
// The VALU tile (IRIS_DECODE_VALU_TILE; measured against the MFMA tile).
template <int D, int KVW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void int4_decode_valu_kernel(DecodeArgs a) {
    decode_body<D, KVW, true>(a);
}

// Blocks of 16 query heads per kv head (more than one only for Hq / Hkv > 16,
// each a workgroup of its own over the same pages).
static int query_blocks(int g) { return g > 16 ? (g + 15) / 16 : 1; }

// kv heads per wavefront: as many as fit in 16 MFMA columns (at most 4),
// dividing Hkv -- and fewer while the grid would hold under 512 wave-tiles
// at the block table's capacity (B=1-sized calls), which spreads the tile
// work over more waves (MI355X, B=1, Hq=32, Hkv=8, D=128: L=128
// 8.5 -> 6.9 us, L=512 12.4 -> 10.3 us, L=4096 15.2 -> 14.5 us).  Plan and
// launch see the same four values, so they agree.
static int pick_kvw(int g, int hkv, int64_t batch, int64_t max_pages, int64_t head_dim) {
    int kvw = head_dim == 256 ? 1 : 4;
    while (kvw > 1 && (kvw * g > 16 || hkv % kvw != 0)) kvw >>= 1;
    const int64_t cap_tiles = (max_pages * kPageSize + kTile - 1) / kTile;
    while (kvw > 1 && batch * (cap_tiles + 1) * (hkv / kvw) < 512) kvw >>= 1;
    return kvw;
}

// Dynamic LDS of one workgroup; above 64 KiB the kernel must be allowed to
// use it (gfx950 has 160 KiB per CU): -1 if that fails.
template <int D, int KVW, bool VALU>
static int lds_bytes(int nw) {
    const int bytes = DecodeLayout<D, KVW>::WAVE_LDS * nw;
    static std::atomic<uint64_t> lds_raised{0};
    const void* k;
    if constexpr (VALU) k = reinterpret_cast<const void*>(&int4_decode_valu_kernel<D, KVW>);
    else k = reinterpret_cast<const void*>(&int4_decode_kernel<D, KVW>);
    if (bytes > 65536 && allow_full_lds(k, lds_raised) != kOk) return -1;
    return bytes;
}

template <int D, int KVW, bool VALU = false>
static int launch_decode(dim3 grid, dim3 block, int nw, hipStream_t s, const DecodeArgs& a) {
    const int lds = lds_bytes<D, KVW, VALU>(nw);
    if (lds < 0) return kLaunchError;
    if constexpr (VALU) hipLaunchKernelGGL((int4_decode_valu_kernel<D, KVW>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((int4_decode_kernel<D, KVW>), grid, block, lds, s, a);
    return kOk;
}

// Workspace layout: [counters: counter_region_bytes(B)]
// [ws_o: B * max_chunks * n_kvb * 16 * D fp32][ws_ml: ... * 16 * 2 fp32].
// A split needs n_kvb <= kCountersPerSeq (every Hkv <= 128 qualifies).
static int64_t workspace_bytes(int64_t batch, int64_t n_kvb, int64_t max_chunks, int64_t head_dim) {
    return counter_region_bytes(batch) + batch * max_chunks * n_kvb * 16 * (head_dim + 2) * (int64_t)sizeof(float);
}

}  // namespace iris

using namespace iris;

constexpr int64_t kPagesMinBytes = 100000000;  // K/V bytes above which the page kernel is preferred

// Kernel choice.  The page-streaming kernel (decode_pages.hip) runs with
// pages_waves() (16) waves per workgroup, the general kernel here with 1-4,
// so the plan's waves_per_block names the kernel for the launch.  A plan
// asked for 16 waves uses the page kernel wherever it supports the shape;
// asked for 1-4, the general kernel.  Two selection bits above the wave
// count (IRIS_DECODE_PAGE_KERNEL, IRIS_DECODE_VALU_TILE of iris_hip.h), for
// A/B measurements and tests, travel from the plan's waves_per_block into
// its out_waves and so into the launch: the first keeps the page kernel
// itself for 16-wave plans (no streaming or MQA kernel), the second runs
// the general kernel with its VALU tile instead of MFMA (g = 4 at D = 128,
// g = 16 at D = 64; other shapes are refused).  Left to choose, the plan
// takes the page kernel where it is the faster one: head_dim 128 with at
// most 4 query heads per kv head and at least 4 kv heads (8 KB page slabs,
// the GQA shapes of 7-70B models), over batches of similar lengths (its one
// workgroup per CU balances ragged batches worse than the general kernel's
// many small ones) that read at least kPagesMinBytes of K/V.
// head_dim 96, 160, 192 and 224 at pages of 16 m tokens plan the head-dim
// kernel (decode_hd.hip) with no bit.  Page sizes that are not multiples
// of 16 up to 256 (which the plan is not told) need a fourth bit, which
// the caller asks for: IRIS_DECODE_TOKEN_PAGES, the head-dim kernel's
// token-page mode (every page size at head_dim 64-256; the plan also
// returns it by itself where it prefers that kernel, hd_preferred below);
// a launch with such a page size and no bit is refused.  Head dims no
// other kernel has (32, 288-512) run on the any-shape kernel
// (decode_any.hip), named by a third bit, IRIS_DECODE_ANY_KERNEL, which
// the plan sets for them by itself (and returns for token-page requests
// at such head dims); it may also be asked for at any shape.
constexpr int32_t kWaveMask = 0xFF;
constexpr int32_t kPageKernel = IRIS_DECODE_PAGE_KERNEL;
constexpr int32_t kValuTile = IRIS_DECODE_VALU_TILE;
constexpr int32_t kAnyKernel = IRIS_DECODE_ANY_KERNEL;
constexpr int32_t kTokenPages = IRIS_DECODE_TOKEN_PAGES;
// The selection bits of waves_per_block, or -1 if it is not a valid request
// (at most one bit).
static int32_t selection_of(int32_t waves_per_block) {
    if (waves_per_block < 0) return 0;  // (as 0: let the plan choose)
    const int32_t sel = waves_per_block & ~kWaveMask;
    if (sel != 0 && sel != kPageKernel && sel != kValuTile && sel != kAnyKernel && sel != kTokenPages) return -1;
    return sel;
}
static bool fast_head_dim(int64_t head_dim) { return head_dim == 64 || head_dim == 128 || head_dim == 256; }
static int32_t waves_of(int32_t waves_per_block) { return waves_per_block < 0 ? 0 : waves_per_block & kWaveMask; }
static bool pages_allowed(int32_t waves_per_block) {
    const int32_t w = waves_of(waves_per_block);
    return (selection_of(waves_per_block) & (kValuTile | kAnyKernel)) == 0 && (w == 0 || w == pages_waves());
}
static bool pages_preferred(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                            int64_t max_pages, int64_t total_tokens, int64_t max_tokens, bool lengths_known,
                            bool page_kernel) {
    // 8 query heads per kv head: only the streaming kernel's chunk mode (its
    // chunks cover at most stream_max_chunks() x 64 tiles of the block table),
    // for batches of similar lengths (configuration 5: B=4, L=131072); the
    // page kernel's g=8 layout is slower there than the general kernel.
    if (num_q_heads == 8 * num_kv_heads && stream_supported(num_q_heads, num_kv_heads, head_dim)) {
        if (page_kernel || max_pages * kPageSize > (int64_t)stream_max_chunks() * 64 * kTile) return false;
        // One or two sequences give its chunk mode too few workgroups
        // (MI355X, L=131072: B=1 100.3 us against 57.0 on the general
        // kernel; B=2 102.1 against 79.9; B=3, L=65536: 63.2 against 64.8).
        if (batch < 3) return false;
        if (total_tokens * num_kv_heads * (head_dim + head_dim / 8) < kPagesMinBytes) return false;
        return 4 * total_tokens >= 3 * batch * max_tokens;
    }
    if (head_dim != 128 || num_kv_heads < 4 || num_q_heads > 4 * num_kv_heads) return false;
    // Below ~100 MB of K/V the launch is too short for the page kernel's
    // deep pipeline (one workgroup per CU, a few stages each) and the
    // general kernel's many small chunks finish first (MI355X: B=8, L=8192,
    // 75 MB: 25 us against 29 us; B=32, L=4096, 151 MB: 36 us against 43).
    if (total_tokens * num_kv_heads * (head_dim + head_dim / 8) < kPagesMinBytes) return false;
    // Ragged lengths, known, go to its balanced mode (MI355X, configuration
    // 3: B=64, lengths log-uniform in [128, 16384]: 67 us against 78); with
    // unknown lengths the plan assumes the widest batch.
    return lengths_known || 4 * total_tokens >= 3 * batch * max_tokens;
}

// The MQA streaming kernel (decode_mqa.hip: one kv head, head_dim 64, at
// most 16 query heads) takes 16-wave plans of its shape.  Left to choose, the
// plan takes it for batches of similar lengths with at least kMqaMinBytes of
// K/V to read (configuration 4: B=128, L=8192, 76 MB); smaller or ragged
// batches go to the general kernel's many small chunks.
// IRIS_DECODE_PAGE_KERNEL keeps the page kernel instead, for A/B runs.
constexpr int64_t kMqaMinBytes = 16000000;
static bool mqa_allowed(int32_t waves_per_block) {
    const int32_t w = waves_of(waves_per_block);
    return selection_of(waves_per_block) == 0 && (w == 0 || w == mqa_waves());
}
static bool mqa_preferred(int64_t batch, int64_t total_tokens, int64_t max_tokens) {
    if (total_tokens * (64 + 8) < kMqaMinBytes) return false;
    return 4 * total_tokens >= 3 * batch * max_tokens;
}

// head_dim 64 and 128 below kPagesMinBytes: the head-dim kernel
// (decode_hd.hip) in its token-page mode takes the shapes the plan would
// give the general kernel when they have at least two kv heads, lengths of
// similar size and at most 256 (sequence, kv head, query block) units, and
// read at least kHdMinBytes of K/V at head_dim 64 -- its W-wave workgroups
// stream a unit's tiles with no workgroup barrier and its grid follows the
// XCDs (MI355X, back-to-back launches, us: B=4, L=8192, Hkv=8: 19.3 against
// 21.8; B=32, L=2048: 25.7 against 30.4; D=64, Hq=32, Hkv=8, B=32, L=2048:
// 16.8 against 21.8; B=1, L=32768: 22.5 against 47.2; B=1, Hq=32, Hkv=8,
// L=128: 7.3 against 8.2).  At head_dim 64 smaller launches favour the
// general kernel (B=1, Hq=32, Hkv=8, L=1024: 9.9 against 9.1), as do one kv
// head (B=1, Hq=16, L=16384: 36.1 against 19.2, the sequence cut into 64
// chunks for one merging workgroup), more units (B=64, L=1024: 34.9 against
// 33.0) and ragged lengths (B=64, lengths in [16, 4096]: 47.5 against 42.5).
// At head_dim 256 (where the general kernel holds one kv head a wave and
// one wave a SIMD) it takes every call with two or more kv heads: 1.4-1.6x
// the general kernel at every shape measured (B=8, L=8192: 47.9 against
// 77.3 us; B=32, L=4096, 303 MB: 78.2 against 119.6; B=1, L=8192: 26.4
// against 41.2; lengths in [128, 4096] at B=16: 41.0 against 59.2).
constexpr int64_t kHdMinBytes = 4000000;
static bool hd_preferred(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                         int64_t total_tokens, int64_t max_tokens) {
    if (num_kv_heads < 2) return false;
    if (head_dim == 256) return true;
    if (head_dim != 64 && head_dim != 128) return false;
    const int64_t units = batch * num_kv_heads * query_blocks((int)(num_q_heads / num_kv_heads));
    const int64_t bytes = total_tokens * num_kv_heads * (head_dim + head_dim / 8);
    return units <= 256 && (head_dim == 128 || bytes >= kHdMinBytes) && bytes < kPagesMinBytes &&
           4 * total_tokens >= 3 * batch * max_tokens;
}

// Split plan for one decode call.  total_tokens / max_tokens may be -1 when
// the caller does not know the sequence lengths; max_pages bounds them.
extern "C" int iris_decode_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                int64_t head_dim, int64_t max_pages, int64_t total_tokens,
                                int64_t max_tokens, int32_t tokens_per_split,
                                int32_t waves_per_block, int32_t* out_chunk_tiles,
                                int32_t* out_max_chunks, int32_t* out_waves,
                                int64_t* out_workspace_bytes) {
    if (batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || !any_supported(head_dim) ||
        max_pages <= 0 || max_pages > 0x3FFFFFFF)
        return kInvalidArgument;
    const int32_t sel = selection_of(waves_per_block);
    if (sel < 0) return kInvalidArgument;
    // head_dim 96, 160, 192 and 224: the MFMA kernel of decode_hd.hip
    // (page sizes of 16 m tokens; the others ask for the any-shape kernel).
    if (sel == 0 && hd_supported(head_dim))
        return hd_plan(batch, num_q_heads, num_kv_heads, head_dim, max_pages, total_tokens, max_tokens,
                       tokens_per_split, false, out_chunk_tiles, out_max_chunks, out_waves, out_workspace_bytes);
    if (sel == kTokenPages && hd_tok_supported(head_dim, num_kv_heads)) {
        const int st = hd_plan(batch, num_q_heads, num_kv_heads, head_dim, max_pages, total_tokens, max_tokens,
                               tokens_per_split, true, out_chunk_tiles, out_max_chunks, out_waves,
                               out_workspace_bytes);
        if (st == kOk) *out_waves |= kTokenPages;
        return st;
    }
    if (sel == kAnyKernel || sel == kTokenPages || !fast_head_dim(head_dim)) {
        const int st = any_plan(batch, num_q_heads, num_kv_heads, head_dim, max_pages * kPageSize, total_tokens,
                                max_tokens, tokens_per_split, out_chunk_tiles, out_max_chunks, out_workspace_bytes);
        if (st == kOk) *out_waves = any_waves() | kAnyKernel;
        return st;
    }
    // Unknown lengths (the sync-free positional handle): the widest batch
    // block_table admits stands in for them.
    const int64_t est_max = max_tokens < 0 ? max_pages * kPageSize : max_tokens;
    const int64_t est_total = total_tokens < 0 ? batch * est_max : total_tokens;
    if (mqa_allowed(waves_per_block) && mqa_supported(num_q_heads, num_kv_heads, head_dim) &&
        (waves_of(waves_per_block) == mqa_waves() || mqa_preferred(batch, est_total, est_max)) &&
        mqa_plan(batch, num_q_heads, head_dim, max_pages, max_tokens, tokens_per_split, out_chunk_tiles,
                 out_max_chunks, out_waves, out_workspace_bytes) == kOk)
        return kOk;
    if (pages_allowed(waves_per_block) && pages_supported(num_q_heads, num_kv_heads, head_dim, max_pages) &&
        (waves_of(waves_per_block) == pages_waves() ||
         pages_preferred(batch, num_q_heads, num_kv_heads, head_dim, max_pages, est_total, est_max,
                         total_tokens >= 0 && max_tokens >= 0, (sel & kPageKernel) != 0))) {
        const int st = pages_plan(batch, num_q_heads, num_kv_heads, head_dim, max_pages, total_tokens, max_tokens,
                                  tokens_per_split, (sel & kPageKernel) == 0, out_chunk_tiles, out_max_chunks,
                                  out_waves, out_workspace_bytes);
        if (st == kOk) *out_waves |= sel & kPageKernel;
        return st;
    }
    if (sel == 0 && waves_of(waves_per_block) == 0 &&
        hd_preferred(batch, num_q_heads, num_kv_heads, head_dim, est_total, est_max)) {
        const int st = hd_plan(batch, num_q_heads, num_kv_heads, head_dim, max_pages, total_tokens, max_tokens,
                               tokens_per_split, true, out_chunk_tiles, out_max_chunks, out_waves,
                               out_workspace_bytes);
        if (st == kOk) *out_waves |= kTokenPages;
        return st;
    }
    const int g = (int)(num_q_heads / num_kv_heads);
    const int kvw = pick_kvw(g, (int)num_kv_heads, batch, max_pages, head_dim);
    const int64_t n_kvb = num_kv_heads / kvw * query_blocks(g);
    const int64_t cap_tokens = max_pages * kPageSize;
    if (max_tokens < 0 || max_tokens > cap_tokens) max_tokens = cap_tokens;
    if (total_tokens < 0) total_tokens = batch * max_tokens;
    // The grid must cover every tile block_table can address (the kernel
    // cannot see a length it was not planned for); the measured lengths only
    // steer the chunk size.
    const int64_t max_tiles = (cap_tokens + kTile - 1) / kTile;
    int nw = waves_of(waves_per_block) > 0 ? waves_of(waves_per_block) : 4;
    if (nw > 4) nw = 4;
    int64_t chunk_tiles;
    if (tokens_per_split > 0) {
        chunk_tiles = (tokens_per_split + kTile - 1) / kTile;
    } else {
        // Aim for ~2048 resident waves (8 per CU on 256 CUs); small batches
        // get chunks of one tile a wave (B=1, L=4096: 15 us against 19 us
        // with four).
        const int64_t total_tiles = ((total_tokens + kTile - 1) / kTile + batch) * n_kvb;
        int64_t per_wave = (total_tiles + 2047) / 2048;
        if (per_wave < 1) per_wave = 1;
        chunk_tiles = per_wave * nw;
    }
    if (chunk_tiles < 1) chunk_tiles = 1;
    if (chunk_tiles > kMaxChunkTiles) chunk_tiles = kMaxChunkTiles;
    // One chunk per sequence when the longest one fits in a chunk.
    const int64_t longest_tiles = (max_tokens + kTile - 1) / kTile;
    if (chunk_tiles >= longest_tiles && max_tiles <= kMaxChunkTiles) chunk_tiles = max_tiles;
    int64_t max_chunks = (max_tiles + chunk_tiles - 1) / chunk_tiles;
    // Grids of at most one workgroup per CU are latency-bound, and there the
    // split-KV merge's round trips cost more than a second tile a wave: one
    // chunk when two tiles a wave cover the longest sequence, else no more
    // chunks than one merge batch reads at once (MI355X: configuration 1
    // 7.4 -> 6.2 us; B=1, Hq=32, Hkv=8, D=128, L=4096: 14.6 -> 12.9 us).
    if (tokens_per_split <= 0 && batch * n_kvb * max_chunks <= 256) {
        const int64_t merge_batch = head_dim == 128 ? 16 : 8;  // CB of the kernel's merge
        if (2 * chunk_tiles >= longest_tiles && max_tiles <= kMaxChunkTiles) {
            chunk_tiles = max_tiles;
        } else {
            while (max_chunks > merge_batch && 2 * chunk_tiles <= kMaxChunkTiles) {
                chunk_tiles *= 2;
                max_chunks = (max_tiles + chunk_tiles - 1) / chunk_tiles;
            }
        }
        max_chunks = (max_tiles + chunk_tiles - 1) / chunk_tiles;
    }
    if (max_chunks > 1 && n_kvb > kCountersPerSeq) return kInvalidArgument;
    *out_chunk_tiles = (int32_t)chunk_tiles;
    *out_max_chunks = (int32_t)max_chunks;
    *out_waves = nw | (sel & kValuTile);
    *out_workspace_bytes = max_chunks > 1 ? workspace_bytes(batch, n_kvb, max_chunks, head_dim) : 0;
    return kOk;
}

extern "C" int iris_int4_paged_decode_attention(
    const void* query, const void* k_data, const void* v_data, const void* k_scale,
    const void* v_scale, const int32_t* block_table, const int32_t* seq_lens, void* output,
    int32_t output_is_f32, void* workspace, int64_t workspace_bytes_avail, int64_t batch,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
    int64_t num_pages, int64_t max_pages, float softmax_scale, int32_t chunk_tiles,
    int32_t max_chunks, int32_t waves_per_block, void* stream) {
    const int32_t sel = selection_of(waves_per_block);
    if (sel < 0) return kInvalidArgument;
    if (sel == kAnyKernel)
        return any_launch(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output, output_is_f32,
                          workspace, workspace_bytes_avail, batch, num_q_heads, num_kv_heads, head_dim, page_size,
                          max_pages, softmax_scale, chunk_tiles, max_chunks, stream);
    if (sel == kTokenPages) {
        // token slots in 32 bits (2^32 slots of the smallest row, 72 bytes at
        // one kv head and head_dim 64, are more than an MI355X's 288 GB)
        if (page_size < 1 || max_pages <= 0 || page_size > 0x3FFFFFFF || max_pages > 0x3FFFFFFF ||
            num_pages < 0 || num_pages > ((int64_t)1 << 32) || num_pages * page_size > ((int64_t)1 << 32))
            return kInvalidArgument;
        // Odd scale rows (head_dim / 32 x Hkv odd) in a pool of an odd
        // number of token slots: the scale tensors end on the first half of
        // a dword, which the mode's dword loads of the last slot's last kv
        // head would pass; such calls run on the any-shape kernel, which
        // takes the same plan (chunks of 32-token tiles, an even count) and
        // the same workspace layout.
        if ((head_dim / 32 * num_kv_heads) % 2 != 0 && (num_pages * page_size) % 2 != 0)
            return any_launch(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output, output_is_f32,
                              workspace, workspace_bytes_avail, batch, num_q_heads, num_kv_heads, head_dim,
                              page_size, max_pages, softmax_scale, chunk_tiles, max_chunks, stream);
        const int64_t pages16 = (max_pages * page_size + kPageSize - 1) / kPageSize;
        return hd_launch(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output, output_is_f32,
                         workspace, workspace_bytes_avail, batch, num_q_heads, num_kv_heads, head_dim, pages16,
                         max_pages, 0, page_size, true, softmax_scale, chunk_tiles, max_chunks,
                         waves_of(waves_per_block), stream);
    }
    // page_size = 16 m (m at most 16): each table entry stands for m
    // consecutive 16-token pages, so the kernels see max_pages * m of them
    // per row (the count the plan was made with); they take the page code
    // log2(m) for a power of two, else -m (virtual_page in common.h).
    if (page_size < kPageSize || page_size > 16 * kPageSize || page_size % kPageSize != 0 || batch <= 0 ||
        num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
        !(fast_head_dim(head_dim) || hd_supported(head_dim)) || max_pages <= 0 ||
        max_pages * (page_size / kPageSize) > 0x3FFFFFFF)
        return kInvalidArgument;
    const int page_mul = (int)(page_size / kPageSize);
    const int shift = (page_mul & (page_mul - 1)) == 0 ? __builtin_ctz((unsigned)page_mul) : -page_mul;
    const int64_t bt_cols = max_pages;
    max_pages *= page_mul;
    const int32_t waves = waves_of(waves_per_block);
    if (hd_supported(head_dim)) {
        if (sel != 0) return kInvalidArgument;
        return hd_launch(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output, output_is_f32,
                         workspace, workspace_bytes_avail, batch, num_q_heads, num_kv_heads, head_dim, max_pages,
                         bt_cols, shift, kPageSize * page_mul, false, softmax_scale, chunk_tiles, max_chunks, waves,
                         stream);
    }
    if (waves == mqa_waves() && mqa_allowed(waves_per_block) &&
        mqa_supported(num_q_heads, num_kv_heads, head_dim) && chunk_tiles > 0)
        return mqa_launch(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output, output_is_f32,
                          workspace, workspace_bytes_avail, batch, num_q_heads, max_pages, bt_cols, shift,
                          softmax_scale, chunk_tiles, max_chunks, stream);
    if (waves == pages_waves() && pages_allowed(waves_per_block) &&
        pages_supported(num_q_heads, num_kv_heads, head_dim, max_pages))
        return pages_launch(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens, output, output_is_f32,
                            workspace, workspace_bytes_avail, batch, num_q_heads, num_kv_heads, head_dim, max_pages,
                            bt_cols, shift, softmax_scale, chunk_tiles, max_chunks, (sel & kPageKernel) == 0,
                            stream);
    if (chunk_tiles <= 0 || chunk_tiles > kMaxChunkTiles || max_chunks <= 0 || waves <= 0 || waves > 4 ||
        (sel & kPageKernel) != 0)
        return kInvalidArgument;
    if ((int64_t)chunk_tiles * max_chunks * 2 < max_pages) return kInvalidArgument;
    const int g = (int)(num_q_heads / num_kv_heads);
    const int kvw = pick_kvw(g, (int)num_kv_heads, batch, max_pages, head_dim);
    DecodeArgs a;
    a.q = (const half_t*)query;
    a.k_data = (const uint8_t*)k_data;
    a.v_data = (const uint8_t*)v_data;
    a.k_scale = (const half_t*)k_scale;
    a.v_scale = (const half_t*)v_scale;
    a.block_table = block_table;
    a.seq_lens = seq_lens;
    a.out = output;
    a.out_f32 = output_is_f32;
    a.batch = (int)batch;
    a.n_q_heads = (int)num_q_heads;
    a.n_kv_heads = (int)num_kv_heads;
    a.group = g;
    a.max_pages = (int)max_pages;
    a.bt_cols = (int)bt_cols;
    a.page_shift = shift;
    a.q_blocks = query_blocks(g);
    if ((int64_t)(num_kv_heads / kvw) * a.q_blocks > 0x7FFFFFFF) return kInvalidArgument;
    a.n_kv_blocks = (int)(num_kv_heads / kvw) * a.q_blocks;
    a.max_chunks = max_chunks;
    a.chunk_tiles = chunk_tiles;
    a.log2_scale = softmax_scale * 1.4426950408889634f;
    a.counters = nullptr;
    a.ws_o = nullptr;
    a.ws_ml = nullptr;
    if (max_chunks > 1) {
        if (a.n_kv_blocks > kCountersPerSeq) return kInvalidArgument;
        const int64_t need = workspace_bytes(batch, a.n_kv_blocks, max_chunks, head_dim);
        if (workspace == nullptr || workspace_bytes_avail < need) return kWorkspaceTooSmall;
        a.counters = (uint32_t*)workspace;
        a.ws_o = (float*)((uint8_t*)workspace + counter_region_bytes(batch));
        a.ws_ml = a.ws_o + batch * max_chunks * a.n_kv_blocks * 16 * head_dim;
    }
    const int64_t nblocks = batch * a.n_kv_blocks * (int64_t)max_chunks;
    if (nblocks > 0x7FFFFFFF) return kInvalidArgument;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((unsigned)nblocks), block(64 * waves);
    int st;
    if ((sel & kValuTile) != 0) {
        // The VALU tile covers the two layouts with 16 columns of one or four
        // kv heads: g = 4 at D = 128 (KVW 4) and g = 16 at D = 64 (KVW 1).
        if (head_dim == 128 && kvw == 4 && g == 4) st = launch_decode<128, 4, true>(grid, block, waves, s, a);
        else if (head_dim == 64 && kvw == 1 && g == 16) st = launch_decode<64, 1, true>(grid, block, waves, s, a);
        else return kInvalidArgument;
    } else if (head_dim == 128) {
        if (kvw == 4) st = launch_decode<128, 4>(grid, block, waves, s, a);
        else if (kvw == 2) st = launch_decode<128, 2>(grid, block, waves, s, a);
        else st = launch_decode<128, 1>(grid, block, waves, s, a);
    } else if (head_dim == 256) {
        st = launch_decode<256, 1>(grid, block, waves, s, a);
    } else {
        if (kvw == 4) st = launch_decode<64, 4>(grid, block, waves, s, a);
        else if (kvw == 2) st = launch_decode<64, 2>(grid, block, waves, s, a);
        else st = launch_decode<64, 1>(grid, block, waves, s, a);
    }
    if (st != kOk || hipGetLastError() != hipSuccess) return kLaunchError;
    return kOk;
}

// ------------------------------------------------ no-allocation entry point

namespace iris {
namespace {

// Split-KV workspace of iris_int4_paged_decode_attention_noalloc: one array
// per GPU (each device holds its own copy, at its own address), kept until
// the process ends.  Host code uses the address hipGetSymbolAddress returns
// on that device, never the array's name.
constexpr int64_t kScratchBytes = 8 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
struct ScratchSlot {
    std::atomic<uintptr_t> ptr{0};   // device address of `scratch` (0: not looked up yet)
    std::atomic<int64_t> batch{0};   // batch of the last split call: counters [0, batch) are zero
};
ScratchSlot g_scratch[kMaxScratchDevices];

__global__ void zero_words(uint32_t* p, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// Device address of `scratch` on the current device `dev`, looked up on the
// first call there (two threads racing store the same address).
int scratch_address(int dev, uint8_t** out) {
    ScratchSlot& s = g_scratch[dev];
    uintptr_t p = s.ptr.load(std::memory_order_acquire);
    if (p == 0) {
        void* addr = nullptr;
        if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || addr == nullptr) return kLaunchError;
        p = (uintptr_t)addr;
        s.ptr.store(p, std::memory_order_release);
    }
    *out = reinterpret_cast<uint8_t*>(p);
    return kOk;
}

}  // namespace
}  // namespace iris

extern "C" int iris_int4_paged_decode_attention_noalloc(
    const void* query, const void* k_data, const void* v_data, const void* k_scale, const void* v_scale,
    const int32_t* block_table, const int32_t* seq_lens, void* output, int32_t output_is_f32, int64_t batch,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_pages,
    int64_t max_pages, float softmax_scale, int32_t chunk_tiles, int32_t max_chunks, int32_t waves_per_block,
    void* stream) {
    using namespace iris;
    if (batch <= 0) return kInvalidArgument;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return kLaunchError;
    uint8_t* ws = nullptr;
    if (const int st = scratch_address(dev, &ws); st != kOk) return st;
    ScratchSlot& slot = g_scratch[dev];
    if (max_chunks > 1) {
        // A split call needs its sequences' counters at zero.  Every call
        // leaves the counters it used at zero, but a call with a smaller
        // batch writes partials over the counters of the sequences past it.
        const int64_t cb = counter_region_bytes(batch);
        if (cb > kScratchBytes) return kWorkspaceTooSmall;
        if (batch > slot.batch.load(std::memory_order_acquire)) {
            const int64_t words = cb / 4;
            const unsigned blocks = (unsigned)((words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024);
            hipLaunchKernelGGL(zero_words, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                               reinterpret_cast<uint32_t*>(ws), words);
            if (hipGetLastError() != hipSuccess) return kLaunchError;
        }
    }
    const int st = iris_int4_paged_decode_attention(query, k_data, v_data, k_scale, v_scale, block_table, seq_lens,
                                                    output, output_is_f32, ws, kScratchBytes, batch, num_q_heads,
                                                    num_kv_heads, head_dim, page_size, num_pages, max_pages,
                                                    softmax_scale, chunk_tiles, max_chunks, waves_per_block, stream);
    if (st == kOk && max_chunks > 1) slot.batch.store(batch, std::memory_order_release);
    return st;
}

extern "C" int iris_version(void) { return 100; }  // 0.1.0
