// Fused RoPE + INT4 group quantisation + nibble packing + paged scatter,
// hand-written for gfx950 (wave64).
//
// Replaces the TileLang kernel `_rope_int4_paged_append`
// (src/iris_kernel/fused_kv.py:419-597 in Hunter2030ZeRo/Iris-Kernel) and
// reproduces the eager semantics of `torch_eager_append`
// (src/iris_kernel/torch_eager_kv.py:110-337) bit for bit for fp16 inputs
// and group_size == 32, with any even rotary_dim <= head_dim (the reference's
// fused kernel requires rotary_dim == head_dim, fused_kv.py:644-645; its
// eager path rotates the first rotary_dim dims and passes the rest through,
// torch_eager_kv.py:35-49).
//
// Work mapping.  One (token, kv-head) row of D fp16 values is split into
// D/8 chunks of 8 dims (16 bytes); lane c of a row owns dims [8c, 8c+8) of K
// and of V.  A row occupies ROWLANES = next_pow2(D/8) consecutive lanes, so
// rows never straddle a wavefront and a wave holds 64/ROWLANES rows
// (D=128: 4 rows of 16 lanes).  With 8 dims per lane, the 4 lanes of a quad
// are exactly one 32-dim scale group, so the group amax is two quad
// shuffles.  Consecutive rows are consecutive heads of one token, whose
// cache rows are adjacent in the NHD page layout, so the code stores of a
// wave cover whole cache rows.
//
// RoPE (rotate-half, as torch_eager_kv.py:38-47) on the first R = rotary_dim
// dims: dim i < R/2 pairs with i + R/2.  When R is a multiple of 16 every
// chunk lies in one rotary half or in the passthrough part, and chunk
// c < R/8 pairs with chunk c +- R/16: one lane shuffle.  Other even R take
// the per-element path (PER_ELEM): each rotated dim reads its partner, cos
// and sin straight from memory.  Each product and each sum is an fp16
// operation, rounded to fp16 like torch's fp16 eager ops; this file is built
// with -ffp-contract=off so no product is fused.
#include "common.h"
#include "iris_hip.h"
#include "quant.h"

namespace iris {

// Lane `i` of this lane's quad (DPP quad_perm broadcast).
__device__ __forceinline__ uint32_t quad_lane(uint32_t x, int i) {
    switch (i) {
        case 1: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x55, 0xF, 0xF, true);
        case 2: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xAA, 0xF, 0xF, true);
        default: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xFF, 0xF, 0xF, true);
    }
}
// The value of the lane 4 above this one in its 16-lane row (DPP row_shl:4;
// used where that lane is in the same append row).
__device__ __forceinline__ uint32_t next_quad(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x104, 0xF, 0xF, true);
}

// Partner chunk's word for the chunk-aligned RoPE: with ROR8 (16 lanes a
// row, rotary_dim 128) chunk c pairs with c ^ 8, one DPP row rotate by 8;
// otherwise a lane shuffle to `partner`.
template <bool ROR8>
__device__ __forceinline__ uint32_t rope_partner(uint32_t x, int partner) {
    if constexpr (ROR8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, false);
    else return (uint32_t)__shfl((int)x, partner, 64);
}

// Maximum over the 4 lanes of a quad (one 32-dim group): DPP quad swaps,
// NaN-propagating maxima.
__device__ __forceinline__ half2_t quad_amax(half2_t m) {
    m = amax_max(m, as_half2((uint32_t)__builtin_amdgcn_mov_dpp((int)as_u32(m), 0xB1, 0xF, 0xF, false)));
    return amax_max(m, as_half2((uint32_t)__builtin_amdgcn_mov_dpp((int)as_u32(m), 0x4E, 0xF, 0xF, false)));
}

// RPT rows per thread: rows k * kRowsPerBlock + (thread's row) of the
// block's RPT * kRowsPerBlock.  Loads go out in three waves, each for all RPT
// rows: the slot and position words, then the K and V chunks, then (once the
// positions are in) the RoPE table chunks, so the table reads overlap the
// K/V reads instead of following them.  The launch uses RPT = 1.
//
// Row r is (token r / n_heads, head r % n_heads); the quotient is taken as
// trunc((r + 0.5) * RN64(1 / n_heads)) in fp64, exact for r < 2^31 and
// n_heads < 2^20 (the error, below 2^-21, stays under the 0.5 / n_heads
// margin).  The cache row of (slot, head) is slot * n_heads + head: pages
// are page_size consecutive slots, so the page split cancels.
template <int ROWLANES, int RPT, bool PER_ELEM, bool ROR8>
__global__ __launch_bounds__(256) void rope_int4_paged_append_kernel(
    const u32x4_t* __restrict__ key, const u32x4_t* __restrict__ value,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ slot_mapping,
    const half_t* __restrict__ cos_cache, const half_t* __restrict__ sin_cache,
    u32x4_t* __restrict__ k_data, u32x4_t* __restrict__ v_data,
    uint32_t* __restrict__ k_scale, uint32_t* __restrict__ v_scale,
    int n_rows, int n_heads, double inv_heads, int head_dim, int rotary_dim) {
    constexpr int kRowsPerBlock = 256 / ROWLANES;
    const int chunks = head_dim >> 3;  // 8 dims per lane
    const bool odd_groups = (head_dim >> 5) & 1;  // (head_dim 32, 96, 160, ...)
    const int lane = threadIdx.x & 63;
    const int c_raw = threadIdx.x & (ROWLANES - 1);
    const int c = c_raw < chunks ? c_raw : 0;  // padding lanes mirror chunk 0
    const int hr = rotary_dim >> 1;            // RoPE table width
    // Chunk-aligned RoPE (R % 16 == 0): chunks below R/8 rotate with the
    // chunk R/16 away; cos/sin chunk cc of the table row.
    const int rot_c = rotary_dim >> 3, half_c = rotary_dim >> 4;
    const bool rotated = !PER_ELEM && c < rot_c;
    const bool lo_half = c < half_c;
    const int cc = rotated ? (lo_half ? c : c - half_c) : 0;
    const int partner = (lane - c_raw) + (lo_half ? c + half_c : (rotated ? c - half_c : c));
    // x' * sin enters the lower rotary half negated: RN16(x' * -sin) is
    // -RN16(x' * sin), and a + (-b) is a - b.
    const uint32_t sin_sign = lo_half ? 0x80008000u : 0u;

    int row[RPT], head[RPT], tok[RPT];
    bool live[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const uint32_t r = blockIdx.x * (uint32_t)(kRowsPerBlock * RPT) + k * kRowsPerBlock + threadIdx.x / ROWLANES;
        live[k] = r < (uint32_t)n_rows && c_raw < chunks;
        row[k] = r < (uint32_t)n_rows ? (int)r : 0;  // tail rows mirror row 0, store nothing
        tok[k] = (int)(((double)row[k] + 0.5) * inv_heads);
        head[k] = row[k] - tok[k] * n_heads;
    }
    int slot[RPT], pos[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        slot[k] = slot_mapping[tok[k]];
        pos[k] = positions[tok[k]];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the three load waves in this order
    u32x4_t kx[RPT], vx[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        kx[k] = key[(uint64_t)(uint32_t)row[k] * (uint32_t)chunks + c];
        vx[k] = value[(uint64_t)(uint32_t)row[k] * (uint32_t)chunks + c];
    }
    __builtin_amdgcn_sched_barrier(0);
    // Unconditional table loads (no branch for the compiler to sink the
    // position loads into): with rotary_dim 0 the host points cos_cache and
    // sin_cache at the key tensor and every lane reads its first 16 bytes.
    u32x4_t cx[RPT], sx[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        cx[k] = sx[k] = u32x4_t{0, 0, 0, 0};
        if constexpr (!PER_ELEM) {
            // Positions of skipped tokens are not validated by the caller;
            // read the RoPE table at row 0 for them (the result is discarded).
            const int64_t p = slot[k] >= 0 ? pos[k] : 0;
            cx[k] = *reinterpret_cast<const u32x4_t*>(cos_cache + p * hr + cc * 8);
            sx[k] = *reinterpret_cast<const u32x4_t*>(sin_cache + p * hr + cc * 8);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        half2_t kr[4], vr[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const half2_t own = as_half2(kx[k][q]);
            const half2_t a = own * as_half2(cx[k][q]);                                    // x*cos, rounded to fp16
            const half2_t b = as_half2(rope_partner<ROR8>(kx[k][q], partner)) *
                              as_half2(sx[k][q] ^ sin_sign);                               // +-x'*sin, rounded
            kr[q] = rotated ? a + b : own;                                                 // rounded to fp16
            vr[q] = as_half2(vx[k][q]);
        }
        if constexpr (PER_ELEM) {
            // Any even R: dim d < R takes its partner, cos and sin from memory.
            const half_t* krow = reinterpret_cast<const half_t*>(key) + (int64_t)row[k] * head_dim;
            const int64_t p = slot[k] >= 0 ? pos[k] : 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = 8 * c + j;
                if (d < rotary_dim) {
                    const bool lo = d < hr;
                    const int ci = lo ? d : d - hr;
                    const half_t x = j & 1 ? kr[j >> 1].y : kr[j >> 1].x;
                    const half_t xp = krow[lo ? d + hr : d - hr];
                    const half_t ea = x * cos_cache[p * hr + ci];   // rounded to fp16
                    const half_t eb = xp * sin_cache[p * hr + ci];  // rounded to fp16
                    const half_t y = lo ? ea - eb : ea + eb;
                    if (j & 1) kr[j >> 1].y = y;
                    else kr[j >> 1].x = y;
                }
            }
        }
        // Group amax of K (low half) and V (high half) together: per-lane
        // maxima of |x| over the even and the odd dims, then the quad.
        half2_t km2 = __builtin_elementwise_abs(kr[0]), vm2 = __builtin_elementwise_abs(vr[0]);
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            km2 = amax_max(km2, __builtin_elementwise_abs(kr[q]));
            vm2 = amax_max(vm2, __builtin_elementwise_abs(vr[q]));
        }
        const half2_t kv_even = {km2.x, vm2.x}, kv_odd = {km2.y, vm2.y};
        const half2_t kvmax = quad_amax(amax_max(kv_even, kv_odd));

        const half_t ks16 = scale_from_amax((float)kvmax.x);
        const half_t vs16 = scale_from_amax((float)kvmax.y);
        const uint32_t kword = pack_group8(kr, (float)ks16);
        const uint32_t vword = pack_group8(vr, (float)vs16);

        // 128-bit code stores: the first lane of each quad (one 32-dim group)
        // gathers the quad's four words; 32-bit scale stores: the first lane
        // of every other quad pairs its group's scale with the next group's.
        const u32x4_t kq = {kword, quad_lane(kword, 1), quad_lane(kword, 2), quad_lane(kword, 3)};
        const u32x4_t vq = {vword, quad_lane(vword, 1), quad_lane(vword, 2), quad_lane(vword, 3)};
        const uint32_t ks = as_u32(half2_t{ks16, ks16});
        const uint32_t vs = as_u32(half2_t{vs16, vs16});
        const uint32_t ks2 = (ks & 0xFFFFu) | (next_quad(ks) << 16);
        const uint32_t vs2 = (vs & 0xFFFFu) | (next_quad(vs) << 16);
        if (live[k] && slot[k] >= 0 && (c & 3) == 0) {
            const uint64_t cache_row = (uint64_t)(uint32_t)slot[k] * (uint32_t)n_heads + (uint32_t)head[k];
            // D/2 bytes per row = chunks / 4 16-byte groups
            k_data[cache_row * (uint32_t)(chunks >> 2) + (c >> 2)] = kq;
            v_data[cache_row * (uint32_t)(chunks >> 2) + (c >> 2)] = vq;
            if (odd_groups) {
                // An odd number of groups: rows of scales are 2-byte aligned,
                // so each group's scale is a 16-bit store of its own.
                reinterpret_cast<uint16_t*>(k_scale)[cache_row * (uint32_t)(head_dim >> 5) + (c >> 2)] = (uint16_t)ks;
                reinterpret_cast<uint16_t*>(v_scale)[cache_row * (uint32_t)(head_dim >> 5) + (c >> 2)] = (uint16_t)vs;
            } else if ((c & 7) == 0) {  // D/32 scales per row, two per 32-bit word
                k_scale[(cache_row * (uint32_t)(head_dim >> 5) + (c >> 2)) >> 1] = ks2;
                v_scale[(cache_row * (uint32_t)(head_dim >> 5) + (c >> 2)) >> 1] = vs2;
            }
        }
    }
}

}  // namespace iris

using namespace iris;

extern "C" int iris_rope_int4_paged_append(
    const void* key, const void* value, const int32_t* positions, const int32_t* slot_mapping,
    const void* cos_cache, const void* sin_cache, void* k_data, void* v_data, void* k_scale,
    void* v_scale, int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim, int64_t rotary_dim,
    int64_t page_size, int64_t num_pages, int64_t max_position, void* stream) {
    (void)num_pages;
    (void)max_position;
    if (num_tokens < 0 || num_kv_heads <= 0 || page_size <= 0 || head_dim <= 0 ||
        head_dim % 32 != 0 || head_dim > 512 || rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 2 != 0)
        return kInvalidArgument;
    if (num_tokens == 0) return kOk;
    // 32-bit row indices and the fp64 row -> (token, head) split: a launch
    // covers fewer than 2^31 rows (2^31 rows of even D = 64 are 256 GiB of
    // fp16 K) of fewer than 2^20 heads.
    if (num_kv_heads >= (1 << 20) || num_tokens > (((int64_t)1 << 31) - 1) / num_kv_heads) return kInvalidArgument;
    const int64_t n_rows = num_tokens * num_kv_heads;
    const int chunks = (int)(head_dim / 8);
    int rowlanes = 8;
    while (rowlanes < chunks) rowlanes <<= 1;
    const int64_t rows_per_block = 256 / rowlanes;
    // One row a thread: the config-5 bulk append (4 x 8192 tokens, Hkv=8,
    // D=128) takes 32.0 us on MI355X against 33.6 with two rows a thread and
    // 34.7 with four, and 32.9 / 32.5 / 35.3 us with 128 / 512 / 1024-thread
    // blocks.
    const int64_t blocks = (n_rows + rows_per_block - 1) / rows_per_block;
    hipStream_t s = (hipStream_t)stream;
    const bool per_elem = rotary_dim % 16 != 0;
    const bool ror8 = rowlanes == 16 && rotary_dim == 128;
    const double inv_heads = 1.0 / (double)num_kv_heads;
    if (rotary_dim == 0) cos_cache = sin_cache = key;  // a readable 16 bytes; the values are not used
#define IRIS_LAUNCH_APPEND(RL, PE, ROR)                                                                      \
    hipLaunchKernelGGL((rope_int4_paged_append_kernel<RL, 1, PE, ROR>), dim3((unsigned)blocks), dim3(256), 0, s, \
                       (const u32x4_t*)key, (const u32x4_t*)value, positions, slot_mapping,                     \
                       (const half_t*)cos_cache, (const half_t*)sin_cache, (u32x4_t*)k_data,                    \
                       (u32x4_t*)v_data, (uint32_t*)k_scale, (uint32_t*)v_scale, (int)n_rows,                   \
                       (int)num_kv_heads, inv_heads, (int)head_dim, (int)rotary_dim)
#define IRIS_LAUNCH_APPEND_RPT(RL)                 \
    if (per_elem) IRIS_LAUNCH_APPEND(RL, true, false); \
    else IRIS_LAUNCH_APPEND(RL, false, false)
    switch (rowlanes) {
        case 8: IRIS_LAUNCH_APPEND_RPT(8); break;
        case 16:
            if (ror8) IRIS_LAUNCH_APPEND(16, false, true);
            else IRIS_LAUNCH_APPEND_RPT(16);
            break;
        case 32: IRIS_LAUNCH_APPEND_RPT(32); break;
        case 64: IRIS_LAUNCH_APPEND_RPT(64); break;
        default: return kInvalidArgument;
    }
#undef IRIS_LAUNCH_APPEND_RPT
#undef IRIS_LAUNCH_APPEND
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}
