// The two other write-side kernels of the reference's fused_kv module, for
// gfx950 (wave64):
//
// * RoPE + paged append into an fp16 cache: replaces the TileLang kernel
//   `_rope_fp16_paged_append` (src/iris_kernel/fused_kv.py:8-150 in
//   Hunter2030ZeRo/Iris-Kernel).  K's first rotary_dim dims are rotated
//   (rotate-half, torch_eager_kv.py:38-49), the rest pass through; V is
//   copied; both go to slot page * page_size + offset of k_cache / v_cache
//   [NP, page_size, Hkv, D]; slots < 0 are skipped.  Every product and every
//   sum is an fp16 operation rounded to fp16, as torch's fp16 eager ops round
//   them (this file is built with -ffp-contract=off), so the cache rows are
//   bit-identical to apply_rope's.
// * Standalone group-32 INT4 quantise + pack: replaces
//   `_quantize_pack_int4_g32` (fused_kv.py:300-362): x [T, H, D] fp16 ->
//   packed [T, H, D/2] uint8 (even dim in the low nibble) and scales
//   [T, H, D/32] fp16, bit-identical to quantize_int4_groupwise + pack_int4
//   (torch_eager_kv.py:52-107) with the arithmetic of quant.h.
//
// Work mapping (both vector kernels): one 16-byte chunk (8 dims) of a
// (token, head) row per lane, rows of next_pow2(D / 8) lanes, so a quad of
// lanes is one 32-dim scale group.  The RoPE append reads its partner chunk
// (the other rotary half) straight from memory.
#include "common.h"
#include "iris_hip.h"
#include "quant.h"

namespace iris {

// RoPE append, 8 dims per lane; needs head_dim % 8 == 0 and rotary_dim % 16
// == 0 (each chunk lies in one rotary half or in the passthrough part).
template <int ROWLANES>
__global__ __launch_bounds__(256) void rope_fp16_append_kernel(
    const u32x4_t* __restrict__ key, const u32x4_t* __restrict__ value, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ slot_mapping, const half_t* __restrict__ cos_cache,
    const half_t* __restrict__ sin_cache, u32x4_t* __restrict__ k_cache, u32x4_t* __restrict__ v_cache,
    int64_t n_rows, int n_heads, int head_dim, int rotary_dim, int page_size) {
    constexpr int kRowsPerBlock = 256 / ROWLANES;
    const int chunks = head_dim >> 3;
    const int c = threadIdx.x & (ROWLANES - 1);
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / ROWLANES;
    if (row >= n_rows || c >= chunks) return;  // no cross-lane work here
    const int64_t tok = row / n_heads;
    const int head = (int)(row - tok * n_heads);
    const int slot = slot_mapping[tok];
    if (slot < 0) return;
    const u32x4_t kx = key[row * chunks + c];
    const u32x4_t vx = value[row * chunks + c];
    u32x4_t ky = kx;
    const int half_c = rotary_dim >> 4, rot_c = rotary_dim >> 3;
    if (c < rot_c) {
        const bool lo = c < half_c;
        const int cc = lo ? c : c - half_c;
        const u32x4_t kp = key[row * chunks + (lo ? c + half_c : c - half_c)];
        const int64_t t = (int64_t)positions[tok] * (rotary_dim >> 1) + cc * 8;
        const u32x4_t cx = *reinterpret_cast<const u32x4_t*>(cos_cache + t);
        const u32x4_t sx = *reinterpret_cast<const u32x4_t*>(sin_cache + t);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const half2_t a = as_half2(kx[q]) * as_half2(cx[q]);  // x * cos, rounded to fp16
            const half2_t b = as_half2(kp[q]) * as_half2(sx[q]);  // x' * sin, rounded to fp16
            ky[q] = as_u32(lo ? a - b : a + b);                   // rounded to fp16
        }
    }
    const int64_t page = slot / page_size;
    const int64_t off = slot - page * page_size;
    const int64_t cache_row = (page * page_size + off) * n_heads + head;
    k_cache[cache_row * chunks + c] = ky;
    v_cache[cache_row * chunks + c] = vx;
}

// RoPE append, one element per thread: any head_dim and any even rotary_dim.
__global__ __launch_bounds__(256) void rope_fp16_append_scalar_kernel(
    const half_t* __restrict__ key, const half_t* __restrict__ value, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ slot_mapping, const half_t* __restrict__ cos_cache,
    const half_t* __restrict__ sin_cache, half_t* __restrict__ k_cache, half_t* __restrict__ v_cache,
    int64_t n_elems, int n_heads, int head_dim, int rotary_dim, int page_size) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_elems) return;
    const int64_t row = e / head_dim;
    const int d = (int)(e - row * head_dim);
    const int64_t tok = row / n_heads;
    const int head = (int)(row - tok * n_heads);
    const int slot = slot_mapping[tok];
    if (slot < 0) return;
    const int half = rotary_dim >> 1;
    const half_t* const x = key + row * head_dim;
    half_t y = x[d];
    if (d < rotary_dim) {
        const int i = d < half ? d : d - half;
        const int64_t t = (int64_t)positions[tok] * half + i;
        const half_t cs = cos_cache[t], sn = sin_cache[t];
        if (d < half) {
            const half_t a = x[d] * cs, b = x[d + half] * sn;
            y = a - b;
        } else {
            const half_t a = x[d] * cs, b = x[d - half] * sn;
            y = a + b;
        }
    }
    const int64_t page = slot / page_size;
    const int64_t off = slot - page * page_size;
    const int64_t cache_row = (page * page_size + off) * n_heads + head;
    k_cache[cache_row * head_dim + d] = y;
    v_cache[cache_row * head_dim + d] = value[row * head_dim + d];
}

// Group-32 INT4 quantise + pack, 8 dims per lane (head_dim % 64 == 0,
// <= 512).  Lanes past the row's chunks and rows past the end mirror a live
// lane so the quad shuffles stay defined; they store nothing.
template <int ROWLANES>
__global__ __launch_bounds__(256) void quantize_pack_int4_kernel(const u32x4_t* __restrict__ x,
                                                                 uint32_t* __restrict__ packed,
                                                                 half_t* __restrict__ scales, int64_t n_rows,
                                                                 int head_dim) {
    constexpr int kRowsPerBlock = 256 / ROWLANES;
    const int chunks = head_dim >> 3;
    const int c_raw = threadIdx.x & (ROWLANES - 1);
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / ROWLANES;
    const bool live = row < n_rows && c_raw < chunks;
    const int64_t r = row < n_rows ? row : 0;
    const int c = c_raw < chunks ? c_raw : 0;
    const u32x4_t vx = x[r * chunks + c];
    half2_t v[4];
    half2_t m2 = {0, 0};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        v[q] = as_half2(vx[q]);
        m2 = amax_max(m2, __builtin_elementwise_abs(v[q]));
    }
    float amax = amax_max((float)m2.x, (float)m2.y);
    amax = amax_max(amax, __shfl_xor(amax, 1, 64));  // a quad is one 32-dim group
    amax = amax_max(amax, __shfl_xor(amax, 2, 64));
    const half_t s16 = scale_from_amax(amax);
    const uint32_t word = pack_group8(v, (float)s16);
    if (live) {
        packed[r * chunks + c] = word;
        if ((c & 3) == 0) scales[r * (head_dim >> 5) + (c >> 2)] = s16;
    }
}

}  // namespace iris

using namespace iris;

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

extern "C" int iris_rope_fp16_paged_append(const void* key, const void* value, const int32_t* positions,
                                           const int32_t* slot_mapping, const void* cos_cache,
                                           const void* sin_cache, void* k_cache, void* v_cache,
                                           int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                                           int64_t rotary_dim, int64_t page_size, int64_t num_pages,
                                           int64_t max_position, void* stream) {
    (void)num_pages;
    (void)max_position;
    if (num_tokens < 0 || num_kv_heads <= 0 || page_size <= 0 || head_dim <= 0 || rotary_dim < 0 ||
        rotary_dim > head_dim || rotary_dim % 2 != 0 || head_dim > (1 << 20))
        return kInvalidArgument;
    if (num_tokens == 0) return kOk;
    hipStream_t s = (hipStream_t)stream;
    const int64_t n_rows = num_tokens * num_kv_heads;
    const bool vec = head_dim % 8 == 0 && rotary_dim % 16 == 0 && head_dim <= 512 && aligned16(key) &&
                     aligned16(value) && aligned16(cos_cache) && aligned16(sin_cache) && aligned16(k_cache) &&
                     aligned16(v_cache);
    if (vec) {
        const int chunks = (int)(head_dim / 8);
        int rowlanes = 1;
        while (rowlanes < chunks) rowlanes <<= 1;
        const int64_t rows_per_block = 256 / rowlanes;
        const int64_t blocks = (n_rows + rows_per_block - 1) / rows_per_block;
        if (blocks > 0x7FFFFFFF) return kInvalidArgument;
#define IRIS_LAUNCH_F16_APPEND(RL)                                                                     \
    hipLaunchKernelGGL(rope_fp16_append_kernel<RL>, dim3((unsigned)blocks), dim3(256), 0, s,          \
                       (const u32x4_t*)key, (const u32x4_t*)value, positions, slot_mapping,            \
                       (const half_t*)cos_cache, (const half_t*)sin_cache, (u32x4_t*)k_cache,          \
                       (u32x4_t*)v_cache, n_rows, (int)num_kv_heads, (int)head_dim, (int)rotary_dim, \
                       (int)page_size)
        switch (rowlanes) {
            case 1: IRIS_LAUNCH_F16_APPEND(1); break;
            case 2: IRIS_LAUNCH_F16_APPEND(2); break;
            case 4: IRIS_LAUNCH_F16_APPEND(4); break;
            case 8: IRIS_LAUNCH_F16_APPEND(8); break;
            case 16: IRIS_LAUNCH_F16_APPEND(16); break;
            case 32: IRIS_LAUNCH_F16_APPEND(32); break;
            case 64: IRIS_LAUNCH_F16_APPEND(64); break;
            default: return kInvalidArgument;
        }
#undef IRIS_LAUNCH_F16_APPEND
    } else {
        const int64_t n_elems = n_rows * head_dim;
        const int64_t blocks = (n_elems + 255) / 256;
        if (blocks > 0x7FFFFFFF) return kInvalidArgument;
        hipLaunchKernelGGL(rope_fp16_append_scalar_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                           (const half_t*)key, (const half_t*)value, positions, slot_mapping,
                           (const half_t*)cos_cache, (const half_t*)sin_cache, (half_t*)k_cache, (half_t*)v_cache,
                           n_elems, (int)num_kv_heads, (int)head_dim, (int)rotary_dim, (int)page_size);
    }
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}

extern "C" int iris_quantize_pack_int4(const void* x, void* packed, void* scales, int64_t num_tokens,
                                       int64_t num_heads, int64_t head_dim, void* stream) {
    if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 64 != 0 || head_dim > 512)
        return kInvalidArgument;
    if (num_tokens == 0) return kOk;
    const int64_t n_rows = num_tokens * num_heads;
    const int chunks = (int)(head_dim / 8);
    int rowlanes = 8;
    while (rowlanes < chunks) rowlanes <<= 1;
    const int64_t rows_per_block = 256 / rowlanes;
    const int64_t blocks = (n_rows + rows_per_block - 1) / rows_per_block;
    if (blocks > 0x7FFFFFFF) return kInvalidArgument;
    hipStream_t s = (hipStream_t)stream;
#define IRIS_LAUNCH_QPACK(RL)                                                                          \
    hipLaunchKernelGGL(quantize_pack_int4_kernel<RL>, dim3((unsigned)blocks), dim3(256), 0, s,          \
                       (const u32x4_t*)x, (uint32_t*)packed, (half_t*)scales, n_rows, (int)head_dim)
    switch (rowlanes) {
        case 8: IRIS_LAUNCH_QPACK(8); break;
        case 16: IRIS_LAUNCH_QPACK(16); break;
        case 32: IRIS_LAUNCH_QPACK(32); break;
        case 64: IRIS_LAUNCH_QPACK(64); break;
        default: return kInvalidArgument;
    }
#undef IRIS_LAUNCH_QPACK
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}
