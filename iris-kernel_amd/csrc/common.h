// Shared helpers for the gfx950 INT4 paged KV-cache kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace iris {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Status codes returned by every extern "C" entry point.
enum Status : int {
    kOk = 0,
    kInvalidArgument = 1,  // a shape / size outside what the kernels support
    kLaunchError = 2,      // hipGetLastError() reported a failure after launch
    kWorkspaceTooSmall = 3,
};

__device__ __forceinline__ half2_t as_half2(uint32_t x) { return __builtin_bit_cast(half2_t, x); }
__device__ __forceinline__ uint32_t as_u32(half2_t x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ uint32_t as_u32(float x) { return __builtin_bit_cast(uint32_t, x); }
// (By value: __builtin_bit_cast applied directly to an element of an
// ext_vector_type value, x[k], reads element 0 with hipcc 7.2's clang.)
__device__ __forceinline__ float as_f32(uint32_t x) { return __builtin_bit_cast(float, x); }

// Maximum / sum over the 16 lanes of a row (DPP: xor 1, xor 2, then the
// half-row and row mirrors).
__device__ __forceinline__ float dpp_f(float x, int ctrl) {
    switch (ctrl) {
        case 0: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
        case 1: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
        case 2: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
        default: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xF, 0xF, true));
    }
}
// Row maximum as four fused DPP maxima (v_max_f32_dpp; a VGPR a VALU
// instruction wrote is read through DPP two wait states later).  NaN
// operands follow v_max_f32: the other operand is returned.
__device__ __forceinline__ float row16_max(float x) {
    float y;
    asm volatile(
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=&v"(y)
        : "v"(x));
    return y;
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f(x, 0);
    x += dpp_f(x, 1);
    x += dpp_f(x, 2);
    return x + dpp_f(x, 3);
}

// Non-finite values inside a sequence's valid range.  The eager attention
// dequantises code * scale in fp32: a NaN K scale, or an infinite one (times
// a zero code, or summed over products of both signs), makes the logits of
// every query head of its kv head NaN, and the softmax makes those heads'
// outputs NaN.  In the kernels a NaN score already spreads to the head's
// softmax sum and output (p = exp2(NaN - m)); an infinite K scale (or query
// element) instead gives a score of +-inf, since the code offset is removed
// by a second sum whose residual need not be zero.  +inf spreads as NaN too
// (m = inf, p = exp2(inf - inf)), but -inf would only drop its token.  With
// finite scales and queries every score is finite, so each kernel keeps the
// lowest score of the valid tokens it has seen and, when that is -inf,
// poisons the head's softmax sum with kNonFinite before its outputs are
// formed.  (The one case that differs from the eager result: an infinite
// scale over nonzero codes whose products all have one sign, where eager
// gives a finite result for a -inf logit and the kernels NaN.)
constexpr float kNonFinite = __builtin_nanf("");
// x through an empty asm: the compiler cannot see where the value comes
// from, so code using it stays where it is written (masking compares of a
// sequence's last tile are not hoisted out of their branch into every tile).
__device__ __forceinline__ int opaque_int(int x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ float poison_if_neg_inf(float lowest, float l) {
    return lowest == -INFINITY ? kNonFinite : l;
}

// Split-KV arrival counters.  Every decode kernel keeps them in one region
// at the head of its workspace, kCountersPerSeq uint32 per sequence
// (sequence b's at [b * kCountersPerSeq, (b + 1) * kCountersPerSeq)), so
// their place never depends on the kernel, its plan or the other shapes:
// a workspace zero-filled once stays valid across calls of any layout, and
// a call with a larger batch than before only needs the counters of the new
// sequences zeroed.  Each launch leaves every counter it used at zero.
constexpr int kCountersPerSeq = 128;
inline int64_t counter_region_bytes(int64_t batch) { return (batch * kCountersPerSeq * 4 + 255) / 256 * 256; }

// Arrival at a split-KV counter, by one thread after every partial of the
// workgroup has been stored and every wave has waited for its stores to
// complete (s_waitcnt, then a workgroup barrier).  Returns true in the
// workgroup whose arrival completes the count, which also resets the counter
// for the next launch.
//
// Why the partials are visible to that workgroup without cache-wide fences:
// * the partials are written with sc1 stores, which write through the
//   non-coherent cache levels to memory, and the writer's wait means they
//   have reached it before its arrival is issued;
// * the arrival is an agent-scope atomic, performed at the device's
//   coherence point, so the count a workgroup sees includes every earlier
//   arrival;
// * the merging workgroup reads the partials with sc1 loads, which bypass
//   the non-coherent caches, and issues them only after its arrival has
//   returned the final count.
// An acquire-release arrival (what the HIP memory model prescribes) makes
// the compiler add buffer_wbl2 sc1 before it and buffer_inv sc1 after it: a
// write-back of the whole L2 and an invalidation of it, which these accesses
// do not need.  On MI355X that cost 1.2-2 us per cfg2 decode launch
// (38.7 against 40.3 us, A/B on one box).  The order this argument needs in
// the emitted code -- stores waited for and a barrier before the arrival, the
// merge's loads after its returned count and a barrier -- is checked on every
// decode kernel's gfx950 code by tests/test_isa_split_kv_order.py.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expect) {
    const uint32_t old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == expect;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return last;
}

// Pages of page_size = 16 m tokens are read as m consecutive 16-token pages
// (the [num_pages, page_size, ...] cache is the same bytes as a
// [num_pages * m, 16, ...] one): virtual 16-token page vp of a block-table
// row is 16-token page row[vp / m] * m + vp % m.  page_code is log2(m) when
// m is a power of two (a shift) and -m otherwise (a division, once per lane
// in a kernel's prologue); a kernel argument, so the branch is uniform.
__device__ __forceinline__ int virtual_page(const int32_t* row, int vp, int page_code) {
    if (page_code >= 0) return (row[vp >> page_code] << page_code) | (vp & ((1 << page_code) - 1));
    const int m = -page_code;
    const int e = vp / m;
    return row[e] * m + (vp - e * m);
}

// Grids whose slowest index is the split-KV chunk c (each XCD -- workgroup
// i runs on XCD i % 8 -- then gets its share of every chunk index, and the
// chunks past the sequences' ends leave no XCD idle) rotate the index r of
// the n sequences (or units) of a chunk by c, so one sequence's chunks run on
// different XCDs: position p of chunk c holds r = (p - c) mod n.
__device__ __forceinline__ int rotate_back(int p, int c, int n) {
    const int r = p - c % n;
    return r < 0 ? r + n : r;
}

// LDS a workgroup may use on gfx950 (per CU).
constexpr int kMaxLdsBytes = 160 * 1024;

// Lets `kernel` take up to kMaxLdsBytes of dynamic LDS on the current device
// (HIP's default limit is 64 KiB).  Done once per device, remembered in the
// caller's atomic bitmask (one per kernel), so concurrent launches from
// several host threads are safe: two threads racing here both set the same
// (idempotent) attribute.
inline int allow_full_lds(const void* kernel, std::atomic<uint64_t>& done) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return kLaunchError;
    const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
    if (bit != 0 && (done.load(std::memory_order_acquire) & bit)) return kOk;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLdsBytes) != hipSuccess)
        return kLaunchError;
    done.fetch_or(bit, std::memory_order_release);
    return kOk;
}

}  // namespace iris
