// INT4 group quantiser arithmetic shared by the append and quantise-pack
// kernels.  Bit-exact with the reference quantiser
// (torch_eager_kv.py:75-86 in Hunter2030ZeRo/Iris-Kernel):
//
//   scale16 = RN16(max(amax / 7, 2^-14))
//   q       = clamp(rint_half_even(x / float(scale16)), -7, 7)
//
// without an IEEE divide per value.  Both replacements below were checked
// exhaustively against the reference formulas for every fp16 input that can
// reach them (oracle/iris_oracle.c: ior_check_scale_mul,
// ior_check_quant_fast); the GPU parity tests run them on every config.
//
// Non-finite groups follow torch: the group amax (torch.amax) and the clamp
// (clamp_min) propagate NaN, so a group holding a NaN gets a NaN scale, and
// a group holding an infinity (and no NaN) an infinite one.  torch's
// fp32 -> fp16 conversion stores every NaN as 0x7E00.  With such a scale
// every x / scale is +-0 or NaN, and float -> int8 turns both into 0, so all
// codes of the group are 0 (the kernels use amax_max below for the group
// maximum and pack_group8 for the codes).
//
// This file must be compiled with -ffp-contract=off: every multiply and add
// below is a separately rounded fp32 operation.
#pragma once

#include "common.h"

namespace iris {

// RN32(1/7).  RN16(max(RN32(amax * kOneSeventh), 2^-14)) equals
// RN16(max(RN32(amax / 7), 2^-14)) for every finite fp16 amax >= 0.
constexpr float kOneSeventh = (float)(1.0 / 7.0);
constexpr float kMinScale = 6.103515625e-05f;  // finfo(float16).tiny = 2^-14
constexpr float kRoundMagic = 12582912.0f;     // 1.5 * 2^23

// max as torch.amax computes it: a NaN operand gives NaN (v_maximum3_f32,
// not the NaN-dropping v_max_f32).
__device__ __forceinline__ float amax_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ half2_t amax_max(half2_t a, half2_t b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ half_t scale_from_amax(float amax) {
    const float s = __builtin_elementwise_maximum(amax * kOneSeventh, kMinScale);  // clamp_min keeps NaN
    if (s != s) return __builtin_bit_cast(half_t, (uint16_t)0x7E00);
    return (half_t)s;  // v_cvt_f16_f32, round to nearest even
}

// Two's-complement INT4 code of clamp(rint(x / s), -7, 7) in bits [3:0] of
// the result; bits [31:4] are garbage.  r must be within 1 ulp of 1/s.
//   y  = x * r                  (|y - x/s| < 2^-19 for |x/s| <= 8)
//   y2 = y + r * (x - y * s)    one correction step; at an exact tie
//                               x/s = k + 1/2 it lands exactly on k + 1/2
//   t  = clamp(y2) + 1.5*2^23   the add rounds to an integer, ties to even,
//                               and leaves that integer in the low mantissa
//                               bits (two's complement for negative values).
__device__ __forceinline__ uint32_t quant_code(float x, float s, float r) {
    float y = x * r;
    float e = __builtin_fmaf(-y, s, x);
    float y2 = __builtin_fmaf(r, e, y);
    y2 = __builtin_amdgcn_fmed3f(y2, -7.0f, 7.0f);
    return as_u32(y2 + kRoundMagic);
}

// Quantise 8 fp16 values (one 16-byte chunk) with a given scale; returns the
// 8 codes packed low nibble first (value i in bits [4i+3:4i]).
__device__ __forceinline__ uint32_t quant_pack8(const half2_t v[4], float s, float r) {
    uint32_t word = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t lo = quant_code((float)v[q].x, s, r) & 0xFu;
        uint32_t hi = quant_code((float)v[q].y, s, r) & 0xFu;
        word |= (lo | (hi << 4)) << (8 * q);
    }
    return word;
}

// quant_pack8 for a group whose stored scale is s: all-zero codes when s is
// NaN or infinite (see the header comment).
__device__ __forceinline__ uint32_t pack_group8(const half2_t v[4], float s) {
    const uint32_t word = quant_pack8(v, s, __builtin_amdgcn_rcpf(s));
    return __builtin_isfinite(s) ? word : 0u;
}

}  // namespace iris
