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
// ior_check_quant_grid); the GPU parity tests run them on every config.
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
// below is a separately rounded fp32 operation unless written as an fma.
#pragma once

#include "common.h"

namespace iris {

// RN32(1/7).  RN16(max(RN32(amax * kOneSeventh), 2^-14)) equals
// RN16(max(RN32(amax / 7), 2^-14)) for every finite fp16 amax >= 0.
constexpr float kOneSeventh = (float)(1.0 / 7.0);
constexpr float kMinScale = 6.103515625e-05f;  // finfo(float16).tiny = 2^-14

// max as torch.amax computes it: a NaN operand gives NaN (v_maximum3_f32,
// not the NaN-dropping v_max_f32).
__device__ __forceinline__ float amax_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ half2_t amax_max(half2_t a, half2_t b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ half_t scale_from_amax(float amax) {
    const float s = __builtin_elementwise_maximum(amax * kOneSeventh, kMinScale);  // clamp_min keeps NaN
    if (s != s) return __builtin_bit_cast(half_t, (uint16_t)0x7E00);
    return (half_t)s;  // v_cvt_f16_f32, round to nearest even
}

// Code of x with scale s, given r within 2 ulp of 1/s, in two roundings:
//   g = RN(x * r + 3072)          one fma: x/s rounded to a 2^-12 grid
//   t = RN(g + (1.5 * 2^23 - 3072))  that rounded to an integer, ties to even
// t's bit pattern is 0x4B400000 + k for the code k.  Why it is exact: x and
// s are fp16, so a quotient x/s that is not a half-integer lies at least
// 2^-12 from every half-integer, while x * r is within 2^-20 of x/s.  The
// grid rounding therefore lands exactly on k + 1/2 at a tie and never lands
// on one otherwise, and the second rounding breaks ties to even as rint does.
// No clamp is needed: |x| <= amax and s >= RN16(amax / 7) bound |x/s| by
// 7.004, so k lies in [-7, 7].
constexpr float kGrid = 3072.0f;                         // 1.5 * 2^11: ulp 2^-12
constexpr float kGridToInt = 12582912.0f - 3072.0f;      // exact in fp32
__device__ __forceinline__ uint32_t code_bits(float x, float r) {
    return as_u32(__builtin_fmaf(x, r, kGrid) + kGridToInt);
}

// 8 codes of one 32-dim group, low nibble first (value i in bits [4i+3:4i]).
// Summing code_bits(x_i) << 4i gives sum(k_i 16^i) plus a known constant;
// adding 8 * 0x11111111 turns that into the offset-binary nibbles k_i + 8
// (each in [1, 15], so no carries), and xor 0x88888888 into two's complement.
constexpr uint32_t kPackBias = 0x11111111u * (8u - 0x4B400000u);
__device__ __forceinline__ uint32_t quant_pack8(const half2_t v[4], float r) {
    uint32_t acc = code_bits((float)v[0].x, r);
    acc += code_bits((float)v[0].y, r) << 4;
#pragma unroll
    for (int q = 1; q < 4; ++q) {
        acc += code_bits((float)v[q].x, r) << (8 * q);
        acc += code_bits((float)v[q].y, r) << (8 * q + 4);
    }
    return (acc + kPackBias) ^ 0x88888888u;
}

// quant_pack8 for a group whose stored scale is s: all-zero codes when s is
// NaN or infinite (see the header comment).
__device__ __forceinline__ uint32_t pack_group8(const half2_t v[4], float s) {
    const uint32_t word = quant_pack8(v, __builtin_amdgcn_rcpf(s));
    return __builtin_isfinite(s) ? word : 0u;
}

}  // namespace iris
