/*
 * iris_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the Iris-Kernel INT4 paged KV-cache semantics,
 * used as a checker by tests/, __graft_entry__.smoke() and the CPU-baseline
 * leg of bench.py.  Nothing in the product path (iris_kernel, libiris_hip.so)
 * links, loads or calls this file.
 *
 * What it restates (reference citations are /root/reference paths):
 *   - fp16 round-to-nearest-even conversion (torch's Tensor.to(float16)).
 *   - apply_rope            src/iris_kernel/torch_eager_kv.py:6-49
 *       rotate-half RoPE; every fp16 product and every fp16 sum/difference is
 *       rounded to fp16, as torch evaluates `x1 * cos - x2 * sin` in fp16.
 *   - quantize_int4_groupwise torch_eager_kv.py:52-88
 *       amax in fp32, scale32 = max(amax / 7, 2^-14) (IEEE division),
 *       scale16 = RN16(scale32), q = clamp(rint(x / fp32(scale16)), -7, 7).
 *   - pack_int4             torch_eager_kv.py:91-107 (even dim -> low nibble)
 *   - torch_eager_append    torch_eager_kv.py:110-337 (skip slot < 0,
 *       duplicate-slot / position / page range errors, scatter).
 *   - unpack_int4 / dequantize_int4_groupwise torch_eager_attention.py:8-53
 *   - torch_eager_int4_paged_decode_attention torch_eager_attention.py:154-239
 *       evaluated here in float64 (brute force), which pins the fp32 torch
 *       oracle and the HIP kernel to within the attention tolerance.
 *
 * It also holds two exhaustive proofs used by the tests: that the cheaper
 * operation sequences the HIP append kernel uses for the scale and for the
 * quantised value give bit-identical results to the reference's IEEE
 * division + round-half-even, for every fp16 input that can reach them.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 */

float ior_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    float out;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in float */
        out = (float)m * 5.9604644775390625e-08f;
        return sign ? -out : out;
    }
    if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    memcpy(&out, &bits, 4);
    return out;
}

/* Round a float to the nearest fp16, ties to even (IEEE 754 RNE). */
uint16_t ior_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7C00u);
    if (ax >= 0x38800000u) { /* result is a normal fp16 (>= 2^-14) */
        uint32_t mant = ax & 0x7FFFFFu;
        uint32_t e = (ax >> 23) - 127u + 15u;
        uint32_t h = (e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    /* subnormal range: units of 2^-24; scaling by 2^24 is exact here and
       rintf rounds half to even in the default rounding mode.  A result of
       1024 units is the smallest normal, whose encoding is also 1024. */
    float v;
    uint32_t a = ax;
    memcpy(&v, &a, 4);
    uint32_t units = (uint32_t)rintf(v * 16777216.0f);
    return (uint16_t)(sign | units);
}

static inline float rn16(float f) { return ior_f16_to_f32(ior_f32_to_f16(f)); }

/* -------------------------------------------------------- quantisation */

/* Reference scale: torch_eager_kv.py:75-83. */
static inline uint16_t scale_ref(float amax) {
    float s32 = amax / 7.0f;
    if (s32 < 6.103515625e-05f) s32 = 6.103515625e-05f; /* finfo(fp16).tiny */
    return ior_f32_to_f16(s32);
}

/* Reference quantised value: torch_eager_kv.py:85-86. */
static inline int quant_ref(float x, float qs) {
    float q = rintf(x / qs);
    if (q < -7.0f) q = -7.0f;
    if (q > 7.0f) q = 7.0f;
    return (int)q;
}

/* --------------------------------------------------------- write path */

/*
 * Fused-append semantics of torch_eager_append (torch_eager_kv.py:110-337)
 * for fp16 inputs.  Returns 0 on success, or
 *   -1 duplicate valid slots       (ValueError, :287-288)
 *   -2 a valid position < 0        (IndexError, :290-291)
 *   -3 a valid position >= maxpos  (IndexError, :293-294)
 *   -4 a valid slot beyond the pool (IndexError, :304-305)
 *   -5 bad static arguments
 * The caches are modified only when the return value is 0.
 */
int ior_append(const uint16_t *key, const uint16_t *value,
               const int64_t *positions, const int64_t *slots,
               const uint16_t *cos_cache, const uint16_t *sin_cache,
               uint8_t *k_data, uint8_t *v_data,
               uint16_t *k_scale, uint16_t *v_scale,
               int64_t T, int64_t H, int64_t D, int64_t P, int64_t NP,
               int64_t maxpos, int64_t rotary_dim, int64_t group_size) {
    if (T < 0 || H <= 0 || D <= 0 || P <= 0 || NP < 0 || group_size <= 0 ||
        D % group_size != 0 || D % 2 != 0 || rotary_dim < 0 ||
        rotary_dim > D || rotary_dim % 2 != 0)
        return -5;
    int64_t nvalid = 0;
    for (int64_t t = 0; t < T; ++t) nvalid += slots[t] >= 0;
    if (nvalid == 0) return 0;

    /* duplicate detection over valid slots: sort a copy */
    int64_t *vs = (int64_t *)malloc(sizeof(int64_t) * (size_t)nvalid);
    int64_t n = 0;
    for (int64_t t = 0; t < T; ++t)
        if (slots[t] >= 0) vs[n++] = slots[t];
    for (int64_t i = 1; i < n; ++i) { /* insertion sort is fine for tests */
        int64_t v = vs[i], j = i - 1;
        while (j >= 0 && vs[j] > v) { vs[j + 1] = vs[j]; --j; }
        vs[j + 1] = v;
    }
    int dup = 0;
    for (int64_t i = 1; i < n; ++i) dup |= vs[i] == vs[i - 1];
    free(vs);
    if (dup) return -1;
    for (int64_t t = 0; t < T; ++t)
        if (slots[t] >= 0 && positions[t] < 0) return -2;
    for (int64_t t = 0; t < T; ++t)
        if (slots[t] >= 0 && positions[t] >= maxpos) return -3;
    for (int64_t t = 0; t < T; ++t)
        if (slots[t] >= 0 && slots[t] / P >= NP) return -4;

    const int64_t half = rotary_dim / 2;
    const int64_t G = D / group_size;
    float *k = (float *)malloc(sizeof(float) * (size_t)D);
    for (int64_t t = 0; t < T; ++t) {
        if (slots[t] < 0) continue;
        const int64_t page = slots[t] / P, off = slots[t] % P;
        const uint16_t *cs = cos_cache + positions[t] * half;
        const uint16_t *sn = sin_cache + positions[t] * half;
        for (int64_t h = 0; h < H; ++h) {
            const uint16_t *kin = key + (t * H + h) * D;
            const uint16_t *vin = value + (t * H + h) * D;
            for (int64_t i = 0; i < half; ++i) {
                float x1 = ior_f16_to_f32(kin[i]);
                float x2 = ior_f16_to_f32(kin[i + half]);
                float c = ior_f16_to_f32(cs[i]);
                float s = ior_f16_to_f32(sn[i]);
                /* each fp16 product is exact in float, then rounded */
                float x1c = rn16(x1 * c), x2s = rn16(x2 * s);
                float x2c = rn16(x2 * c), x1s = rn16(x1 * s);
                k[i] = rn16(x1c - x2s);
                k[i + half] = rn16(x2c + x1s);
            }
            for (int64_t i = rotary_dim; i < D; ++i) k[i] = ior_f16_to_f32(kin[i]);

            const int64_t row = (page * P + off) * H + h;
            for (int pass = 0; pass < 2; ++pass) {
                uint8_t *dst = (pass == 0 ? k_data : v_data) + row * (D / 2);
                uint16_t *sdst = (pass == 0 ? k_scale : v_scale) + row * G;
                for (int64_t g = 0; g < G; ++g) {
                    float xs[4096];
                    float amax = 0.0f;
                    for (int64_t i = 0; i < group_size; ++i) {
                        int64_t d = g * group_size + i;
                        xs[i] = pass == 0 ? k[d] : ior_f16_to_f32(vin[d]);
                        float a = fabsf(xs[i]);
                        amax = a > amax ? a : amax;
                    }
                    uint16_t s16 = scale_ref(amax);
                    float qs = ior_f16_to_f32(s16);
                    sdst[g] = s16;
                    for (int64_t i = 0; i < group_size; i += 2) {
                        int64_t d = g * group_size + i;
                        int lo = quant_ref(xs[i], qs) & 0xF;
                        int hi = quant_ref(xs[i + 1], qs) & 0xF;
                        dst[d / 2] = (uint8_t)(lo | (hi << 4));
                    }
                }
            }
        }
    }
    free(k);
    return 0;
}

/* ---------------------------------------------------------- read path */

/* Signed nibble of a packed byte, even dim in the low nibble
   (torch_eager_attention.py:13-17: n >= 8 -> n - 16). */
static inline int nib(const uint8_t *row, int64_t d) {
    int b = row[d >> 1];
    int n = (d & 1) ? (b >> 4) & 0xF : b & 0xF;
    return n >= 8 ? n - 16 : n;
}

/*
 * Decode attention of torch_eager_int4_paged_decode_attention, in float64.
 * out: [B, Hq, D] doubles.  Returns 0, or
 *   -1 a sequence length <= 0           (ValueError, :134-135)
 *   -2 block_table has too few columns  (ValueError, :137-143)
 *   -3 an invalid physical page id used (IndexError, :145-149)
 *   -5 bad static arguments
 */
int ior_decode(const uint16_t *query, const uint8_t *k_data, const uint8_t *v_data,
               const uint16_t *k_scale, const uint16_t *v_scale,
               const int64_t *block_table, const int64_t *seq_lens,
               int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t P,
               int64_t group_size, int64_t NP, int64_t maxP, double softmax_scale,
               double *out) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D <= 0 || P <= 0 ||
        group_size <= 0 || D % group_size != 0)
        return -5;
    for (int64_t b = 0; b < B; ++b)
        if (seq_lens[b] <= 0) return -1;
    for (int64_t b = 0; b < B; ++b)
        if ((seq_lens[b] + P - 1) / P > maxP) return -2;
    for (int64_t b = 0; b < B; ++b) {
        int64_t used = (seq_lens[b] + P - 1) / P;
        for (int64_t i = 0; i < used; ++i) {
            int64_t pg = block_table[b * maxP + i];
            if (pg < 0 || pg >= NP) return -3;
        }
    }
    const int64_t g = Hq / Hkv, G = D / group_size;
    const int64_t nunits = B * Hq;
    int64_t u;
#pragma omp parallel for schedule(dynamic)
    for (u = 0; u < nunits; ++u) {
        const int64_t b = u / Hq, hq = u % Hq, hk = hq / g;
        const int64_t L = seq_lens[b];
        double *sc = (double *)malloc(sizeof(double) * (size_t)L);
        double q[1024];
        for (int64_t d = 0; d < D; ++d) q[d] = ior_f16_to_f32(query[(b * Hq + hq) * D + d]);
        double mx = -INFINITY;
        for (int64_t t = 0; t < L; ++t) {
            int64_t pg = block_table[b * maxP + t / P];
            int64_t row = (pg * P + t % P) * Hkv + hk;
            const uint8_t *kr = k_data + row * (D / 2);
            const uint16_t *ks = k_scale + row * G;
            double acc = 0.0;
            for (int64_t d = 0; d < D; ++d)
                acc += q[d] * (double)nib(kr, d) * (double)ior_f16_to_f32(ks[d / group_size]);
            sc[t] = acc * softmax_scale;
            mx = sc[t] > mx ? sc[t] : mx;
        }
        double den = 0.0;
        for (int64_t t = 0; t < L; ++t) { sc[t] = exp(sc[t] - mx); den += sc[t]; }
        double o[1024];
        for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
        for (int64_t t = 0; t < L; ++t) {
            int64_t pg = block_table[b * maxP + t / P];
            int64_t row = (pg * P + t % P) * Hkv + hk;
            const uint8_t *vr = v_data + row * (D / 2);
            const uint16_t *vs = v_scale + row * G;
            double p = sc[t] / den;
            for (int64_t d = 0; d < D; ++d)
                o[d] += p * (double)nib(vr, d) * (double)ior_f16_to_f32(vs[d / group_size]);
        }
        for (int64_t d = 0; d < D; ++d) out[(b * Hq + hq) * D + d] = o[d];
        free(sc);
    }
    return 0;
}

/* ------------------------------------------------------ exhaustive proofs */

/*
 * Scale: the HIP append kernel computes RN16(max(RN32(amax * RN32(1/7)), 2^-14))
 * instead of RN16(max(RN32(amax / 7), 2^-14)).  Count the fp16 amax values
 * (every finite non-negative fp16) where the two differ.
 */
int64_t ior_check_scale_mul(void) {
    const float c7 = (float)(1.0 / 7.0);
    int64_t bad = 0;
    for (uint32_t h = 0; h <= 0x7BFFu; ++h) {
        float a = ior_f16_to_f32((uint16_t)h);
        float f = a * c7;
        if (f < 6.103515625e-05f) f = 6.103515625e-05f;
        bad += ior_f32_to_f16(f) != scale_ref(a);
    }
    return bad;
}

/*
 * Quantised value: the HIP kernels compute, with r an approximation of 1/s
 * (v_rcp_f32, accurate to 1 ulp),
 *     t = RN(RN(x * r + 3072) + (1.5 * 2^23 - 3072))      (the first an fma)
 * and take the low nibble of t's bit pattern as the two's-complement INT4
 * code, with no clamp.  Count the (x, s) pairs where that nibble differs from
 * the reference's clamp(rint(x / s), -7, 7) & 0xF, over every scale s the
 * quantiser can emit (normal fp16 in [2^-14, RN16(65504/7)]) and every fp16 x
 * that can be quantised with it: |x| at most the largest fp16 amax whose
 * scale is s, since x belongs to the group whose amax set s.
 * rvariant: r = RN(1/s) moved by rvariant floats (+-2 covers any reciprocal
 * accurate to 2 ulp).  mode 1 widens x to |x| <= 8 s, past any group amax,
 * where the missing clamp shows; mode 2 rounds in one step,
 * t = RN(x * r + 1.5 * 2^23), which gets round-half-even cases wrong.  The
 * tests use modes 1 and 2 to show that the check detects such mistakes.
 */
int64_t ior_check_quant_grid(int rvariant, int mode) {
    static float amax_top[0x10000];
    for (uint32_t h = 0; h <= 0x7BFFu; ++h) { /* fp16 bit order is magnitude order */
        const float a = ior_f16_to_f32((uint16_t)h);
        amax_top[scale_ref(a)] = a;
    }
    const uint16_t smax = scale_ref(65504.0f);
    int64_t bad = 0;
    int32_t sh;
#pragma omp parallel for schedule(dynamic) reduction(+ : bad)
    for (sh = 0x0400; sh <= (int32_t)smax; ++sh) {
        const float s = ior_f16_to_f32((uint16_t)sh);
        float r = 1.0f / s;
        for (int i = 0; i < abs(rvariant); ++i) r = nextafterf(r, rvariant < 0 ? 0.0f : INFINITY);
        const float lim = mode == 1 ? 8.0f * s : amax_top[sh];
        for (uint32_t xh = 0; xh <= 0x7BFFu; ++xh) {
            const float xa = ior_f16_to_f32((uint16_t)xh);
            if (xa > lim) break;
            for (int sg = 0; sg < 2; ++sg) {
                const float x = sg ? -xa : xa;
                const float t = mode == 2 ? fmaf(x, r, 12582912.0f)
                                          : fmaf(x, r, 3072.0f) + (12582912.0f - 3072.0f);
                uint32_t tb;
                memcpy(&tb, &t, 4);
                bad += (int)(tb & 0xFu) != (quant_ref(x, s) & 0xF);
            }
        }
    }
    return bad;
}

/*
 * Packing: the kernels sum the 8 code bit patterns t_i = 0x4B400000 + k_i
 * of a group, shifted left by 4i, add 0x11111111 * (8 - 0x4B400000) and
 * xor 0x88888888 (all mod 2^32).  Count the tuples (k_0..k_7) in [-7, 7]^8
 * (all 15^8) for which that differs from the nibble packing of
 * pack_int4 (code i in bits [4i+3:4i], two's complement).  bias_delta is
 * added to the bias; the tests pass 1 to show that a wrong constant fails.
 */
int64_t ior_check_pack_sum(int32_t bias_delta) {
    const uint32_t bias = 0x11111111u * (8u - 0x4B400000u) + (uint32_t)bias_delta;
    int64_t bad = 0;
    int32_t hi;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (hi = 0; hi < 15 * 15 * 15 * 15; ++hi) {
        uint32_t acc_hi = 0, want_hi = 0;
        for (int i = 4, h = hi; i < 8; ++i, h /= 15) {
            const int k = h % 15 - 7;
            acc_hi += (0x4B400000u + (uint32_t)k) << (4 * i);
            want_hi |= ((uint32_t)k & 0xFu) << (4 * i);
        }
        for (int lo = 0; lo < 15 * 15 * 15 * 15; ++lo) {
            uint32_t acc = acc_hi, want = want_hi;
            for (int i = 0, l = lo; i < 4; ++i, l /= 15) {
                const int k = l % 15 - 7;
                acc += (0x4B400000u + (uint32_t)k) << (4 * i);
                want |= ((uint32_t)k & 0xFu) << (4 * i);
            }
            bad += ((acc + bias) ^ 0x88888888u) != want;
        }
    }
    return bad;
}

/* Array forms of the fp16 conversions, for the tests that pin them against
   numpy's float16 casts. */
void ior_f32_to_f16_array(const float *in, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ior_f32_to_f16(in[i]);
}

void ior_f16_to_f32_array(const uint16_t *in, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ior_f16_to_f32(in[i]);
}
