// FP16 paged decode attention for gfx950 (MI355X): the matched FP16 baseline
// of the INT4 path.
//
// Replaces the TileLang kernel `_fp16_paged_decode_attention`
// (src/iris_kernel/fused_attention.py:223-370 in Hunter2030ZeRo/Iris-Kernel)
// and computes what `torch_eager_fp16_paged_decode_attention`
// (torch_eager_attention.py:242-294) computes: for sequence b and query head
// h, softmax(q . K^T * scale) . V over the first seq_lens[b] tokens, K and V
// read from kv head h / (Hq / Hkv) of the fp16 cache [NP, 16, Hkv, D]
// through block_table.
//
// Work decomposition
// ------------------
// * Workgroup = (sequence b, kv head j, chunk of pages), 4 waves.  Wave w
//   takes the chunk's pages w, w + 4, ... (a fixed split, so results do not
//   depend on timing) and keeps its own online softmax; the four are merged
//   in LDS at the end.
// * Unit of work: one 16-token page of one kv head.  Its K and V rows are
//   16 x D fp16 at a stride of Hkv * D halves; lane (row n, quarter jq)
//   loads 16 bytes of token n per 32 dims, so each load instruction covers
//   64 contiguous bytes of every row of the page and the four instructions
//   of a page cover the rows whole.
// * QK: v_mfma_f32_16x16x32_f16 with A = the K rows exactly as loaded
//   (token n, dims 32 m + 8 jq .. + 7) and B = q (query head n, same dims),
//   so C[token][head] lands as lane (head n, jq): tokens 4 jq .. 4 jq + 3.
// * PV: v_mfma_f32_16x16x16_f16 with B = P^T, whose layout (lane (head n,
//   jq): tokens 4 jq .. + 3) is exactly the lane's own softmax values, and
//   A = V^T (dims x tokens) read back from a per-wave LDS copy of the page
//   (rows padded by 4 halves, so the four 4-token groups of a read hit
//   different banks).  P is rounded to fp16 for the product, as the
//   reference kernel does (fused_attention.py:339).
// * One page ahead is in flight per wave (two register sets); four
//   workgroups fit on a CU.
// * Tokens past seq_len in the last page: their logits are masked to -inf
//   and their V rows are written to LDS as zeros, so garbage (NaN) in the
//   unused slots never reaches the output.
// * Split-KV: sequences longer than one chunk publish (m, l, o / l) per
//   query head with device-coherent stores; the last chunk of each (b, j) to
//   arrive merges them and resets its arrival counter.
#include <cstdlib>

#include "common.h"
#include "decode_fp16_stream.h"
#include "iris_hip.h"

namespace iris {
namespace f16 {

constexpr int kPage = 16;
constexpr int kWaves = 4;
constexpr int kPad = 4;           // halves of padding per LDS V row
constexpr int kMaxMergeChunks = 512;
constexpr int kMaxChunkPages = kWaves * 64;  // a wave's page ids fill one VGPR
constexpr int kSC1 = 16;          // cache-policy bit sc1: device-coherent access
constexpr int kNT = 2;            // cache-policy bit nt: streaming (each page is read once)

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float2v_t __attribute__((ext_vector_type(2)));

struct Args {
    const half_t* q;
    const half_t* k;
    const half_t* v;
    const int32_t* block_table;
    const int32_t* seq_lens;
    void* out;
    uint32_t* counters;  // counter j of sequence b at b * kCountersPerSeq + j; zero between calls
    float* ws_o;         // [B][Hkv][max_chunks][g][D] chunk o / l
    float* ws_ml;        // [B][Hkv][max_chunks][g][2] chunk (m, l), base-2 logits
    int out_f32;
    int batch, n_q_heads, n_kv_heads, group;
    int max_pages, max_chunks, chunk_pages;
    float log2_scale;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// v_permlane32_swap / v_permlane16_swap (the s_nop covers the VALU-write ->
// permlane-read hazard).
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// Max / sum over the four 16-lane rows (lanes n, n + 16, n + 32, n + 48).
__device__ __forceinline__ float rows_max(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    swap32(a, b);
    uint32_t c = __builtin_bit_cast(uint32_t, fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)));
    uint32_t d = c;
    swap16(c, d);
    return fmaxf(__builtin_bit_cast(float, c), __builtin_bit_cast(float, d));
}
__device__ __forceinline__ float rows_sum(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    swap32(a, b);
    uint32_t c = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b));
    uint32_t d = c;
    swap16(c, d);
    return __builtin_bit_cast(float, c) + __builtin_bit_cast(float, d);
}

template <int D>
struct Layout {
    static constexpr int ROW = D + kPad;                    // LDS V row, halves
    static constexpr int PAGE_LDS = kPage * ROW * 2;        // bytes per wave
    static constexpr int EPI = (32 + 16 * D) * 4;           // per wave: m[16], l[16], o[16][D]
    static constexpr int MERGE = (kMaxMergeChunks * 16 + 32) * 4;
    static constexpr int LDS = (kWaves * EPI > kWaves * PAGE_LDS ? kWaves * EPI : kWaves * PAGE_LDS) > MERGE
                                   ? (kWaves * EPI > kWaves * PAGE_LDS ? kWaves * EPI : kWaves * PAGE_LDS)
                                   : MERGE;
};

template <int D>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(4)))
void fp16_decode_kernel(Args a) {
    constexpr int NM = D / 32;  // QK products per page (32 dims each)
    constexpr int NC = D / 16;  // PV products per page (16 dims each)
    using L = Layout<D>;
    __shared__ __align__(16) uint8_t smem[L::LDS];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, jq = lane >> 4;

    // kv head fastest: the Hkv workgroups of a chunk read their slices of
    // the same pages side by side (MI355X, B=32, L=4096: 120.9 us against
    // 122.8 with the chunks of one head adjacent); chunk slowest, sequences
    // rotated by the chunk (rotate_back in common.h).
    const int wg = blockIdx.x;
    const int j = wg % a.n_kv_heads;
    const int chunk = wg / a.n_kv_heads / a.batch;
    const int b = rotate_back((wg / a.n_kv_heads) % a.batch, chunk, a.batch);
    const int bj = b * a.n_kv_heads + j;
    const int g = a.group;

    const int seq_len = a.seq_lens[b];
    const int n_pages = (seq_len + kPage - 1) / kPage;
    const int p_begin = chunk * a.chunk_pages;
    if (p_begin >= n_pages) return;  // uniform over the workgroup
    const int p_end = min(p_begin + a.chunk_pages, n_pages);
    const int n_chunks = (n_pages + a.chunk_pages - 1) / a.chunk_pages;

    // q as the B operand of QK: lane (head n, jq), dims 32 m + 8 jq .. + 7.
    const bool col_valid = n < g;
    half8_t qb[NM];
    {
        const half_t* qrow = a.q + ((int64_t)b * a.n_q_heads + j * g + (col_valid ? n : 0)) * D + 8 * jq;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            u32x4_t raw = {0, 0, 0, 0};
            if (col_valid) raw = *reinterpret_cast<const u32x4_t*>(qrow + 32 * m);
            qb[m] = __builtin_bit_cast(half8_t, raw);
        }
    }

    // Page ids of this wave's pages p_begin + wave + 4 t, lane t (a chunk
    // holds at most 4 x 64 pages).
    const int32_t* bt = a.block_table + (int64_t)b * a.max_pages;
    const int first = p_begin + wave;
    int pid = 0;
    if (first + kWaves * lane < p_end) pid = bt[first + kWaves * lane];
    const int64_t row_stride = (int64_t)a.n_kv_heads * D;  // halves between token rows
    // Page `lp` of this chunk into (kr, vr): this lane's 16 bytes per 32 dims
    // of token n.  A page past the chunk gets a buffer of size 0: its loads
    // return zeros without a memory access, so every iteration issues the
    // same loads.
    const uint32_t page_bytes = (uint32_t)(kPage * row_stride * 2);
    const uint32_t voff = (uint32_t)(((int64_t)n * row_stride + (int64_t)j * D + 8 * jq) * 2);
    auto load_page = [&](int lp, u32x4_t (&kr)[NM], u32x4_t (&vr)[NM]) __attribute__((always_inline)) {
        const bool ok = lp < p_end;
        const int64_t base = (int64_t)__builtin_amdgcn_readlane(pid, min((lp - first) / kWaves, 63)) * kPage * row_stride;
        const auto rk = rsrc(a.k + base, ok ? page_bytes : 0u), rv = rsrc(a.v + base, ok ? page_bytes : 0u);
#pragma unroll
        for (int m = 0; m < NM; ++m)
            kr[m] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, voff + 64 * m, 0, kNT));
#pragma unroll
        for (int m = 0; m < NM; ++m)
            vr[m] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, voff + 64 * m, 0, kNT));
    };

    half_t* const vl = reinterpret_cast<half_t*>(smem + wave * L::PAGE_LDS);
    const float c = a.log2_scale;
    float m_run = -INFINITY;  // running max of the base-2 logits (s * c)
    float l_part = 0.0f;      // this lane's share of the softmax denominator
    float4_t o[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) o[k] = float4_t{0, 0, 0, 0};

    auto compute = [&](int lp, const u32x4_t (&kr)[NM], const u32x4_t (&vr)[NM]) __attribute__((always_inline)) {
        const int tok0 = lp * kPage;
        const int valid = seq_len - tok0;  // >= 1; tokens >= valid are masked
        // V rows to LDS (zeros for tokens past the sequence).
        const bool row_ok = n < valid;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const u32x4_t x = row_ok ? vr[m] : u32x4_t{0, 0, 0, 0};
            u32x2_t* dst = reinterpret_cast<u32x2_t*>(vl + n * L::ROW + 32 * m + 8 * jq);
            dst[0] = u32x2_t{x[0], x[1]};
            dst[1] = u32x2_t{x[2], x[3]};
        }
        // S = K q^T: lane (head n, jq) holds tokens 4 jq + i.
        float4_t acc = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < NM; ++m)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, kr[m]), qb[m], acc, 0, 0, 0);
        float s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = 4 * jq + i < valid ? acc[i] * c : -INFINITY;
        const float mx = rows_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));  // finite: token 0 is valid
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first page
        m_run = m_new;
        half4_t pb;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(s[i] - m_new);
            psum += p;
            pb[i] = (half_t)p;
        }
        l_part = l_part * alpha + psum;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // O^T += V^T P^T per 16 dims: lane (dim 16 k + n, jq) supplies tokens
        // 4 jq .. 4 jq + 3 of its dim.
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            half4_t va;
#pragma unroll
            for (int i = 0; i < 4; ++i) va[i] = vl[(4 * jq + i) * L::ROW + 16 * k + n];
            o[k] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb, o[k] * alpha, 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    };

    // ---- the page loop: pages p_begin + wave + 4 t, one page ahead in flight.
    if (first < p_end) {
        u32x4_t ka[NM], va_[NM], kb[NM], vb[NM];
        load_page(first, ka, va_);
        for (int lp = first; lp < p_end; lp += 2 * kWaves) {
            load_page(lp + kWaves, kb, vb);
            compute(lp, ka, va_);
            if (lp + kWaves >= p_end) break;
            load_page(lp + 2 * kWaves, ka, va_);
            compute(lp + kWaves, kb, vb);
        }
    }
    l_part = rows_sum(l_part);

    // ---- merge the four waves in LDS: per wave m[16], l[16], o[16][D]
    // (m in base-2 logit units, o unnormalised).
    __syncthreads();
    float* const ep = reinterpret_cast<float*>(smem + wave * L::EPI);
    if (jq == 0) {
        ep[n] = m_run;
        ep[16 + n] = l_part;
    }
#pragma unroll
    for (int k = 0; k < NC; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) ep[32 + n * D + 16 * k + 4 * jq + i] = o[k][i];
    __syncthreads();

    const int total = g * D, n4 = total / 4;
    auto chunk4 = [&](int e4, float& mstar, float& lsum) -> float4_t {
        const int h = 4 * e4 / D, d = 4 * e4 - h * D;
        mstar = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mstar = fmaxf(mstar, reinterpret_cast<const float*>(smem + w * L::EPI)[h]);
        lsum = 0.0f;
        float4_t acc = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float* wp = reinterpret_cast<const float*>(smem + w * L::EPI);
            const float f = __builtin_amdgcn_exp2f(wp[h] - mstar);  // 0 for an idle wave
            lsum += wp[16 + h] * f;
            acc += *reinterpret_cast<const float4_t*>(wp + 32 + h * D + d) * f;
        }
        return acc * (1.0f / lsum);
    };
    const int64_t out_base = ((int64_t)b * a.n_q_heads + (int64_t)j * g) * D;
    auto store_out4 = [&](int e4, float4_t x) {
        if (a.out_f32) {
            *reinterpret_cast<float4_t*>(reinterpret_cast<float*>(a.out) + out_base + 4 * e4) = x;
        } else {
            const half2_t lo = {(half_t)x[0], (half_t)x[1]}, hi = {(half_t)x[2], (half_t)x[3]};
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

    // ---- split-KV: publish this chunk with device-coherent (sc1) stores,
    // then the last chunk of (b, j) to arrive merges all of them.
    const int64_t row0 = (int64_t)bj * a.max_chunks;
    const uint32_t part_o = (uint32_t)total * 4, part_ml = (uint32_t)g * 8;
    {
        const auto ro = rsrc(a.ws_o + (row0 + chunk) * total, part_o);
        const auto rm = rsrc(a.ws_ml + (row0 + chunk) * g * 2, part_ml);
        for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
            float mstar, lsum;
            const float4_t x = chunk4(e4, mstar, lsum);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, x), ro, (uint32_t)e4 * 16, 0, kSC1);
            if ((4 * e4) % D == 0)
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, float2v_t{mstar, lsum}), rm,
                                                      (uint32_t)(4 * e4 / D) * 8, 0, kSC1);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    uint32_t* const ctl = reinterpret_cast<uint32_t*>(smem);
    if (threadIdx.x == 0)
        ctl[0] = arrive_last(a.counters + (int64_t)b * kCountersPerSeq + j, (uint32_t)n_chunks) ? 1u : 0u;
    __syncthreads();
    if (ctl[0] == 0) return;
    __syncthreads();  // ctl is overwritten by the merge weights below

    // Merge weights w[c][h] = l_c 2^(m_c - m*) / L in LDS, a thread per
    // (head, chunk) with the chunks of a head in adjacent lanes.
    const int M = n_chunks;
    const auto ro = rsrc(a.ws_o + row0 * total, part_o * M);
    const auto rm = rsrc(a.ws_ml + row0 * g * 2, part_ml * M);
    float* const wts = reinterpret_cast<float*>(smem);  // [M][g]
    for (int h0 = 0; h0 < g; ++h0) {
        float mstar = -INFINITY;
        for (int c0 = 0; c0 < M; c0 += (int)blockDim.x) {
            const int cc = c0 + (int)threadIdx.x;
            const float2v_t ml = cc < M ? __builtin_bit_cast(float2v_t, __builtin_amdgcn_raw_buffer_load_b64(
                                                                             rm, (uint32_t)(cc * g + h0) * 8, 0, kSC1))
                                        : float2v_t{-INFINITY, 0.0f};
            mstar = fmaxf(mstar, ml[0]);
        }
        // block max of mstar
        for (int off = 32; off > 0; off >>= 1) mstar = fmaxf(mstar, __shfl_xor(mstar, off, 64));
        float* const red = wts + kMaxMergeChunks * 16;
        if (lane == 0) red[wave] = mstar;
        __syncthreads();
        mstar = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        float lsum = 0.0f;
        for (int c0 = 0; c0 < M; c0 += (int)blockDim.x) {
            const int cc = c0 + (int)threadIdx.x;
            if (cc < M) {
                const float2v_t ml = __builtin_bit_cast(
                    float2v_t, __builtin_amdgcn_raw_buffer_load_b64(rm, (uint32_t)(cc * g + h0) * 8, 0, kSC1));
                const float w = ml[1] * __builtin_amdgcn_exp2f(ml[0] - mstar);
                wts[cc * g + h0] = w;
                lsum += w;
            }
        }
        for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off, 64);
        if (lane == 0) red[4 + wave] = lsum;
        __syncthreads();
        lsum = red[4] + red[5] + red[6] + red[7];
        const float inv = 1.0f / lsum;
        for (int cc = threadIdx.x; cc < M; cc += blockDim.x) wts[cc * g + h0] *= inv;
        __syncthreads();
    }
    constexpr int CB = 8;
    for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
        const int h = 4 * e4 / D;
        float4_t acc = {0, 0, 0, 0};
        for (int c0 = 0; c0 < M; c0 += CB) {
            float4_t oc[CB];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                oc[cb] = float4_t{0, 0, 0, 0};
                if (c0 + cb < M)
                    oc[cb] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                              ro, (uint32_t)(c0 + cb) * part_o + (uint32_t)e4 * 16, 0, kSC1));
            }
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                if (c0 + cb < M) acc += oc[cb] * wts[(c0 + cb) * g + h];
        }
        store_out4(e4, acc);
    }
}

}  // namespace f16

// ------------------------------------------------------------------ host side

namespace {

// [counters: counter_region_bytes(B)][o: B * Hkv * max_chunks * g * D fp32][(m, l)]; a split
// needs Hkv <= kCountersPerSeq.
int64_t f16_workspace_bytes(int64_t batch, int64_t hq, int64_t hkv, int64_t head_dim, int64_t max_chunks) {
    const int64_t g = hq / hkv;
    const int64_t o = batch * hkv * max_chunks * g * head_dim * 4;
    const int64_t ml = batch * hkv * max_chunks * g * 2 * 4;
    return counter_region_bytes(batch) + (o + 255) / 256 * 256 + ml;
}

}  // namespace

}  // namespace iris

using namespace iris;

// Split plan of the FP16 decode: pages per chunk, chunks per sequence and
// workspace bytes.  The page-streaming kernel (decode_fp16_stream.hip) takes
// its shapes for batches of similar lengths with enough work (at least 8
// sequences and 64 MB of K/V, fp16_stream_preferred; unknown lengths count as
// the widest batch), with about one workgroup of all kv heads a CU; its plan
// has a negative chunk_pages.  Ragged batches and the other shapes get the
// per-kv-head kernel's plan: about 1024 workgroups (four per CU), at least 8
// pages (two per wave) each; one chunk when the longest sequence fits.  Both
// kernels' workspaces have the same size for the same chunk count.
extern "C" int iris_fp16_decode_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                     int64_t head_dim, int64_t max_pages, int64_t total_tokens,
                                     int64_t max_tokens, int32_t tokens_per_split, int32_t* out_chunk_pages,
                                     int32_t* out_max_chunks, int64_t* out_workspace_bytes) {
    if (batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
        num_q_heads / num_kv_heads > 16 || (head_dim != 64 && head_dim != 128) || max_pages <= 0)
        return kInvalidArgument;
    const int64_t cap_tokens = max_pages * f16::kPage;
    if (max_tokens < 0 || max_tokens > cap_tokens) max_tokens = cap_tokens;
    if (total_tokens < 0) total_tokens = batch * max_tokens;
    // A negative tokens_per_split asks for the page-streaming kernel with
    // chunks of -tokens_per_split tokens (A/B runs and tests).
    const bool ask_stream = tokens_per_split < 0;
    if (ask_stream) {
        if (!fp16_stream_supported(num_q_heads, num_kv_heads, head_dim) || tokens_per_split == INT32_MIN)
            return kInvalidArgument;
        tokens_per_split = -tokens_per_split;
    }
    if (fp16_stream_supported(num_q_heads, num_kv_heads, head_dim) &&
        (ask_stream || fp16_stream_preferred(batch, num_kv_heads, head_dim, total_tokens, max_tokens)) &&
        fp16_stream_plan(batch, max_pages, total_tokens, max_tokens, tokens_per_split, out_chunk_pages,
                         out_max_chunks) == kOk) {
        *out_workspace_bytes =
            *out_max_chunks > 1 ? fp16_stream_workspace_bytes(batch, num_q_heads, head_dim, *out_max_chunks) : 0;
        *out_chunk_pages = -*out_chunk_pages;  // negative: the page-streaming kernel
        return kOk;
    }
    if (ask_stream) return kInvalidArgument;  // chunks longer than 128 pages
    int64_t chunk_pages;
    if (tokens_per_split > 0) {
        chunk_pages = (tokens_per_split + f16::kPage - 1) / f16::kPage;
    } else {
        const int64_t units = ((total_tokens + f16::kPage - 1) / f16::kPage + batch) * num_kv_heads;
        chunk_pages = (units + 1023) / 1024;
        if (chunk_pages < 8) chunk_pages = 8;
        const int64_t longest = (max_tokens + f16::kPage - 1) / f16::kPage;
        const int64_t pieces = (longest + chunk_pages - 1) / chunk_pages;
        if (pieces > 0) chunk_pages = (longest + pieces - 1) / pieces;
    }
    if (chunk_pages < 1) chunk_pages = 1;
    if (chunk_pages >= (max_tokens + f16::kPage - 1) / f16::kPage) chunk_pages = max_pages;
    if (chunk_pages > f16::kMaxChunkPages) chunk_pages = f16::kMaxChunkPages;
    // The grid covers every page block_table can address; the merge holds
    // the weights of at most kMaxMergeChunks chunks.
    int64_t max_chunks = (max_pages + chunk_pages - 1) / chunk_pages;
    if (max_chunks > f16::kMaxMergeChunks) {
        chunk_pages = (max_pages + f16::kMaxMergeChunks - 1) / f16::kMaxMergeChunks;
        max_chunks = (max_pages + chunk_pages - 1) / chunk_pages;
    }
    if (chunk_pages > f16::kMaxChunkPages) return kInvalidArgument;  // block_table too wide
    if (max_chunks > 1 && num_kv_heads > kCountersPerSeq) return kInvalidArgument;
    *out_chunk_pages = (int32_t)chunk_pages;
    *out_max_chunks = (int32_t)max_chunks;
    *out_workspace_bytes =
        max_chunks > 1 ? f16_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, max_chunks) : 0;
    return kOk;
}

extern "C" int iris_fp16_paged_decode_attention(const void* query, const void* k_cache, const void* v_cache,
                                                const int32_t* block_table, const int32_t* seq_lens, void* output,
                                                int32_t output_is_f32, void* workspace,
                                                int64_t workspace_bytes_avail, int64_t batch, int64_t num_q_heads,
                                                int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                                int64_t num_pages, int64_t max_pages, float softmax_scale,
                                                int32_t chunk_pages, int32_t max_chunks, void* stream) {
    (void)num_pages;
    if (page_size != f16::kPage || batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
        num_q_heads / num_kv_heads > 16 || (head_dim != 64 && head_dim != 128) || max_pages <= 0)
        return kInvalidArgument;
    // A negative chunk_pages: the page-streaming kernel's plan.
    if (chunk_pages < 0) {
        const int64_t cp = -(int64_t)chunk_pages;
        if (cp > 0x7FFFFFFF) return kInvalidArgument;
        return fp16_stream_launch(query, k_cache, v_cache, block_table, seq_lens, output, output_is_f32, workspace,
                                  workspace_bytes_avail, batch, num_q_heads, num_kv_heads, head_dim, max_pages,
                                  softmax_scale, (int32_t)cp, max_chunks, stream);
    }
    if (chunk_pages <= 0 || chunk_pages > f16::kMaxChunkPages || max_chunks <= 0 || max_chunks > f16::kMaxMergeChunks ||
        (int64_t)chunk_pages * max_chunks < max_pages)
        return kInvalidArgument;
    f16::Args a;
    a.q = (const half_t*)query;
    a.k = (const half_t*)k_cache;
    a.v = (const half_t*)v_cache;
    a.block_table = block_table;
    a.seq_lens = seq_lens;
    a.out = output;
    a.out_f32 = output_is_f32;
    a.batch = (int)batch;
    a.n_q_heads = (int)num_q_heads;
    a.n_kv_heads = (int)num_kv_heads;
    a.group = (int)(num_q_heads / num_kv_heads);
    a.max_pages = (int)max_pages;
    a.max_chunks = max_chunks;
    a.chunk_pages = chunk_pages;
    a.log2_scale = softmax_scale * 1.4426950408889634f;
    a.counters = nullptr;
    a.ws_o = a.ws_ml = nullptr;
    if (max_chunks > 1) {
        if (num_kv_heads > kCountersPerSeq) return kInvalidArgument;
        const int64_t need = f16_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, max_chunks);
        if (workspace == nullptr || workspace_bytes_avail < need) return kWorkspaceTooSmall;
        const int64_t g = num_q_heads / num_kv_heads;
        uint8_t* const ws = (uint8_t*)workspace;
        a.counters = (uint32_t*)ws;
        a.ws_o = (float*)(ws + counter_region_bytes(batch));
        const int64_t o = batch * num_kv_heads * max_chunks * g * head_dim * 4;
        a.ws_ml = (float*)(ws + counter_region_bytes(batch) + (o + 255) / 256 * 256);
    }
    const int64_t nblocks = batch * num_kv_heads * (int64_t)max_chunks;
    if (nblocks > 0x7FFFFFFF) return kInvalidArgument;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((unsigned)nblocks), block(64 * f16::kWaves);
    if (head_dim == 128)
        hipLaunchKernelGGL(f16::fp16_decode_kernel<128>, grid, block, 0, s, a);
    else
        hipLaunchKernelGGL(f16::fp16_decode_kernel<64>, grid, block, 0, s, a);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}
