// INT4 paged decode attention for gfx950 (MI355X): the any-shape kernel.
//
// Replaces the TileLang kernel `_int4_paged_decode_attention`
// (src/iris_kernel/fused_attention.py:11-220 in Hunter2030ZeRo/Iris-Kernel)
// for every shape its eager counterpart takes and the other kernels of this
// library do not: head_dim any multiple of 32 up to 512, any page size (one
// token a page, 8, 48, ...), any number of query heads per kv head.  The
// eager path takes all of these (torch_eager_attention.py:72, :93); the
// reference's fused path only page_size 16 and head_dim 64 or 128
// (fused_attention.py:390-403).
//
// Work: a workgroup of 4 waves owns (sequence, kv head, block of up to 16
// of its query heads, chunk of tokens) and walks the chunk in 64-token
// tiles, one token a lane.  Each tile's packed K and V rows (16-byte loads,
// every token's page looked up on its own) and their scales are staged in
// LDS, the V codes transposed (a dword holds four tokens of one dim pair).
// * QK: lane = token; each group's 32 codes are dequantised once as
//   code * scale in fp32, exactly as the eager dequantisation
//   (torch_eager_attention.py:29-53) does, and every query head of the wave
//   takes its fp32 dot product against them (the query rows broadcast from
//   LDS).  So non-finite scales behave as in the eager path: 0 * inf = NaN,
//   products of mixed signs NaN, one sign +-inf.
// * fp32 online softmax in base 2 per query head (wave-wide maxima), guarded
//   so a tile of -inf logits drops out instead of making 0 * inf.
// * PV: lane = dim pair; V dequantised once per (token, pair), fp32 FMAs
//   with every query head's weights (broadcast from LDS).
// Split-KV: chunks publish (o / l, m, l) per query head with device-coherent
// stores; the last to arrive merges them in chunk order (the protocol of
// arrive_last in common.h).
#include "common.h"
#include "decode_any.h"
#include "iris_hip.h"

namespace iris {
namespace an {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTok = 64;       // tokens a tile, one a lane
constexpr int kMergeBatch = 8;  // partials a merge round trip loads
constexpr int kMaxHeads = 16;  // query heads a workgroup: a block of its kv head's
constexpr int kHeadsPerWave = kMaxHeads / kWaves;
constexpr int kMaxDim = 512;
constexpr int kPairSlots = kMaxDim / 2 / 64;  // dim pairs a lane covers at head_dim 512
constexpr int kVtRow = kTok + 4;              // bytes a transposed V row (padded: no bank conflicts)
constexpr int kSC1 = 16;                      // cache-policy bit sc1: device-coherent access

struct Args {
    const half_t* q;
    const uint8_t* k_data;
    const uint8_t* v_data;
    const half_t* k_scale;
    const half_t* v_scale;
    const int32_t* block_table;
    const int32_t* seq_lens;
    void* out;
    uint32_t* counters;  // sequence b's at b * kCountersPerSeq; zero between calls
    float* part_o;       // [B][max_chunks][Hq][D] o / l of each chunk
    float* part_ml;      // [B][max_chunks][Hq][2] (m, l), base-2 logits
    int out_f32;
    int batch, n_q_heads, n_kv_heads, group, q_blocks, head_dim, page_size, bt_cols;
    int chunk_tok, max_chunks;
    float log2_scale;  // softmax_scale * log2(e)
};

// Byte offsets of the LDS areas for head_dim D (host and device).
struct Lds {
    int q, kc, vt, ks, vs, p, total;
};
__host__ __device__ constexpr int kc_row(int G) { return 16 * G + 16; }  // K codes of a token, padded
__host__ __device__ inline Lds lds_layout(int D) {
    const int G = D / 32;
    Lds L{};
    L.q = 0;                                // [16][D] fp32 query rows
    L.kc = L.q + kMaxHeads * D * 4;         // [64][kc_row] u8 K codes
    L.vt = L.kc + kTok * kc_row(G);         // [D/2][kVtRow] u8 V codes, pair-major
    L.ks = L.vt + (D / 2) * kVtRow;         // [64][G + 1] fp32 K scales
    L.vs = L.ks + kTok * (G + 1) * 4;       // [G][64] fp32 V scales, group-major
    L.p = L.vs + G * kTok * 4;              // [16][64] fp32 softmax weights of the tile
    L.total = (L.p + kMaxHeads * kTok * 4 + 15) / 16 * 16;
    return L;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}
// Signed INT4 code n (0..7) of a dword, low nibble first.
__device__ __forceinline__ float nib(uint32_t w, int n) { return (float)((int32_t)(w << (28 - 4 * n)) >> 28); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

__global__ __launch_bounds__(kThreads) void int4_decode_any_kernel(Args a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int D = a.head_dim, G = D >> 5, P = a.page_size;
    const Lds L = lds_layout(D);
    float* const q_s = reinterpret_cast<float*>(smem + L.q);
    uint8_t* const kc_s = smem + L.kc;
    uint8_t* const vt_s = smem + L.vt;
    float* const ks_s = reinterpret_cast<float*>(smem + L.ks);
    float* const vs_s = reinterpret_cast<float*>(smem + L.vs);
    float* const p_s = reinterpret_cast<float*>(smem + L.p);
    const int SK = kc_row(G);

    // ---- (chunk, sequence, kv head, query block), chunks slowest, the
    // sequences rotated by the chunk (rotate_back in common.h)
    int rest = blockIdx.x;
    const int qb = rest % a.q_blocks;
    rest /= a.q_blocks;
    const int kvh = rest % a.n_kv_heads;
    rest /= a.n_kv_heads;
    const int chunk = rest / a.batch;
    const int b = rotate_back(rest % a.batch, chunk, a.batch);
    const int seq_len = a.seq_lens[b];
    const int64_t t_begin64 = (int64_t)chunk * a.chunk_tok;
    if (t_begin64 >= seq_len) return;  // uniform: this chunk holds no token
    const int t_begin = (int)t_begin64;
    const int t_end = (int)min((int64_t)seq_len, t_begin64 + a.chunk_tok);
    const int n_chunks = (int)(((int64_t)seq_len + a.chunk_tok - 1) / a.chunk_tok);
    const int h_first = qb * kMaxHeads;
    const int nh = min(a.group - h_first, kMaxHeads);
    const int hq0 = kvh * a.group + h_first;  // the block's first query head

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t* const bt = a.block_table + (int64_t)b * a.bt_cols;

    // query rows of the block, fp32 (exact)
    {
        const half_t* const qg = a.q + ((int64_t)b * a.n_q_heads + hq0) * D;
        for (int i = tid; i < nh * D; i += kThreads) q_s[i] = (float)qg[i];
    }

    // per wave: query heads h = wave + 4 k of the block
    float m_run[kHeadsPerWave], l_part[kHeadsPerWave], acc[kHeadsPerWave][kPairSlots][2];
#pragma unroll
    for (int k = 0; k < kHeadsPerWave; ++k) {
        m_run[k] = -INFINITY;
        l_part[k] = 0.0f;
#pragma unroll
        for (int i = 0; i < kPairSlots; ++i) acc[k][i][0] = acc[k][i][1] = 0.0f;
    }
    const int n_pairs = D >> 1;

    for (int t0 = t_begin; t0 < t_end; t0 += kTok) {
        const int nval = min(kTok, t_end - t0);
        __syncthreads();  // the previous tile's reads are done (and the query rows are in)
        // ---- stage the tile: 16-byte piece gi of token tok's K and V rows,
        // and their scales; tokens past the chunk get zeros (never read).
        for (int idx = tid; idx < kTok * G; idx += kThreads) {
            const int tok = idx / G, gi = idx - tok * G;
            u32x4_t kw = {0, 0, 0, 0}, vw = {0, 0, 0, 0};
            float ksf = 0.0f, vsf = 0.0f;
            if (tok < nval) {
                const int t = t0 + tok;
                const int e = t / P;  // block-table entry and token of its page
                const int64_t row = ((int64_t)bt[e] * P + (t - e * P)) * a.n_kv_heads + kvh;
                kw = *reinterpret_cast<const u32x4_t*>(a.k_data + row * (16 * G) + 16 * gi);
                vw = *reinterpret_cast<const u32x4_t*>(a.v_data + row * (16 * G) + 16 * gi);
                ksf = (float)a.k_scale[row * G + gi];
                vsf = (float)a.v_scale[row * G + gi];
            }
            *reinterpret_cast<u32x4_t*>(kc_s + tok * SK + 16 * gi) = kw;
            ks_s[tok * (G + 1) + gi] = ksf;
            vs_s[gi * kTok + tok] = vsf;
#pragma unroll
            for (int j = 0; j < 16; ++j) vt_s[(16 * gi + j) * kVtRow + tok] = (uint8_t)(vw[j >> 2] >> (8 * (j & 3)));
        }
        __syncthreads();

        // ---- QK: lane = token; the group's K values dequantised once
        const bool valid = lane < nval;
        float s[kHeadsPerWave];
#pragma unroll
        for (int k = 0; k < kHeadsPerWave; ++k) s[k] = 0.0f;
        for (int gi = 0; gi < G; ++gi) {
            const u32x4_t w = *reinterpret_cast<const u32x4_t*>(kc_s + lane * SK + 16 * gi);
            const float sc = ks_s[lane * (G + 1) + gi];
            float kv[32];
#pragma unroll
            for (int d = 0; d < 32; ++d) kv[d] = nib(w[d >> 3], d & 7) * sc;
#pragma unroll
            for (int k = 0; k < kHeadsPerWave; ++k) {
                const int h = wave + kWaves * k;
                if (h < nh) {  // uniform over the wave
                    const float4_t* const qr = reinterpret_cast<const float4_t*>(q_s + h * D + 32 * gi);
#pragma unroll
                    for (int d4 = 0; d4 < 8; ++d4) {
                        const float4_t qv = qr[d4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) s[k] = __builtin_fmaf(qv[u], kv[4 * d4 + u], s[k]);
                    }
                }
            }
        }

        // ---- online softmax per query head (base 2)
#pragma unroll
        for (int k = 0; k < kHeadsPerWave; ++k) {
            const int h = wave + kWaves * k;
            if (h >= nh) continue;
            const float x = valid ? s[k] * a.log2_scale : -INFINITY;
            const float m_new = fmaxf(m_run[k], wave_max(x));
            // a tile (and all before it) of -inf logits: weights 0, no rescale
            const bool none = m_new == -INFINITY;
            const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_run[k] - m_new);
            const float p = none ? 0.0f : __builtin_amdgcn_exp2f(x - m_new);
            m_run[k] = m_new;
            l_part[k] = l_part[k] * alpha + p;
#pragma unroll
            for (int i = 0; i < kPairSlots; ++i) {
                acc[k][i][0] *= alpha;
                acc[k][i][1] *= alpha;
            }
            p_s[h * kTok + lane] = p;
        }
        __syncthreads();

        // ---- PV: lane = dim pair (pairs lane + 64 i); four tokens a step
        // (tokens past the chunk: weight 0, codes and scales 0)
        const int nval4 = (nval + 3) & ~3;
#pragma unroll
        for (int i = 0; i < kPairSlots; ++i) {
            const int j = lane + 64 * i;
            if (64 * i >= n_pairs) break;  // uniform
            if (j >= n_pairs) continue;
            const uint8_t* const vrow = vt_s + j * kVtRow;
            const float* const vsr = vs_s + (j >> 4) * kTok;  // dims 2j, 2j + 1: group j / 16
            for (int t4 = 0; t4 < nval4; t4 += 4) {
                const uint32_t cb = *reinterpret_cast<const uint32_t*>(vrow + t4);
                const float4_t vsc = *reinterpret_cast<const float4_t*>(vsr + t4);
                float v0[4], v1[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    v0[u] = nib(cb, 2 * u) * vsc[u];
                    v1[u] = nib(cb, 2 * u + 1) * vsc[u];
                }
#pragma unroll
                for (int k = 0; k < kHeadsPerWave; ++k) {
                    const int h = wave + kWaves * k;
                    if (h < nh) {
                        const float4_t pv = *reinterpret_cast<const float4_t*>(p_s + h * kTok + t4);
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            acc[k][i][0] = __builtin_fmaf(pv[u], v0[u], acc[k][i][0]);
                            acc[k][i][1] = __builtin_fmaf(pv[u], v1[u], acc[k][i][1]);
                        }
                    }
                }
            }
        }
    }

    // ---- the chunk's result per query head: o / l, and (m, l)
    const int hq = a.n_q_heads;
    const int64_t seq_rows = (int64_t)a.max_chunks * hq;  // partial rows of a sequence
    const auto ro = buf_rsrc(a.part_o + (int64_t)b * seq_rows * D, (uint32_t)(seq_rows * D * 4));
    const auto rm = buf_rsrc(a.part_ml + (int64_t)b * seq_rows * 2, (uint32_t)(seq_rows * 8));
#pragma unroll
    for (int k = 0; k < kHeadsPerWave; ++k) {
        const int h = wave + kWaves * k;
        if (h >= nh) continue;
        const float l = wave_sum(l_part[k]);
        const int qh = hq0 + h;
        for (int i = 0; i < kPairSlots; ++i) {
            const int j = lane + 64 * i;
            if (64 * i >= n_pairs) break;
            if (j >= n_pairs) continue;
            // A chunk whose logits are all -inf (l = 0) publishes o = 0, not
            // 0 / 0: the merge gives it weight 0, and 0 * NaN would poison a
            // sequence whose other tokens are finite.  Alone, 0 / 0 is NaN,
            // as the eager softmax of -inf logits is.
            const float inv = (n_chunks > 1 && l == 0.0f) ? 0.0f : 1.0f / l;
            const float o0 = n_chunks == 1 ? acc[k][i][0] / l : acc[k][i][0] * inv;
            const float o1 = n_chunks == 1 ? acc[k][i][1] / l : acc[k][i][1] * inv;
            if (n_chunks == 1) {
                const int64_t at = ((int64_t)b * hq + qh) * D + 2 * j;
                if (a.out_f32) {
                    reinterpret_cast<float*>(a.out)[at] = o0;
                    reinterpret_cast<float*>(a.out)[at + 1] = o1;
                } else {
                    *reinterpret_cast<half2_t*>(reinterpret_cast<half_t*>(a.out) + at) = half2_t{(half_t)o0, (half_t)o1};
                }
            } else {
                const uint32_t off = (uint32_t)((((int64_t)chunk * hq + qh) * D + 2 * j) * 4);
                __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{as_u32(o0), as_u32(o1)}, ro, off, 0, kSC1);
            }
        }
        if (n_chunks > 1 && lane == 0) {
            const uint32_t off = (uint32_t)(((int64_t)chunk * hq + qh) * 8);
            __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{as_u32(m_run[k]), as_u32(l)}, rm, off, 0, kSC1);
        }
    }
    if (n_chunks == 1) return;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // (the flag lives in the weights area, free after the last tile: no
    // static LDS, so the whole 160 KiB stays available as dynamic LDS)
    uint32_t* const last = reinterpret_cast<uint32_t*>(p_s);
    if (tid == 0)
        *last = arrive_last(a.counters + (int64_t)b * kCountersPerSeq + kvh * a.q_blocks + qb, (uint32_t)n_chunks) ? 1u : 0u;
    __syncthreads();
    if (*last == 0) return;

    // ---- merge the chunks in order: o = sum_c w_c (o / l)_c / sum_c w_c,
    // w_c = l_c 2^(m_c - m*), m* the running maximum; the partials of
    // kMergeBatch chunks loaded together (one round trip a batch)
    for (int e = tid; e < nh * D; e += kThreads) {
        const int h = e / D, d = e - h * D, qh = hq0 + h;
        float mstar = -INFINITY, lsum = 0.0f, o = 0.0f;
        for (int c0 = 0; c0 < n_chunks; c0 += kMergeBatch) {
            u32x2_t ml[kMergeBatch];
            float oc[kMergeBatch];
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                const int c = min(c0 + j, n_chunks - 1);
                ml[j] = __builtin_amdgcn_raw_buffer_load_b64(rm, (uint32_t)(((int64_t)c * hq + qh) * 8), 0, kSC1);
                oc[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                      ro, (uint32_t)((((int64_t)c * hq + qh) * D + d) * 4), 0, kSC1));
            }
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                if (c0 + j >= n_chunks) break;  // uniform
                const float mc = as_f32(ml[j][0]), lc = as_f32(ml[j][1]);
                const float mb = fmaxf(mstar, mc);
                const bool none = mb == -INFINITY;
                const float r = none ? 1.0f : __builtin_amdgcn_exp2f(mstar - mb);
                const float w = none ? 0.0f : lc * __builtin_amdgcn_exp2f(mc - mb);
                o = o * r + w * oc[j];
                lsum = lsum * r + w;
                mstar = mb;
            }
        }
        const float res = o / lsum;
        const int64_t at = ((int64_t)b * hq + qh) * D + d;
        if (a.out_f32) reinterpret_cast<float*>(a.out)[at] = res;
        else reinterpret_cast<half_t*>(a.out)[at] = (half_t)res;
    }
}

}  // namespace an

// ------------------------------------------------------------------ host side

namespace {

struct AnyWorkspace {
    int64_t part_o, part_ml, total;
};
AnyWorkspace any_workspace(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t max_chunks) {
    AnyWorkspace w;
    w.part_o = counter_region_bytes(batch);
    w.part_ml = w.part_o + (batch * max_chunks * num_q_heads * head_dim * 4 + 255) / 256 * 256;
    w.total = w.part_ml + batch * max_chunks * num_q_heads * 2 * 4;
    return w;
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

}  // namespace

bool any_supported(int64_t head_dim) { return head_dim >= 32 && head_dim <= an::kMaxDim && head_dim % 32 == 0; }

int any_waves() { return an::kWaves; }

int any_plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t cap_tokens,
             int64_t total_tokens, int64_t max_tokens, int32_t tokens_per_split, int32_t* out_chunk_tiles,
             int32_t* out_max_chunks, int64_t* out_workspace_bytes) {
    if (!any_supported(head_dim) || batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
        cap_tokens <= 0 || cap_tokens > 0x7FFFFFFF)
        return kInvalidArgument;
    (void)total_tokens;
    const int64_t g = num_q_heads / num_kv_heads;
    const int64_t q_blocks = (g + an::kMaxHeads - 1) / an::kMaxHeads;
    const int64_t units = batch * num_kv_heads * q_blocks;
    if (max_tokens < 0 || max_tokens > cap_tokens) max_tokens = cap_tokens;
    if (max_tokens < 1) max_tokens = 1;
    int64_t chunk_tok;
    if (tokens_per_split > 0) {
        chunk_tok = round_up(tokens_per_split, an::kTok);
    } else {
        // About 1024 workgroups (four a CU): as many chunks of the longest
        // sequence as that leaves room for; with fewer than 16 units, no
        // more than 64 partial elements a thread for the merging workgroup
        // (one round trip per kMergeBatch chunks; MI355X, B=1, Hq=16, Hkv=1,
        // D=96, L=16384: 256 chunks 411 us, 10 chunks 279; with more units
        // the workgroups' count matters more: B=4, Hq=64, Hkv=8, D=160,
        // L=32768: 32 chunks 469 us, 12 chunks 599).
        int64_t per = (1024 + units - 1) / units;
        if (per < 1) per = 1;
        const int64_t nh = g < an::kMaxHeads ? g : an::kMaxHeads;
        const int64_t per_thread = (nh * head_dim + an::kThreads - 1) / an::kThreads;
        const int64_t most = 64 / per_thread > 1 ? 64 / per_thread : 1;
        if (units < 16 && per > most) per = most;
        chunk_tok = round_up((max_tokens + per - 1) / per, an::kTok);
    }
    // The arrival counters of a sequence: one per (kv head, query block).
    if (num_kv_heads * q_blocks > kCountersPerSeq) chunk_tok = round_up(cap_tokens, an::kTok);
    int64_t max_chunks = (cap_tokens + chunk_tok - 1) / chunk_tok;
    while (units * max_chunks > 0x7FFFFFFF || max_chunks * num_q_heads * head_dim * 4 > 0x7FFFFFFF) {
        chunk_tok *= 2;
        max_chunks = (cap_tokens + chunk_tok - 1) / chunk_tok;
    }
    if (chunk_tok / 32 > 0x7FFFFFFF) return kInvalidArgument;
    *out_chunk_tiles = (int32_t)(chunk_tok / 32);
    *out_max_chunks = (int32_t)max_chunks;
    *out_workspace_bytes = max_chunks > 1 ? any_workspace(batch, num_q_heads, head_dim, max_chunks).total : 0;
    return kOk;
}

int any_launch(const void* query, const void* k_data, const void* v_data, const void* k_scale, const void* v_scale,
               const int32_t* block_table, const int32_t* seq_lens, void* output, int32_t output_is_f32,
               void* workspace, int64_t workspace_bytes_avail, int64_t batch, int64_t num_q_heads,
               int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t bt_cols, float softmax_scale,
               int32_t chunk_tiles, int32_t max_chunks, void* stream) {
    if (!any_supported(head_dim) || batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
        page_size <= 0 || bt_cols <= 0 || chunk_tiles <= 0 || (chunk_tiles & 1) != 0 || max_chunks <= 0)
        return kInvalidArgument;
    const int64_t cap_tokens = bt_cols * page_size;
    const int64_t chunk_tok = (int64_t)chunk_tiles * 32;
    // every token a block-table row addresses lies in a chunk; 32-bit token
    // indices and partial offsets
    if (cap_tokens > 0x7FFFFFFF || chunk_tok > 0x7FFFFFFF || chunk_tok * max_chunks < cap_tokens ||
        (int64_t)max_chunks * num_q_heads * head_dim * 4 > 0x7FFFFFFF)
        return kInvalidArgument;
    const int64_t g = num_q_heads / num_kv_heads;
    const int64_t q_blocks = (g + an::kMaxHeads - 1) / an::kMaxHeads;
    const int64_t nblocks = batch * num_kv_heads * q_blocks * max_chunks;
    if (nblocks > 0x7FFFFFFF || num_q_heads > 0x7FFFFFFF / head_dim) return kInvalidArgument;
    an::Args a;
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
    a.group = (int)g;
    a.q_blocks = (int)q_blocks;
    a.head_dim = (int)head_dim;
    a.page_size = (int)page_size;
    a.bt_cols = (int)bt_cols;
    a.chunk_tok = (int)chunk_tok;
    a.max_chunks = max_chunks;
    a.log2_scale = softmax_scale * 1.4426950408889634f;
    a.counters = nullptr;
    a.part_o = a.part_ml = nullptr;
    if (max_chunks > 1) {
        if (num_kv_heads * q_blocks > kCountersPerSeq) return kInvalidArgument;
        const AnyWorkspace w = any_workspace(batch, num_q_heads, head_dim, max_chunks);
        if (workspace == nullptr || workspace_bytes_avail < w.total) return kWorkspaceTooSmall;
        uint8_t* const ws = (uint8_t*)workspace;
        a.counters = (uint32_t*)ws;
        a.part_o = (float*)(ws + w.part_o);
        a.part_ml = (float*)(ws + w.part_ml);
    }
    const int lds = an::lds_layout((int)head_dim).total;
    if (lds > kMaxLdsBytes) return kInvalidArgument;
    static std::atomic<uint64_t> lds_raised{0};
    if (lds > 65536 && allow_full_lds(reinterpret_cast<const void*>(&an::int4_decode_any_kernel), lds_raised) != kOk)
        return kLaunchError;
    hipLaunchKernelGGL(an::int4_decode_any_kernel, dim3((unsigned)nblocks), dim3(an::kThreads), lds,
                       (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}

}  // namespace iris
