// FP16 paged decode attention for gfx950 (MI355X): the page-streaming kernel
// of the matched FP16 baseline.
//
// Replaces the TileLang kernel `_fp16_paged_decode_attention`
// (src/iris_kernel/fused_attention.py:223-370 in Hunter2030ZeRo/Iris-Kernel)
// for the shapes whose half-page K and V slabs of every kv head fit a 32 KiB
// LDS slot (head_dim 128 with 4 or 8 kv heads, head_dim 64 with 8 or 16); it
// computes what `torch_eager_fp16_paged_decode_attention`
// (torch_eager_attention.py:242-294) computes.  The other shapes run the
// per-kv-head kernel of decode_fp16.hip.
//
// Streaming
// ---------
// A 16-token page of the fp16 cache [NP, 16, Hkv, D] is one contiguous slab
// of 16 rows (a token's Hkv x D halves each) per tensor.  Read as 256-byte
// head slices by a workgroup per kv head, the configuration-2 cache streams
// at about 4.6 TB/s on MI355X; read as contiguous 4 KiB pieces by the same
// grid, at about 5.9 TB/s.  So:
// * a workgroup owns (sequence, chunk of pages) and has one wave per kv head;
// * a tile is half a page (8 tokens): its K slab and V slab, 8 rows each,
//   fill one LDS slot, written by 1 KiB direct-to-LDS loads (D / 32 a wave);
// * a ring of four slots, three in flight while one is computed, one
//   workgroup barrier a tile (it publishes the slot and frees the one the
//   next load goes to).
// * The 16-byte chunks of a row sit at positions chunk ^ ((row & 3) << 2) in
//   the slot, so the 8 rows' chunks of one kv head spread over the banks.
//
// Compute (wave = kv head j, its g query heads)
// ---------------------------------------------
// * QK: v_mfma_f32_16x16x32_f16 with A = K rows (token n & 7, dims 32 m +
//   8 jq .. + 7; rows 8-15 repeat them and are masked) and B = q (query head
//   n < g); C lane (head n, jq) holds tokens 4 jq + i (jq < 2: the tile's 8).
// * fp32 online softmax in base 2; P rounded to fp16 for the product, as
//   the reference kernel does (fused_attention.py:339).
// * PV: v_mfma_f32_16x16x16_f16 with A = V^T read by ds_read_b64_tr_b16
//   (within each 16-lane group the lanes form 4 rows of 16 halves: lanes
//   4 r .. 4 r + 3 address row r, and lane n receives column n of the 4 rows)
//   and B = P^T, which is the lane's own softmax values.  Rows of tokens
//   outside the tile or past the sequence point at a zero chunk, so garbage
//   (NaN) in unused cache slots never reaches the output.
//
// Split-KV: sequences longer than one chunk publish (o / l, m, l) per query
// head with device-coherent stores; the last chunk to arrive merges them.
#include "common.h"
#include "decode_fp16_stream.h"
#include "iris_hip.h"

namespace iris {
namespace f16s {

constexpr int kPage = 16;
constexpr int kTok = 8;            // tokens a tile (half a page)
constexpr int kSlots = 4;
constexpr int kAhead = 3;          // slots in flight while one is computed
constexpr int kSlotBytes = 32768;  // half-page slabs of K and V, every kv head (Hkv x D <= 1024)
constexpr int kMaxChunkPages = 128;  // a chunk's page ids fill two VGPRs
constexpr int kMaxChunks = 16;     // partials one merge reads
constexpr int kMergeBatch = 8;
constexpr int kSC1 = 16;  // cache-policy bit sc1: device-coherent access
constexpr int kNT = 2;    // cache-policy bit nt: streaming
// LDS: the ring, a zero chunk, the arrival flag.
constexpr int kZeroOff = kSlots * kSlotBytes;
constexpr int kCtlOff = kZeroOff + 16;
constexpr int kLdsBytes = kCtlOff + 16;

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float2v_t __attribute__((ext_vector_type(2)));
#define IRIS_LDS __attribute__((address_space(3)))

struct Args {
    const half_t* q;
    const half_t* k;
    const half_t* v;
    const int32_t* block_table;
    const int32_t* seq_lens;
    void* out;
    uint32_t* counters;  // counter of sequence b at b * kCountersPerSeq; zero between calls
    float* part_o;       // [B][max_chunks][Hq][D] chunk o / l
    float* part_ml;      // [B][max_chunks][Hq][2] chunk (m, l), base-2 logits
    int out_f32;
    int n_q_heads, n_kv_heads, group;
    int max_pages, max_chunks, chunk_pages;
    float log2_scale;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const IRIS_LDS void*)p;
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ int swz(int row) { return (row & 3) << 2; }

// Reads of slot data, which direct-to-LDS loads wrote, are inline assembly
// waiting for their own results (the compiler cannot tell them from the
// loads still streaming into the other slots).  A vmcnt wait and a
// workgroup barrier precede them.
template <int NM>
__device__ __forceinline__ void k_reads(const uint32_t (&addr)[NM], u32x4_t (&k)[NM]) {
    if constexpr (NM == 4) {
        asm volatile(
            "ds_read_b128 %0, %4\n\t"
            "ds_read_b128 %1, %5\n\t"
            "ds_read_b128 %2, %6\n\t"
            "ds_read_b128 %3, %7\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3])
            : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3])
            : "memory");
    } else {
        asm volatile(
            "ds_read_b128 %0, %2\n\t"
            "ds_read_b128 %1, %3\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(k[0]), "=&v"(k[1])
            : "v"(addr[0]), "v"(addr[1])
            : "memory");
    }
}
template <int NC>
__device__ __forceinline__ void v_reads(const uint32_t (&addr)[NC], u32x2_t (&v)[NC]) {
    if constexpr (NC == 8) {
        asm volatile(
            "ds_read_b64_tr_b16 %0, %8\n\t"
            "ds_read_b64_tr_b16 %1, %9\n\t"
            "ds_read_b64_tr_b16 %2, %10\n\t"
            "ds_read_b64_tr_b16 %3, %11\n\t"
            "ds_read_b64_tr_b16 %4, %12\n\t"
            "ds_read_b64_tr_b16 %5, %13\n\t"
            "ds_read_b64_tr_b16 %6, %14\n\t"
            "ds_read_b64_tr_b16 %7, %15\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
              "=&v"(v[7])
            : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "v"(addr[4]), "v"(addr[5]), "v"(addr[6]),
              "v"(addr[7])
            : "memory");
    } else {
        asm volatile(
            "ds_read_b64_tr_b16 %0, %4\n\t"
            "ds_read_b64_tr_b16 %1, %5\n\t"
            "ds_read_b64_tr_b16 %2, %6\n\t"
            "ds_read_b64_tr_b16 %3, %7\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
            : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3])
            : "memory");
    }
}

// Max / sum over the four 16-lane rows (lanes n, n + 16, n + 32, n + 48).
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
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

// The scalars the prologue needs come first, as separate arguments.
template <int D>
__global__ __launch_bounds__(1024) void fp16_decode_stream_kernel(const int32_t* p_seq_lens,
                                                                  const int32_t* p_block_table, int p_max_chunks,
                                                                  int p_chunk_pages, int p_max_pages, int p_hkv,
                                                                  Args a) {
    constexpr int NM = D / 32;   // QK products a tile (32 dims each)
    constexpr int NC = D / 16;   // PV products a tile (16 dims each)
    constexpr int NL = D / 32;   // 1 KiB loads a wave a slot
    constexpr int CPH = D / 8;   // 16-byte chunks of a head's row
    extern __shared__ __align__(16) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // kv head
    const int n = lane & 15, jq = lane >> 4;
    const int hkv = p_hkv;
    const int cpr = hkv * CPH;          // chunks of a token row
    const int rowb = cpr * 16;          // bytes of a token row
    const int g = a.group;

    // chunk slowest, sequences rotated by the chunk (rotate_back in common.h)
    const int batch = gridDim.x / p_max_chunks;
    const int chunk = blockIdx.x / batch, b = rotate_back(blockIdx.x - chunk * batch, chunk, batch);
    const int p0 = chunk * p_chunk_pages;
    const int32_t* bt = p_block_table + (int64_t)b * p_max_pages;
    // page ids of the chunk: logical page p0 + i in lane i of pid0 / pid1
    // (clamped into the table row; past the sequence: its last page)
    int pid0 = bt[min(p0 + lane, p_max_pages - 1)];
    int pid1 = bt[min(p0 + 64 + lane, p_max_pages - 1)];
    // q as the QK B operand: lane (head n, jq), dims 32 m + 8 jq .. + 7 (zero for n >= g)
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
    const int seq_len = p_seq_lens[b];
    asm volatile("" ::: "memory");  // keeps the loads above issued before the early return below

    const int n_pages = (seq_len + kPage - 1) / kPage;
    if (p0 >= n_pages) return;  // uniform over the workgroup
    const int n_tiles_seq = (seq_len + kTok - 1) / kTok;
    const int t_begin = 2 * p0;
    const int t_end = min(t_begin + 2 * p_chunk_pages, n_tiles_seq);
    const int n_steps = t_end - t_begin;
    const int n_chunks = (n_pages + p_chunk_pages - 1) / p_chunk_pages;
    const int last_lp = n_pages - 1;

    // ---- loads: this wave's NL 1 KiB pieces of a slot.  Piece I = j NL + i
    // covers slot bytes [1024 I, + 1024): lane l writes chunk position P =
    // 64 I + l, i.e. tensor P / (8 cpr) (K, then V), row r = (P / cpr) % 8,
    // position q = P % cpr, holding chunk q ^ swz(r) of that row.
    // (arrays of a fixed size: sized by the kernel's template-dependent NL and
    // captured by the lambda below, they make clang's host pass drop the
    // kernel's launch stub)
    static_assert(NL <= 4, "loads a wave a slot");
    uint32_t src_off[4] = {0, 0, 0, 0};  // byte offset in the tile's half page
    bool src_v[4] = {false, false, false, false};
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int P = 64 * (j * NL + i) + lane;
        const int r = (P / cpr) % kTok, q = P % cpr;
        src_v[i] = 64 * (j * NL + i) >= kTok * cpr;  // (wave-uniform: whole pieces are K or V)
        src_off[i] = (uint32_t)(r * rowb + (q ^ swz(r)) * 16);
    }
    const uint32_t page_bytes = (uint32_t)(kPage * rowb);
    auto page_of = [&](int lp) -> int64_t {
        const int rel = min(lp, last_lp) - p0;
        return (int64_t)__builtin_amdgcn_readlane(rel < 64 ? pid0 : pid1, rel & 63);
    };
    // Tile s of the chunk into slot s % kSlots; tiles past the chunk load with
    // zero-size descriptors (no memory access; zeros written), so every wave
    // has NL loads of every slot in flight.
    auto issue = [&](int s) __attribute__((always_inline)) {
        const int t = t_begin + s;
        const bool ok = s < n_steps;
        const int64_t pg = ok ? page_of(t >> 1) : 0;
        const uint32_t half_off = (uint32_t)((t & 1) * kTok * rowb);
        const auto rk = rsrc(a.k + pg * (page_bytes / 2), ok ? page_bytes : 0u);
        const auto rv = rsrc(a.v + pg * (page_bytes / 2), ok ? page_bytes : 0u);
        uint8_t* const dst = smem + (s % kSlots) * kSlotBytes + 1024 * j * NL;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            if (src_v[i])
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (IRIS_LDS void*)(dst + 1024 * i), 16,
                                                         src_off[i] + half_off, 0, 0, kNT);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (IRIS_LDS void*)(dst + 1024 * i), 16,
                                                         src_off[i] + half_off, 0, 0, kNT);
        }
    };
#pragma unroll
    for (int s = 0; s < kAhead; ++s) issue(s);

    // ---- per-lane LDS offsets within a slot
    // K operand m: row n & 7, chunk j CPH + 4 m + jq.
    uint32_t k_off[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const int r = n & 7;
        k_off[m] = (uint32_t)(r * rowb + ((j * CPH + 4 * m + jq) ^ swz(r)) * 16);
    }
    // V^T operand k (dims 16 k .. + 15): group jq's lane 4 r + kk points at
    // token 4 jq + r, dims 16 k + 4 kk .. + 3 (chunk j CPH + 2 k + (kk >> 1),
    // half kk & 1); tokens 8-15 (jq >= 2) at the zero chunk.
    const int v_row = 4 * jq + (n >> 2), v_kk = n & 3;
    uint32_t v_off[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k)
        v_off[k] = (uint32_t)(kTok * rowb + v_row * rowb +
                              ((j * CPH + 2 * k + (v_kk >> 1)) ^ swz(v_row)) * 16 + 8 * (v_kk & 1));
    const uint32_t zero_addr = lds_addr(smem + kZeroOff);
    if (threadIdx.x < 4) reinterpret_cast<uint32_t*>(smem + kZeroOff)[threadIdx.x] = 0u;

    const float c = a.log2_scale;
    float m_run = -INFINITY;  // running max of the base-2 logits
    float l_part = 0.0f;      // this lane's share of the softmax denominator
    float4_t o[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) o[k] = float4_t{0, 0, 0, 0};

    const uint32_t ring = lds_addr(smem);
    for (int s = 0; s < n_steps; ++s) {
        wait_vmcnt<(kAhead - 1) * NL>();
        __syncthreads();  // every wave's loads of slot s have landed; slot s - 1 is free
        issue(s + kAhead);
        const uint32_t base = ring + (uint32_t)((s % kSlots) * kSlotBytes);
        const int tok0 = (t_begin + s) * kTok;
        const int valid = min(seq_len - tok0, kTok);  // >= 1
        // S = K q^T: lane (head n, jq) holds tokens 4 jq + i.
        uint32_t ka[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) ka[m] = base + k_off[m];
        u32x4_t kr[NM];
        k_reads<NM>(ka, kr);
        float4_t acc = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < NM; ++m)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, kr[m]), qb[m], acc, 0, 0, 0);
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = 4 * jq + i < valid ? acc[i] * c : -INFINITY;
        const float mx = rows_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));  // finite: token 0 is valid
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
        m_run = m_new;
        half4_t pb;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(sc[i] - m_new);
            psum += p;
            pb[i] = (half_t)p;
        }
        l_part = l_part * alpha + psum;
        // O^T += V^T P^T per 16 dims
        const bool row_ok = v_row < valid;
        uint32_t va[NC];
#pragma unroll
        for (int k = 0; k < NC; ++k) va[k] = row_ok ? base + v_off[k] : zero_addr;
        u32x2_t vr[NC];
        v_reads<NC>(va, vr);
#pragma unroll
        for (int k = 0; k < NC; ++k)
            o[k] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, vr[k]), pb, o[k] * alpha, 0, 0,
                                                         0);
    }
    wait_vmcnt<0>();  // the empty loads past the chunk still write LDS
    l_part = rows_sum(l_part);

    // ---- this wave's result for head j g + n (n < g), dims 16 k + 4 jq + i
    const int64_t hq = a.n_q_heads;
    const int head = j * g + n;
    auto store_out = [&](const float4_t (&v)[NC]) {
        if (!col_valid) return;
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            const int64_t idx = ((int64_t)b * hq + head) * D + 16 * k + 4 * jq;
            if (a.out_f32) {
                *reinterpret_cast<float4_t*>(reinterpret_cast<float*>(a.out) + idx) = v[k];
            } else {
                const half2_t lo = {(half_t)v[k][0], (half_t)v[k][1]}, hi = {(half_t)v[k][2], (half_t)v[k][3]};
                *reinterpret_cast<u32x2_t*>(reinterpret_cast<half_t*>(a.out) + idx) = u32x2_t{as_u32(lo), as_u32(hi)};
            }
        }
    };
    const float inv = 1.0f / l_part;
    float4_t res[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) res[k] = o[k] * inv;
    if (n_chunks == 1) {
        store_out(res);
        return;
    }

    // ---- split-KV: publish (o / l, m, l) with device-coherent stores; the
    // last chunk to arrive (the protocol of arrive_last) merges every chunk
    // of the sequence.
    const int64_t row0 = (int64_t)b * p_max_chunks;
    const uint32_t part_o = (uint32_t)(hq * D * 4), part_ml = (uint32_t)(hq * 8);  // bytes per partial
    {
        const auto ro = rsrc(a.part_o + (row0 + chunk) * hq * D, part_o);
        const auto rm = rsrc(a.part_ml + (row0 + chunk) * hq * 2, part_ml);
        if (col_valid) {
#pragma unroll
            for (int k = 0; k < NC; ++k)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, res[k]), ro,
                                                       (uint32_t)((head * D + 16 * k + 4 * jq) * 4), 0, kSC1);
            if (jq == 0)
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, float2v_t{m_run, l_part}), rm,
                                                      (uint32_t)(head * 8), 0, kSC1);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();
    uint32_t* const ctl = reinterpret_cast<uint32_t*>(smem + kCtlOff);
    if (threadIdx.x == 0)
        ctl[0] = arrive_last(a.counters + (int64_t)b * kCountersPerSeq, (uint32_t)n_chunks) ? 1u : 0u;
    __syncthreads();
    if (ctl[0] == 0) return;

    // Merge the M partials, each thread a float4 of the output: o = sum_c w_c
    // (o / l)_c / sum_c w_c, w_c = l_c 2^(m_c - m*), kMergeBatch partials in
    // flight, m* the running maximum.
    const int M = n_chunks;
    const auto ro = rsrc(a.part_o + row0 * hq * D, part_o * (uint32_t)M);
    const auto rm = rsrc(a.part_ml + row0 * hq * 2, part_ml * (uint32_t)M);
    const int n4 = (int)(hq * D / 4);
    for (int e4 = threadIdx.x; e4 < n4; e4 += blockDim.x) {
        const int h = 4 * e4 / D;
        float mstar = -INFINITY, lsum = 0.0f;
        float4_t acc4 = {0, 0, 0, 0};
        for (int c0 = 0; c0 < M; c0 += kMergeBatch) {
            float4_t oc[kMergeBatch];
            float2v_t ml[kMergeBatch];
#pragma unroll
            for (int cb = 0; cb < kMergeBatch; ++cb) {
                const int cc = min(c0 + cb, M - 1);  // past M: a repeat of partial M - 1 with weight 0
                oc[cb] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                          ro, (uint32_t)cc * part_o + (uint32_t)e4 * 16, 0, kSC1));
                ml[cb] = __builtin_bit_cast(float2v_t, __builtin_amdgcn_raw_buffer_load_b64(
                                                           rm, ((uint32_t)cc * (uint32_t)hq + (uint32_t)h) * 8, 0,
                                                           kSC1));
            }
            float mb = mstar;
#pragma unroll
            for (int cb = 0; cb < kMergeBatch; ++cb) mb = fmaxf(mb, ml[cb][0]);
            const float r = __builtin_amdgcn_exp2f(mstar - mb);  // 0 on the first batch
            acc4 *= r;
            lsum *= r;
#pragma unroll
            for (int cb = 0; cb < kMergeBatch; ++cb) {
                const float w = c0 + cb < M ? ml[cb][1] * __builtin_amdgcn_exp2f(ml[cb][0] - mb) : 0.0f;
                acc4 += oc[cb] * w;
                lsum += w;
            }
            mstar = mb;
        }
        const float4_t v4 = acc4 * (1.0f / lsum);
        const int64_t idx = (int64_t)b * hq * D + 4 * e4;
        if (a.out_f32) {
            *reinterpret_cast<float4_t*>(reinterpret_cast<float*>(a.out) + idx) = v4;
        } else {
            const half2_t lo = {(half_t)v4[0], (half_t)v4[1]}, hi = {(half_t)v4[2], (half_t)v4[3]};
            *reinterpret_cast<u32x2_t*>(reinterpret_cast<half_t*>(a.out) + idx) = u32x2_t{as_u32(lo), as_u32(hi)};
        }
    }
}

}  // namespace f16s

// ------------------------------------------------------------------ host side

bool fp16_stream_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim) {
    if (num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || num_q_heads / num_kv_heads > 16) return false;
    if (head_dim == 128) return num_kv_heads == 4 || num_kv_heads == 8;
    if (head_dim == 64) return num_kv_heads == 8 || num_kv_heads == 16;
    return false;
}

bool fp16_stream_preferred(int64_t batch, int64_t num_kv_heads, int64_t head_dim, int64_t total_tokens,
                           int64_t max_tokens) {
    // Batches of similar lengths (ragged ones leave the long sequences'
    // chunks, at most 16 a sequence, running after the rest: configuration 3,
    // 345 us against 235), enough sequences that their chunks fill half the
    // CUs, and at least 64 MB of K/V.  MI355X, Hq=32, Hkv=8, D=128, against
    // the per-kv-head kernel: B=1..4 at L=4096 (17-67 MB) 32.7-33.5 us
    // against 18.6-29.8; B=4, L=16384 (64 workgroups) 100.8 against 72.4;
    // B=8, L=4096 36.8 against 41.7; B=32 90.2 against 124.5.
    if (4 * total_tokens < 3 * batch * max_tokens) return false;
    if (batch * f16s::kMaxChunks < 128) return false;
    return total_tokens * num_kv_heads * head_dim * 4 >= 64000000;
}

int64_t fp16_stream_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t max_chunks) {
    const int64_t o = batch * max_chunks * num_q_heads * head_dim * 4;
    return counter_region_bytes(batch) + (o + 255) / 256 * 256 + batch * max_chunks * num_q_heads * 2 * 4;
}

bool fp16_stream_plan_fits(int64_t max_pages, int32_t chunk_pages, int32_t max_chunks) {
    return chunk_pages > 0 && chunk_pages <= f16s::kMaxChunkPages && max_chunks > 0 &&
           max_chunks <= f16s::kMaxChunks && (int64_t)chunk_pages * max_chunks >= max_pages;
}

int fp16_stream_plan(int64_t batch, int64_t max_pages, int64_t total_tokens, int64_t max_tokens,
                     int32_t tokens_per_split, int32_t* out_chunk_pages, int32_t* out_max_chunks) {
    // The grid covers every page block_table can address; the lengths steer
    // the chunk size: about one workgroup a CU (256), at least 8 pages each,
    // the longest sequence cut into equal chunks, at most kMaxChunks of them.
    const int64_t cap_tokens = max_pages * f16s::kPage;
    if (max_tokens < 0 || max_tokens > cap_tokens) max_tokens = cap_tokens;
    if (total_tokens < 0) total_tokens = batch * max_tokens;
    const int64_t longest = (max_tokens + f16s::kPage - 1) / f16s::kPage;
    int64_t chunk_pages;
    if (tokens_per_split > 0) {
        chunk_pages = (tokens_per_split + f16s::kPage - 1) / f16s::kPage;
    } else {
        const int64_t pages = (total_tokens + f16s::kPage - 1) / f16s::kPage + batch;
        chunk_pages = (pages + 255) / 256;
        if (chunk_pages < 8) chunk_pages = 8;
        const int64_t pieces = (longest + chunk_pages - 1) / chunk_pages;
        if (pieces > 0) chunk_pages = (longest + pieces - 1) / pieces;
    }
    if (chunk_pages < 1) chunk_pages = 1;
    if (chunk_pages >= longest && max_pages <= f16s::kMaxChunkPages) chunk_pages = max_pages;
    if ((max_pages + chunk_pages - 1) / chunk_pages > f16s::kMaxChunks)
        chunk_pages = (max_pages + f16s::kMaxChunks - 1) / f16s::kMaxChunks;
    if (chunk_pages > f16s::kMaxChunkPages) return kInvalidArgument;
    *out_chunk_pages = (int32_t)chunk_pages;
    *out_max_chunks = (int32_t)((max_pages + chunk_pages - 1) / chunk_pages);
    return kOk;
}

int fp16_stream_launch(const void* query, const void* k_cache, const void* v_cache, const int32_t* block_table,
                       const int32_t* seq_lens, void* output, int32_t output_is_f32, void* workspace,
                       int64_t workspace_bytes_avail, int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                       int64_t head_dim, int64_t max_pages, float softmax_scale, int32_t chunk_pages,
                       int32_t max_chunks, void* stream) {
    if (!fp16_stream_supported(num_q_heads, num_kv_heads, head_dim) ||
        !fp16_stream_plan_fits(max_pages, chunk_pages, max_chunks))
        return kInvalidArgument;
    f16s::Args a;
    a.q = (const half_t*)query;
    a.k = (const half_t*)k_cache;
    a.v = (const half_t*)v_cache;
    a.block_table = block_table;
    a.seq_lens = seq_lens;
    a.out = output;
    a.out_f32 = output_is_f32;
    a.n_q_heads = (int)num_q_heads;
    a.n_kv_heads = (int)num_kv_heads;
    a.group = (int)(num_q_heads / num_kv_heads);
    a.max_pages = (int)max_pages;
    a.max_chunks = max_chunks;
    a.chunk_pages = chunk_pages;
    a.log2_scale = softmax_scale * 1.4426950408889634f;
    a.counters = nullptr;
    a.part_o = a.part_ml = nullptr;
    if (max_chunks > 1) {
        const int64_t need = fp16_stream_workspace_bytes(batch, num_q_heads, head_dim, max_chunks);
        if (workspace == nullptr || workspace_bytes_avail < need) return kWorkspaceTooSmall;
        uint8_t* const ws = (uint8_t*)workspace;
        const int64_t o = batch * max_chunks * num_q_heads * head_dim * 4;
        a.counters = (uint32_t*)ws;
        a.part_o = (float*)(ws + counter_region_bytes(batch));
        a.part_ml = (float*)(ws + counter_region_bytes(batch) + (o + 255) / 256 * 256);
    }
    const int64_t nblocks = batch * (int64_t)max_chunks;
    if (nblocks > 0x7FFFFFFF) return kInvalidArgument;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((unsigned)nblocks), block((unsigned)(64 * num_kv_heads));
    static std::atomic<uint64_t> raised128{0}, raised64{0};
    if (head_dim == 128) {
        if (allow_full_lds(reinterpret_cast<const void*>(&f16s::fp16_decode_stream_kernel<128>), raised128) != kOk)
            return kLaunchError;
        hipLaunchKernelGGL(f16s::fp16_decode_stream_kernel<128>, grid, block, f16s::kLdsBytes, s, seq_lens,
                           block_table, max_chunks, chunk_pages, (int)max_pages, (int)num_kv_heads, a);
    } else {
        if (allow_full_lds(reinterpret_cast<const void*>(&f16s::fp16_decode_stream_kernel<64>), raised64) != kOk)
            return kLaunchError;
        hipLaunchKernelGGL(f16s::fp16_decode_stream_kernel<64>, grid, block, f16s::kLdsBytes, s, seq_lens,
                           block_table, max_chunks, chunk_pages, (int)max_pages, (int)num_kv_heads, a);
    }
    return hipGetLastError() == hipSuccess ? kOk : kLaunchError;
}

}  // namespace iris
