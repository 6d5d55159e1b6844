// HBM streaming ceiling of the cfg2 decode's access pattern (loads only, no
// compute): 32 sequences x 4096 tokens of an INT4 paged cache (Hkv=8, D=128,
// 16-token pages in random order), read by 256 workgroups of 16 waves as
// 1 KiB loads (16 bytes a lane), N loads in flight per wave.  Three ways of
// splitting the work, each reading the same 151 MB:
//   WP: workgroup (sequence, 32-page chunk), whole 1 KiB pieces of every page
//       (the decode kernels' split);
//   HP: workgroup (sequence, kv-head pair, half), 128-byte row pieces;
//   HQ: workgroup (sequence, kv-head quad, quarter), 256-byte row pieces.
// A load = (base for lanes 0-31, base for lanes 32-63, lane pattern), from a
// host-built list; wave w takes loads w, w + 16, ...  Four disjoint page
// sets rotate (a 576 MiB pool), so the 256 MB MALL serves nothing.  The 8
// workgroups of a sequence sit on one XCD (workgroup i on XCD i % 8).
//
// Measurement aid only (not part of the library):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       tests/probe/page_stream_probe.hip -o /tmp/page_stream_probe && /tmp/page_stream_probe
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>
#include <random>
#include <cstdint>

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int B = 32, PPS = 256, NSETS = 4, NP = NSETS * B * PPS, GRID = 256, PER_WG = 576;
constexpr uint64_t DB = (uint64_t)NP * 8192, SB = (uint64_t)NP * 1024, POOL = 2 * DB + 2 * SB;

template <int N>
__device__ __forceinline__ void vwait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// lane patterns: 0 contiguous; 1 128 B rows; 2 256 B rows; 3 HP scales (16 B rows, K|V); 4 HQ scales (32 B rows, K|V)
__device__ __forceinline__ unsigned lane_pattern(int p, int lane) {
    switch (p) {
        case 0: return lane * 16;
        case 1: return (lane / 8) * 512 + (lane % 8) * 16;
        case 2: return (lane / 16) * 512 + (lane % 16) * 16;
        case 3: return (unsigned)(((lane >> 4) & 1) * SB) + (lane & 15) * 64;
        default: return (unsigned)((lane >> 5) * SB) + ((lane >> 1) & 15) * 64 + (lane & 1) * 16;
    }
}

template <int DEPTH>
__global__ __launch_bounds__(1024) void st(const unsigned char* __restrict__ pool, const uint64_t* __restrict__ blocks, unsigned* out) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint64_t* my = blocks + (uint64_t)blockIdx.x * PER_WG * 2;
    constexpr int NB = PER_WG / 16;  // 36
    uint64_t oa = 0, ob = 0;
    if (lane < NB) { oa = my[2 * (wave + 16 * lane)]; ob = my[2 * (wave + 16 * lane) + 1]; }
    const unsigned lp0 = lane_pattern(0, lane), lp1 = lane_pattern(1, lane), lp2 = lane_pattern(2, lane),
                   lp3 = lane_pattern(3, lane), lp4 = lane_pattern(4, lane);
    u32x4 acc = {0, 0, 0, 0};
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(pool), 0, (int)POOL, 0x00020000);
    u32x4 buf[DEPTH];
#define VOFF_OF(jj)                                                                       \
    ({                                                                                    \
        int jv_ = (jj);                                                                   \
        asm volatile("" : "+s"(jv_));                                                     \
        const unsigned alo_ = __builtin_amdgcn_readlane((unsigned)oa, jv_);               \
        const unsigned blo_ = __builtin_amdgcn_readlane((unsigned)ob, jv_);               \
        const int pat_ = (int)(alo_ & 15);                                                \
        unsigned l_ = lp0;                                                                \
        l_ = pat_ == 1 ? lp1 : l_;                                                        \
        l_ = pat_ == 2 ? lp2 : l_;                                                        \
        l_ = pat_ == 3 ? lp3 : l_;                                                        \
        l_ = pat_ == 4 ? lp4 : l_;                                                        \
        ((lane < 32 ? alo_ : blo_) & ~15u) + l_;                                          \
    })
#pragma unroll
    for (int jj = 0; jj < DEPTH; ++jj)
        buf[jj] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, VOFF_OF(jj), 0, 2));
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) {
        acc ^= buf[jj % DEPTH];
        asm volatile("" : "+v"(acc));
        if (jj + DEPTH < NB) {
            unsigned v = VOFF_OF(jj + DEPTH);
            asm volatile("" : "+v"(v) : "v"(buf[jj % DEPTH].x));  // issue after block jj arrived
            buf[jj % DEPTH] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, v, 0, 2));
        }
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345679u) out[0] = 1;
}

int main() {
    unsigned char* pool;
    uint64_t* dblocks;
    unsigned* out;
    if (hipMalloc(&pool, POOL) || hipMalloc(&out, 4)) { printf("alloc\n"); return 1; }
    (void)hipMemset(pool, 1, POOL);
    std::vector<int> perm(NP);
    for (int i = 0; i < NP; ++i) perm[i] = i;
    std::mt19937 rng(5);
    std::shuffle(perm.begin(), perm.end(), rng);
    const size_t set_len = (size_t)GRID * PER_WG * 2;
    std::vector<uint64_t> blocks(NSETS * set_len);
    if (hipMalloc(&dblocks, blocks.size() * 8)) { printf("alloc\n"); return 1; }
    auto put = [&](uint64_t* o, int& n, uint64_t a, uint64_t b, int pat) {
        const uint64_t ext = pat == 0 ? 1024 : pat == 1 ? 3712 : pat == 2 ? 1792 : pat == 3 ? SB + 976 : SB + 992;
        if (a + ext > POOL || b + ext > POOL) { printf("bad offset\n"); exit(1); }
        o[2 * n] = a | pat; o[2 * n + 1] = b | pat; ++n;
    };
    auto fill = [&](int kind) {
        for (int s = 0; s < NSETS; ++s)
            for (int w = 0; w < GRID; ++w) {
                const int x = w % 8, sl = w / 8, b = x * 4 + sl / 8, k = sl % 8;
                const int* pt = perm.data() + (s * B + b) * PPS;
                uint64_t* o = blocks.data() + (size_t)s * set_len + (size_t)w * PER_WG * 2;
                int n = 0;
                if (kind == 0) {
                    for (int p = 0; p < 32; ++p) {
                        const uint64_t pid = pt[k * 32 + p];
                        for (int i = 0; i < 8; ++i) put(o, n, pid * 8192 + i * 1024, pid * 8192 + i * 1024, 0);
                        for (int i = 0; i < 8; ++i) put(o, n, DB + pid * 8192 + i * 1024, DB + pid * 8192 + i * 1024, 0);
                        put(o, n, 2 * DB + pid * 1024, 2 * DB + pid * 1024, 0);
                        put(o, n, 2 * DB + SB + pid * 1024, 2 * DB + SB + pid * 1024, 0);
                    }
                } else if (kind == 1) {
                    const int sub = k / 2, p0 = (k % 2) * 128;
                    for (int p = 0; p < 128; p += 2) {
                        for (int q = 0; q < 2; ++q) {
                            const uint64_t pid = pt[p0 + p + q];
                            for (int t = 0; t < 2; ++t)
                                for (int h = 0; h < 2; ++h) {
                                    const uint64_t a = t * DB + pid * 8192 + h * 8 * 512 + sub * 128;
                                    put(o, n, a, a, 1);
                                }
                        }
                        const uint64_t pa = pt[p0 + p], pb = pt[p0 + p + 1];
                        put(o, n, 2 * DB + pa * 1024 + sub * 16, 2 * DB + pb * 1024 + sub * 16, 3);
                    }
                } else {
                    const int sub = k / 4, p0 = (k % 4) * 64;
                    for (int p = 0; p < 64; ++p) {
                        const uint64_t pid = pt[p0 + p];
                        for (int t = 0; t < 2; ++t)
                            for (int h = 0; h < 4; ++h) {
                                const uint64_t a = t * DB + pid * 8192 + h * 4 * 512 + sub * 256;
                                put(o, n, a, a, 2);
                            }
                        put(o, n, 2 * DB + pid * 1024 + sub * 32, 2 * DB + pid * 1024 + sub * 32, 4);
                    }
                }
                if (n != PER_WG) { printf("count %d\n", n); exit(1); }
            }
        (void)hipMemcpy(dblocks, blocks.data(), blocks.size() * 8, hipMemcpyHostToDevice);
    };
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    const double useful = (double)GRID * PER_WG * 1024;
    auto run = [&](const char* name, auto kern) {
        for (int i = 0; i < 8; ++i) hipLaunchKernelGGL(kern, dim3(GRID), dim3(1024), 0, 0, pool, dblocks + (i % NSETS) * set_len, out);
        if (hipDeviceSynchronize() != hipSuccess) { printf("kernel failed\n"); exit(1); }
        float best = 1e9;
        for (int rep = 0; rep < 5; ++rep) {
            (void)hipEventRecord(e0);
            const int reps = 40;
            for (int i = 0; i < reps; ++i) hipLaunchKernelGGL(kern, dim3(GRID), dim3(1024), 0, 0, pool, dblocks + (i % NSETS) * set_len, out);
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            float ms;
            (void)hipEventElapsedTime(&ms, e0, e1);
            best = std::min(best, ms * 1000.0f / reps);
        }
        printf("  %-26s %7.2f us  %5.0f GB/s\n", name, best, useful / (best * 1e3));
        fflush(stdout);
    };
    const char* kn[3] = {"WP whole pages", "HP head pairs (128 B)", "HQ head quads (256 B)"};
    for (int kind = 0; kind < 3; ++kind) {
        fill(kind);
        printf("%s, %.1f MB\n", kn[kind], useful / 1e6);
        run("buffer depth 1", st<1>);
        run("buffer depth 2", st<2>);
        run("buffer depth 3", st<3>);
        run("buffer depth 4", st<4>);
    }
    return 0;
}
