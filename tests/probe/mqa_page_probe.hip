// HBM streaming ceiling of configuration 4's decode access pattern (loads
// only, no compute): 128 sequences x 8192 tokens of an INT4 paged cache with
// one kv head and D=64, i.e. 16-token pages of 512 B of K codes, 512 B of V
// codes and 64 B of each scale tensor, four separate regions per page.
// 512 workgroups of W waves, one per (sequence, 128-page chunk); wave w of a
// workgroup takes tiles w, w + W, ... (a tile = two pages = four 16-byte-a-lane
// loads: K and V codes of both pages, K and V scales of both pages), with N
// tiles in flight per wave.  Pages in random order (the decode benchmark's
// block tables) or consecutive per sequence; four page sets rotate over a
// 302 MB pool, so the 256 MB MALL serves nothing.
//
// Measurement aid only (not part of the library):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       tests/probe/mqa_page_probe.hip -o /tmp/mqa_page_probe && /tmp/mqa_page_probe
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int B = 128, PPS = 512, NSETS = 4, NP = NSETS * B * PPS;
constexpr uint64_t V_OFF = (uint64_t)NP * 512, KS_OFF = 2ull * NP * 512, VS_OFF = KS_OFF + (uint64_t)NP * 64;
constexpr uint64_t POOL = VS_OFF + (uint64_t)NP * 64;
constexpr int GRID = 512, TILES_PER_WG = 64, LOADS_PER_TILE = 4, PER_WG = TILES_PER_WG * LOADS_PER_TILE;
static_assert(POOL < (1ull << 31), "32-bit buffer offsets");

// A load: lanes 0-31 read from offset a, lanes 32-63 from offset b (both 64-byte
// aligned; bit 0 = pattern): pattern 0, 512 bytes a half (16 B a lane);
// pattern 1, 64 bytes a half (lanes 4..31 repeat lanes 0..3's addresses).
__device__ __forceinline__ unsigned lane_off(unsigned pat, int lane) {
    return pat ? (unsigned)(lane & 3) * 16 : (unsigned)(lane & 31) * 16;
}

template <int WAVES, int DEPTH>
__global__ __launch_bounds__(1024) void st(const unsigned char* __restrict__ pool, const uint32_t* __restrict__ list,
                                           unsigned* out) {
    constexpr int N = PER_WG / WAVES;  // loads per wave
    static_assert(N <= 64, "a wave's offsets fit one VGPR pair");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t* my = list + (uint64_t)blockIdx.x * PER_WG * 2;
    unsigned oa = 0, ob = 0;
    if (lane < N) {  // load k of wave w is load (k / 4) * WAVES * 4 + w * 4 + k % 4 of the workgroup
        const int e = (lane / 4) * WAVES * 4 + wave * 4 + lane % 4;
        oa = my[2 * e];
        ob = my[2 * e + 1];
    }
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(pool), 0, (int)POOL, 0x00020000);
    auto voff = [&](int j) {
        int jv = j;
        asm volatile("" : "+s"(jv));
        const unsigned a = __builtin_amdgcn_readlane(oa, jv), b = __builtin_amdgcn_readlane(ob, jv);
        return ((lane < 32 ? a : b) & ~63u) + lane_off(a & 1, lane);
    };
    constexpr int D = DEPTH * LOADS_PER_TILE;
    u32x4 acc = {0, 0, 0, 0};
    u32x4 buf[D];
#pragma unroll
    for (int j = 0; j < D; ++j) buf[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff(j), 0, 0));
#pragma unroll
    for (int j = 0; j < N; ++j) {
        acc ^= buf[j % D];
        asm volatile("" : "+v"(acc));
        if (j + D < N) {
            unsigned v = voff(j + D);
            asm volatile("" : "+v"(v) : "v"(buf[j % D].x));  // issued after load j arrived
            buf[j % D] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, v, 0, 0));
        }
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345679u) out[0] = 1;
}

int main() {
    unsigned char* pool;
    uint32_t* dlist;
    unsigned* out;
    if (hipMalloc(&pool, POOL) || hipMalloc(&out, 4)) { printf("alloc\n"); return 1; }
    (void)hipMemset(pool, 1, POOL);
    const size_t set_len = (size_t)GRID * PER_WG * 2;
    std::vector<uint32_t> list(NSETS * set_len);
    if (hipMalloc(&dlist, list.size() * 4)) { printf("alloc\n"); return 1; }
    std::vector<int> perm(NP);
    auto fill = [&](bool random) {
        for (int i = 0; i < NP; ++i) perm[i] = i;
        if (random) {
            std::mt19937 rng(5);
            std::shuffle(perm.begin(), perm.end(), rng);
        }
        for (int s = 0; s < NSETS; ++s)
            for (int w = 0; w < GRID; ++w) {
                const int b = w / 4, k = w % 4;
                const int* pt = perm.data() + ((size_t)s * B + b) * PPS + k * 128;
                uint32_t* o = list.data() + (size_t)s * set_len + (size_t)w * PER_WG * 2;
                for (int t = 0; t < TILES_PER_WG; ++t) {
                    const uint64_t p0 = pt[2 * t], p1 = pt[2 * t + 1];
                    const uint64_t e[4][2] = {{p0 * 512, p1 * 512},
                                              {V_OFF + p0 * 512, V_OFF + p1 * 512},
                                              {KS_OFF + p0 * 64 + 1, KS_OFF + p1 * 64 + 1},
                                              {VS_OFF + p0 * 64 + 1, VS_OFF + p1 * 64 + 1}};
                    for (int q = 0; q < 4; ++q) {
                        const uint64_t ext = (e[q][0] & 1) ? 64 : 512;  // bytes a half reads
                        if ((e[q][0] & ~63ull) + ext > POOL || (e[q][1] & ~63ull) + ext > POOL) { printf("bad offset\n"); exit(1); }
                        o[2 * (4 * t + q)] = (uint32_t)e[q][0];
                        o[2 * (4 * t + q) + 1] = (uint32_t)e[q][1];
                    }
                }
            }
        (void)hipMemcpy(dlist, list.data(), list.size() * 4, hipMemcpyHostToDevice);
    };
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    const double useful = (double)B * PPS * (2 * 512 + 2 * 64);
    auto run = [&](const char* name, auto kern, int waves) {
        for (int i = 0; i < 8; ++i)
            hipLaunchKernelGGL(kern, dim3(GRID), dim3(64 * waves), 0, 0, pool, dlist + (i % NSETS) * set_len, out);
        if (hipDeviceSynchronize() != hipSuccess) { printf("kernel failed\n"); exit(1); }
        float best = 1e9;
        for (int rep = 0; rep < 5; ++rep) {
            (void)hipEventRecord(e0);
            const int reps = 40;
            for (int i = 0; i < reps; ++i)
                hipLaunchKernelGGL(kern, dim3(GRID), dim3(64 * waves), 0, 0, pool, dlist + (i % NSETS) * set_len, out);
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            float ms;
            (void)hipEventElapsedTime(&ms, e0, e1);
            best = std::min(best, ms * 1000.0f / reps);
        }
        printf("  %-34s %7.2f us  %5.0f GB/s\n", name, best, useful / (best * 1e3));
        fflush(stdout);
    };
    for (int random = 1; random >= 0; --random) {
        fill(random != 0);
        printf("%s page order, %.1f MB a launch\n", random ? "random" : "consecutive", useful / 1e6);
        run("4 waves, 1 tile in flight a wave", st<4, 1>, 4);
        run("4 waves, 2 tiles in flight a wave", st<4, 2>, 4);
        run("4 waves, 4 tiles in flight a wave", st<4, 4>, 4);
        run("16 waves, 1 tile in flight a wave", st<16, 1>, 16);
        run("16 waves, 2 tiles in flight a wave", st<16, 2>, 16);
        run("16 waves, 4 tiles in flight a wave", st<16, 4>, 16);
    }
    return 0;
}
