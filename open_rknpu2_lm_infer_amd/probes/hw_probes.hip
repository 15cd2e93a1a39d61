// Hardware calibration probes behind the roofline figures: what one MI355X actually
// delivers to the kernels of this library.
//
//   hw_probes mfma   int8 MFMA rate (v_mfma_i32_16x16x64_i8, 8 independent chains per wave)
//                    and the shader clock under that load (s_memtime against s_memrealtime)
//   hw_probes dma    global -> LDS copy rate (buffer_load_dwordx4 ... lds) from an L2-resident
//                    1 MiB source
//   hw_probes lds    ds_read_b128 cost and SQ_LDS_BANK_CONFLICT-visible patterns: lane address
//                    patterns that separate bank-count and lane-grouping models (run under
//                    rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT for the conflict counts)
//   hw_probes floor  back-to-back launches in a hipGraph: an empty kernel, and a kernel that
//                    only streams each decode weight matrix once (36 copies rotated), i.e. the
//                    floor of a one-launch-per-linear decode step
//
// Every index is bounded by the buffer it addresses (comments at each kernel).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <vector>

typedef int v4i __attribute__((ext_vector_type(4)));

#define CK(x)                                                                                   \
    do {                                                                                        \
        hipError_t e_ = (x);                                                                    \
        if (e_ != hipSuccess) {                                                                 \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);          \
            return 1;                                                                           \
        }                                                                                       \
    } while (0)

// ---- mfma: out[2 * block + {0, 1}], block < 4096 ------------------------------------------
__global__ __launch_bounds__(256) void mfma_rate(int iters, unsigned long long* out, int* sink) {
    v4i acc[8];
    for (int j = 0; j < 8; ++j) acc[j] = v4i{0, 0, 0, 0};
    const v4i a = {(int)threadIdx.x, 1, 2, 3}, b = {3, 2, 1, (int)blockIdx.x};
    const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[j], 0, 0, 0);
    }
    const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    int s = 0;
    for (int j = 0; j < 8; ++j) s += acc[j][0] ^ acc[j][3];
    if (s == 0x1234567) sink[threadIdx.x] = s;  // sink: 256 ints
    if (threadIdx.x == 0 && blockIdx.x < 4096) {
        out[blockIdx.x * 2] = c1 - c0;
        out[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

// ---- dma: 1 KiB blocks of a 1 MiB source into a 32 KiB LDS ring ------------------------------
// LDS offset (wave * 8 + it % 8) KiB < 32 KiB; source offset (block & 1023) KiB + lane * 16 < 1 MiB.
__global__ __launch_bounds__(256) void dma_rate(const unsigned char* src, int iters, unsigned long long* out) {
    __shared__ __attribute__((aligned(16))) unsigned char s[32768];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, 1 << 20, 0x00020000);
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
        const int blk = (blockIdx.x * 4 + w + it * 7) & 1023;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(s + ((w * 8 + (it & 7)) << 10)),
                                                 16, l * 16, blk << 10, 0, 0);
        if ((it & 7) == 7) __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8));  // vmcnt <= 8
    }
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    if (threadIdx.x == 0 && blockIdx.x < 4096) out[blockIdx.x] = c1 - c0;
}

// ---- lds: lane address patterns, 8 reads per iteration at +1 KiB steps -----------------------
// Largest pattern address 63 * 256 = 16128; + 7 KiB + 16 B < 32 KiB.
__device__ __forceinline__ int lds_addr(int P, int l) {
    const int fr = l & 15, fc = l >> 4;
    switch (P) {
        case 0: return l * 16;                                         // contiguous 1 KiB
        case 1: return l * 256;                                        // one bank group
        case 2: return l * 128;
        case 3: return (l & 7) * 16 + (l >> 3) * 128;                  // octets in alternating 128-byte halves
        case 4: return (l & 7) * 16 + (l >> 3) * 256;                  // octets in the same half
        case 5: return ((l & 7) * 16 + (l >> 3) * 128) ^ ((l >> 4) & 1) * 128;  // halves swapped per 16 lanes
        case 6: return fr * 128 + (((2 * fc) ^ (fr & 7)) << 4);       // 128-byte rows, swizzle row & 7
        case 7: return fr * 128 + (((2 * fc) ^ ((fr >> 1) & 3)) << 4);  // 128-byte rows, swizzle (row >> 1) & 3
        case 8: return fr * 64 + ((fc ^ ((fr >> 1) & 3)) << 4);       // 64-byte rows, swizzle (row >> 1) & 3
        case 9: return fr * 64 + ((fc ^ ((fr >> 2) & 3)) << 4);       // 64-byte rows, swizzle (row >> 2) & 3
        // 128-byte rows, swizzle bit 1 -> 1, bit 2 -> 4 of the row (k halves 0 and 1)
        case 10: return fr * 128 + (((2 * fc) ^ (((fr >> 1) & 1) | ((fr >> 2) & 1) << 2)) << 4);
        case 11: return fr * 128 + (((2 * fc + 1) ^ (((fr >> 1) & 1) | ((fr >> 2) & 1) << 2)) << 4);
        // 128-byte rows, swizzle bit 1 -> 1, bit 2 -> 4, bit 3 -> 6
        default: return fr * 128 + (((2 * fc) ^ (((fr >> 1) & 1) ^ ((fr >> 2) & 1) * 4 ^ ((fr >> 3) & 1) * 6)) << 4);
    }
}
constexpr int kLdsPatterns = 13;
template <int P>
__global__ void lds_read(unsigned long long* out, int iters, int* sink) {
    __shared__ __attribute__((aligned(16))) unsigned char s[32768];
    for (int i = threadIdx.x; i < 32768 / 4; i += blockDim.x) reinterpret_cast<int*>(s)[i] = i;
    __syncthreads();
    const int a = lds_addr(P, threadIdx.x & 63);
    v4i x = {0, 0, 0, 0};
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < 8; ++k) x ^= *reinterpret_cast<const v4i*>(s + a + 1024 * k);
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    if ((threadIdx.x & 63) == 0) out[threadIdx.x >> 6] = t1 - t0;  // out: 16 entries (<= 16 waves)
    if (x[0] + x[1] + x[2] + x[3] == 0x12345678) sink[threadIdx.x] = 1;  // sink: 1024 ints
}

// ---- floor --------------------------------------------------------------------------------
__global__ void empty_kernel(int* sink) {
    if (threadIdx.x == 4096) sink[0] = 1;  // never true: the launch only
}
// Workgroup b reads 16-byte elements [b * n16 / G, (b + 1) * n16 / G) of src; every index is
// checked against that range.
__global__ __launch_bounds__(512) void stream_kernel(const v4i* __restrict__ src, long n16, int* sink) {
    const long b0 = n16 * blockIdx.x / gridDim.x, b1 = n16 * (blockIdx.x + 1) / gridDim.x;
    v4i x = {0, 0, 0, 0};
    for (long i = b0 + threadIdx.x; i < b1; i += 512L * 8) {
        v4i r[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const long j = i + 512L * u;
            r[u] = j < b1 ? __builtin_nontemporal_load(src + j) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) x ^= r[u];
    }
    if (x[0] == 0x12345 && x[1] == 0x777) sink[threadIdx.x] = x[2];  // sink: 1024 ints
}

static int run_mfma() {
    unsigned long long* d;
    int* sink;
    CK(hipMalloc(&d, 16 * 4096));
    CK(hipMalloc(&sink, 4096));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    std::vector<unsigned long long> h(2 * 4096);
    for (int blocks : {256, 1024}) {
        const int iters = 4000;
        mfma_rate<<<blocks, 256>>>(iters, d, sink);
        CK(hipEventRecord(e0));
        mfma_rate<<<blocks, 256>>>(iters, d, sink);
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        CK(hipMemcpy(h.data(), d, 16 * 4096, hipMemcpyDeviceToHost));
        const double cyc = (double)h[0], us = h[1] / 100.0;
        const double ops = 2.0 * 16 * 16 * 64 * 8 * (double)iters * 4 * blocks;
        std::printf("mfma: %4d workgroups x 4 waves: %.3f POPS, shader clock %.3f GHz, %.2f cycles per MFMA per wave\n",
                    blocks, ops / (ms * 1e-3) / 1e15, cyc / us / 1e3, cyc / (8.0 * iters));
    }
    return 0;
}

static int run_dma() {
    unsigned long long* d;
    unsigned char* src;
    CK(hipMalloc(&d, 8 * 4096));
    CK(hipMalloc(&src, 1 << 20));
    CK(hipMemset(src, 1, 1 << 20));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    std::vector<unsigned long long> h(4096);
    for (int blocks : {256, 512}) {
        const int iters = 4096;
        dma_rate<<<blocks, 256>>>(src, iters, d);
        CK(hipEventRecord(e0));
        dma_rate<<<blocks, 256>>>(src, iters, d);
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        CK(hipMemcpy(h.data(), d, 8 * 4096, hipMemcpyDeviceToHost));
        const double bytes = 1024.0 * iters * 4 * blocks;
        std::printf("dma: %4d workgroups: %.2f TB/s in total, %.1f B per shader clock per workgroup\n", blocks,
                    bytes / (ms * 1e-3) / 1e12, 4096.0 * iters / (double)h[0]);
    }
    return 0;
}

template <int P>
static int lds_row(unsigned long long* d, int* sink) {
    for (int waves : {1, 8, 16}) {
        const int iters = 2000;
        lds_read<P><<<1, 64 * waves>>>(d, iters, sink);
        CK(hipDeviceSynchronize());
        unsigned long long h[16];
        CK(hipMemcpy(h, d, 8 * waves, hipMemcpyDeviceToHost));
        const unsigned long long mx = *std::max_element(h, h + waves);
        std::printf("lds: pattern %d, %2d waves: %6.2f cycles per ds_read_b128 per wave, %6.1f B per clock per CU\n", P,
                    waves, (double)mx / (iters * 8.0), 1024.0 * 8 * iters * waves / (double)mx);
    }
    return 0;
}
template <int P>
static int lds_all(unsigned long long* d, int* sink) {
    if constexpr (P < kLdsPatterns) {
        if (lds_row<P>(d, sink)) return 1;
        return lds_all<P + 1>(d, sink);
    }
    return 0;
}
static int run_lds() {
    unsigned long long* d;
    int* sink;
    CK(hipMalloc(&d, 8 * 16));
    CK(hipMalloc(&sink, 4096));
    return lds_all<0>(d, sink);
}

static int run_floor() {
    const long sizes[4] = {7888896, 5253120, 24981504, 12462080};  // W4 qkv, o, gate_up, down + scales
    const char* names[4] = {"qkv", "o", "gate_up", "down"};
    const int L = 36, R = 20;
    int* sink;
    CK(hipMalloc(&sink, 4096));
    hipStream_t st;
    CK(hipStreamCreate(&st));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    auto time_graph = [&](auto launch, double* us) -> int {
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
        for (int l = 0; l < L; ++l) launch(l);
        CK(hipStreamEndCapture(st, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, st));
        CK(hipStreamSynchronize(st));
        CK(hipEventRecord(e0, st));
        for (int r = 0; r < R; ++r) CK(hipGraphLaunch(ge, st));
        CK(hipEventRecord(e1, st));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
        *us = ms * 1e3 / (L * R);
        return 0;
    };
    double us, total = 0;
    if (time_graph([&](int) { empty_kernel<<<256, 512, 0, st>>>(sink); }, &us)) return 1;
    std::printf("floor: empty kernel, 256 x 512 threads: %.2f us per launch\n", us);
    long bytes = 0;
    for (int s = 0; s < 4; ++s) {
        std::vector<v4i*> bufs(L);
        for (int l = 0; l < L; ++l) {
            CK(hipMalloc(&bufs[l], sizes[s]));
            CK(hipMemset(bufs[l], l, sizes[s]));
        }
        const long n16 = sizes[s] / 16;
        if (time_graph([&](int l) { stream_kernel<<<256, 512, 0, st>>>(bufs[l], n16, sink); }, &us)) return 1;
        std::printf("floor: stream %-8s %9ld B: %6.2f us per launch, %6.0f GB/s\n", names[s], sizes[s], us,
                    sizes[s] / us / 1e3);
        total += us;
        bytes += sizes[s];
        for (int l = 0; l < L; ++l) CK(hipFree(bufs[l]));
    }
    std::printf("floor: one layer as four streaming launches: %.2f us, %.0f GB/s\n", total, bytes / total / 1e3);
    return 0;
}

int main(int argc, char** argv) {
    const char* what = argc > 1 ? argv[1] : "all";
    const bool all = !std::strcmp(what, "all");
    if ((all || !std::strcmp(what, "mfma")) && run_mfma()) return 1;
    if ((all || !std::strcmp(what, "dma")) && run_dma()) return 1;
    if ((all || !std::strcmp(what, "lds")) && run_lds()) return 1;
    if ((all || !std::strcmp(what, "floor")) && run_floor()) return 1;
    return 0;
}
