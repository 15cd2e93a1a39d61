// Calibration kernels for the roofline figures of the quantized-linear path on MI355X.
// Built into libqlcalib.so, apart from libqlinear.so (nothing here is on the product
// path); bench.py --mode calib times them with HIP events and prints the figures.
//
//   qcal_empty    an empty kernel: the cost of one launch in a HIP graph
//   qcal_stream   reads `bytes` once, split evenly over `grid` workgroups of 512 threads
//                 (16-byte loads, 8 in flight per thread): the floor of a kernel whose only
//                 work is streaming a decode weight matrix
//   qcal_mfma     v_mfma_i32_16x16x64_i8 back to back on register operands, 4 independent
//                 accumulators per wave: the int8 matrix-core rate the chip sustains
//   qcal_stream_lds as qcal_stream, with direct global -> LDS copies (16 bytes a lane,
//                 8 per wave in flight) instead of loads into registers: the HBM rate of
//                 the copies a kernel that stages weights in LDS depends on
//   qcal_lds_copy global -> LDS copies (buffer_load_dwordx4 ... lds, 1 KiB per
//                 instruction) of a 64 KiB L2-resident block, repeated: the per-CU operand
//                 copy rate the prefill GEMM's k loop depends on
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr;

__global__ void empty_kernel() {}

__global__ __launch_bounds__(512) void stream_kernel(const uint4* __restrict__ p, int64_t n16, uint32_t* sink) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = per * blockIdx.x, b1 = b0 + per < n16 ? b0 + per : n16;
    uint32_t x = 0;
    for (int64_t i = b0 + threadIdx.x; i < b1; i += 8 * 512) {
        uint4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = i + j * 512 < b1 ? p[i + j * 512] : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    if (x == 0x9e3779b9u) sink[0] = x;  // keeps the loads; practically never stored
}

__global__ __launch_bounds__(256) void mfma_kernel(int iters, int* out) {
    const int lane = threadIdx.x & 63;
    v4i a = {lane, lane + 1, lane + 2, lane + 3}, b = {3 * lane, 5, 7, lane};
    v4i c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
    for (int i = 0; i < iters; ++i) {
        c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c3, 0, 0, 0);
    }
    const v4i s = c0 + c1 + c2 + c3;
    if (s[0] == 0x7fffffff) out[0] = s[1];  // keeps the products
}

// Reads `bytes` once, split evenly over `grid` workgroups of 512 threads, as direct
// 16-byte-per-lane copies into LDS: each wave keeps 8 copies (8 KiB) in flight in its
// own 8 KiB of LDS.
__global__ __launch_bounds__(512) void stream_lds_kernel(const uint8_t* p, int64_t bytes, int* out) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t per = (bytes / 16 + gridDim.x - 1) / gridDim.x * 16;
    const int64_t b0 = per * blockIdx.x;
    const int64_t b1 = b0 + per < bytes ? b0 + per : bytes;
    // a resource over this workgroup's range: copies past its end read zeros
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(p + (b0 < bytes ? b0 : 0)), (short)0, (int)(b1 > b0 ? b1 - b0 : 0), 0x00020000);
    const int64_t n = b1 - b0;
    for (int64_t o = (int64_t)wave * 8192; o < n; o += 8 * 8192) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(smem + wave * 8192 + j * 1024), 16,
                                                     (int)(o + j * 1024 + lane * 16), 0, 0, 0);
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0)
    }
    __syncthreads();
    if (smem[threadIdx.x] == 0xAB && smem[threadIdx.x + 1] == 0xCD && threadIdx.x == 0) out[0] = 1;
}

// Each wave copies its 8 KiB of a 64 KiB block into LDS, `iters` times.
__global__ __launch_bounds__(512) void lds_copy_kernel(const uint8_t* src, int iters, int* out) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), (short)0, 64 * 1024, 0x00020000);
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(smem + (wave * 8 + j) * 1024), 16,
                                                     (wave * 8 + j) * 1024 + lane * 16, 0, 0, 0);
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): this round's copies have landed
    }
    __syncthreads();
    if (smem[threadIdx.x] == 0xAB && smem[threadIdx.x + 1] == 0xCD && threadIdx.x == 0) out[0] = 1;
}

}  // namespace

extern "C" {

int qcal_empty(int grid, int threads, void* stream) {
    hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(threads), 0, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int qcal_stream(const void* p, int64_t bytes, int grid, uint32_t* sink, void* stream) {
    hipLaunchKernelGGL(stream_kernel, dim3(grid), dim3(512), 0, (hipStream_t)stream, (const uint4*)p, bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int qcal_mfma(int grid, int iters, int* out, void* stream) {
    hipLaunchKernelGGL(mfma_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, iters, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int qcal_stream_lds(const void* p, int64_t bytes, int grid, int* out, void* stream) {
    if (bytes <= 0 || bytes / grid >= ((int64_t)1 << 31)) return -1;
    hipLaunchKernelGGL(stream_lds_kernel, dim3(grid), dim3(512), 64 * 1024, (hipStream_t)stream, (const uint8_t*)p, bytes,
                       out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int qcal_lds_copy(const void* src, int grid, int iters, int* out, void* stream) {
    hipLaunchKernelGGL(lds_copy_kernel, dim3(grid), dim3(512), 64 * 1024, (hipStream_t)stream, (const uint8_t*)src,
                       iters, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
