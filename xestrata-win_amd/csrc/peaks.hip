// xestrata-win_amd/csrc/peaks.hip - two measuring kernels for the achieved peaks the MoE kernels are compared with on
// the box they run on (the published MI355X figures are 8 TB/s of HBM and 2.5 PFLOP/s of dense f16/bf16 MFMA):
//
//  * hbm_read_kernel: reads `bytes` once (16-byte nontemporal loads, four in flight a lane, grid-stride over the whole
//    span) and folds them into one word a work-group, so nothing is written but grid-size words - the read-only
//    stream rate of HBM, and, over a span the size of one decode layer's experts, the one-launch rate;
//  * mfma_loop_kernel: v_mfma_f32_32x32x16_f16 back to back on eight independent accumulators a wave (enough to keep
//    the matrix pipe full: 32 cycles an instruction, a chain's next issue waits for its result), 2 waves a SIMD -
//    the dense rate the prompt GEMMs' instruction uses.
// No counterpart in the reference; used by bench.py's roofline lines.  lds_read_kernel measures the LDS read rate
// (the operand supply of LDS-fed MFMA tiles); occupy_kernel holds compute units for a bounded time (tests of the
// decode layer beside other work).
#include "../../include/xs_moe.h"
#include "xs_error.h"

#include <hip/hip_runtime.h>

#include <string>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4* __restrict__ src, size_t n16,
                                                       unsigned int* __restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * 256;
    unsigned int acc = 0;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 a = __builtin_nontemporal_load(src + i), b = __builtin_nontemporal_load(src + i + stride),
                    c = __builtin_nontemporal_load(src + i + 2 * stride),
                    d = __builtin_nontemporal_load(src + i + 3 * stride);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const u32x4 a = __builtin_nontemporal_load(src + i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    __shared__ unsigned int s_acc;
    if (threadIdx.x == 0) s_acc = 0;
    __syncthreads();
    atomicXor(&s_acc, acc);
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = s_acc;
}

__global__ __launch_bounds__(128) void mfma_loop_kernel(int iters, float* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    f16x8_t a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(0.001f * (float)(lane + i));
        b[i] = (_Float16)(0.002f * (float)(lane - i));
    }
    f32x16_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[j][q] = 0.0f;
    for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) s += acc[j][q];
    if (s == 12345.678f) sink[blockIdx.x * blockDim.x + threadIdx.x] = s;   // keeps the products live
}

// ds_read_b128 back to back from LDS, conflict-free (lane l reads 16 bytes at 16 l of its wave's 1 KB row, 8 rows a
// wave in turn), eight reads in flight a lane; folded into one word a work-group
__global__ __launch_bounds__(1024) void lds_read_kernel(int iters, unsigned int* __restrict__ sink) {
    __shared__ uint4 s_buf[64 * 128];   // 128 KB
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 64 * 128; i += 1024) s_buf[i] = make_uint4(i, i + 1, i + 2, i + 3);
    __syncthreads();
    uint4 acc = make_uint4(0, 0, 0, 0);
    const int base = (wave * 8) * 64 + lane;
    for (int it = 0; it < iters; ++it) {
        uint4 v[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = s_buf[(base + 64 * ((r + it) & 7)) & (64 * 128 - 1)];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            acc.x ^= v[r].x;
            acc.y ^= v[r].y;
            acc.z ^= v[r].z;
            acc.w ^= v[r].w;
        }
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678u) sink[blockIdx.x] = acc.x;
}

// holds its compute unit (its dynamic LDS) for `ticks` of the wall clock, then ends: a bounded stand-in for other
// work that owns part of the GPU while a layer runs
__global__ __launch_bounds__(64) void occupy_kernel(long long ticks, unsigned int* __restrict__ sink) {
    extern __shared__ unsigned int s_hold[];
    const long long t0 = wall_clock64();
    unsigned int n = 0;
    while (wall_clock64() - t0 < ticks) {
        __builtin_amdgcn_s_sleep(127);
        ++n;
    }
    s_hold[threadIdx.x] = n;
    __syncthreads();
    if (threadIdx.x == 0 && s_hold[1] == 0xFFFFFFFFu) sink[blockIdx.x] = n;   // (keeps the LDS allocation live)
}

}  // namespace

extern "C" {

int xs_bench_hbm_read(const void* src, size_t bytes, unsigned int* sink, int grid, void* stream) {
    if (!src || !sink || ((uintptr_t)src % 16) || bytes % 16 || grid <= 0)
        return xs::set_error(XS_EINVAL, "bench_hbm_read: a span is missing or misaligned, or grid <= 0");
    hipLaunchKernelGGL(hbm_read_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const u32x4*)src,
                       bytes / 16, sink);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? XS_OK : xs::set_error(XS_EDEVICE, std::string("bench_hbm_read: ") + hipGetErrorString(e));
}

int xs_bench_mfma_f16(int iters, int grid, float* sink, void* stream) {
    if (iters <= 0 || grid <= 0 || !sink) return xs::set_error(XS_EINVAL, "bench_mfma_f16: iters, grid or sink");
    hipLaunchKernelGGL(mfma_loop_kernel, dim3((unsigned)grid), dim3(128), 0, (hipStream_t)stream, iters, sink);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? XS_OK : xs::set_error(XS_EDEVICE, std::string("bench_mfma_f16: ") + hipGetErrorString(e));
}

int xs_bench_lds_read(int iters, int grid, unsigned int* sink, void* stream) {
    if (iters <= 0 || grid <= 0 || !sink) return xs::set_error(XS_EINVAL, "bench_lds_read: iters, grid or sink");
    hipLaunchKernelGGL(lds_read_kernel, dim3((unsigned)grid), dim3(1024), 0, (hipStream_t)stream, iters, sink);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? XS_OK : xs::set_error(XS_EDEVICE, std::string("bench_lds_read: ") + hipGetErrorString(e));
}

int xs_bench_occupy(int n_wg, int lds_bytes, long long ticks, unsigned int* sink, void* stream) {
    if (n_wg <= 0 || lds_bytes < 256 || lds_bytes > 160 * 1024 || ticks <= 0 || ticks > 2000000000ll || !sink)
        return xs::set_error(XS_EINVAL, "bench_occupy: work-groups, LDS (256 B .. 160 KB) or ticks (<= 20 s)");
    hipError_t e = hipFuncSetAttribute((const void*)occupy_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       lds_bytes);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(occupy_kernel, dim3((unsigned)n_wg), dim3(64), (size_t)lds_bytes, (hipStream_t)stream,
                           ticks, sink);
        e = hipGetLastError();
    }
    return e == hipSuccess ? XS_OK : xs::set_error(XS_EDEVICE, std::string("bench_occupy: ") + hipGetErrorString(e));
}

}  // extern "C"
