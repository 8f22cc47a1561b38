// xestrata-win_amd/csrc/tiers.hip - the tier protocol's device steps (include/xs_tiers.h): the flag wait, the copies
// out of mapped host memory, the PCIe share's staging and the hit rows' add (reference
// src/kernels/xe/verify_kernels.cpp:783-788, 1051-1068; src/kernels/xe/elementwise.cpp:196-257;
// src/kernels/xe/s2_expert_grouped.cpp:913-925).
//
// All of it is data movement, bound by PCIe (mapped host reads) or HBM.  Reads of memory the host writes while the
// layer runs (the flag, the plan, the CPU's rows) are volatile, so each goes to memory at system scope rather than
// to a cache line an earlier read filled.
#include "../../include/xs_moe.h"
#include "../../include/xs_tiers.h"
#include "xs_device.h"
#include "xs_error.h"

#include <hip/hip_runtime.h>

#include <string>

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// one thread polls the flag, sleeping a little between reads, until it reaches `value` or the wall clock passes the
// bound; then the acquire that orders the host's earlier writes before everything after this kernel
__global__ void wait_flag_kernel(const uint32_t* flag, uint32_t value, long long ticks, int32_t* status) {
    if (threadIdx.x != 0) return;
    const long long t0 = wall_clock64();
    while (*(const volatile uint32_t*)flag < value) {
        if (wall_clock64() - t0 > ticks) {
            if (status) *status = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    __atomic_thread_fence(__ATOMIC_ACQUIRE);
}

__global__ __launch_bounds__(256) void copy_i32_mapped_kernel(int32_t* __restrict__ dst, const int32_t* src, int64_t n,
                                                              int vec) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x, g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t done = 0;
    if (vec) {
        const int64_t n4 = n / 4;
        for (int64_t i = g; i < n4; i += step) ((i32x4*)dst)[i] = ((const volatile i32x4*)src)[i];
        done = 4 * n4;
    }
    for (int64_t i = done + g; i < n; i += step) dst[i] = ((const volatile int32_t*)src)[i];
}

// one work-group (two waves) a row: whether the row is a hit is decided by the whole group, then 16-byte copies
__global__ __launch_bounds__(128) void copy_rows_mapped_kernel(float* __restrict__ dst, const float* src, int64_t width,
                                                               const int32_t* __restrict__ hit_rows,
                                                               const int32_t* __restrict__ count) {
    const int64_t row = blockIdx.x;
    const int c = *count;
    int h = 0;
    for (int i = threadIdx.x; i < c; i += 128) h |= hit_rows[i] == row;
    const bool hit = __syncthreads_or(h) != 0;
    f32x4* d = (f32x4*)(dst + row * width);
    const volatile f32x4* s = (const volatile f32x4*)(src + row * width);
    const int64_t w4 = width / 4;
    for (int64_t i = threadIdx.x; i < w4; i += 128) d[i] = hit ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : s[i];
}

// blob k = blockIdx.y; the x work-groups stride over its 16-byte words (no division a word)
__global__ __launch_bounds__(256) void fetch_blobs_kernel(const unsigned long long* __restrict__ src,
                                                          const int32_t* __restrict__ n, u32x4* __restrict__ dst,
                                                          long long per) {
    const int k = blockIdx.y;
    if (k >= *n) return;
    const u32x4* s = (const u32x4*)src[k];
    u32x4* d = dst + (long long)k * per;
    const long long step = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < per; i += step) d[i] = s[i];
}

__global__ __launch_bounds__(128) void rebase_ptrs_kernel(unsigned long long* __restrict__ ptr,
                                                          const int32_t* __restrict__ n, unsigned long long base,
                                                          unsigned long long bytes) {
    const int k = threadIdx.x;
    if (k < *n) ptr[k] = base + (unsigned long long)k * bytes;
}

__global__ __launch_bounds__(256) void hit_add_kernel(float* __restrict__ parts, const float* __restrict__ hit_out,
                                                      const int32_t* __restrict__ dst,
                                                      const int32_t* __restrict__ count, int64_t n_embd) {
    const int h = blockIdx.y;
    if (h >= *count) return;
    const int64_t row = (int64_t)dst[h] * n_embd;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_embd; i += step)
        parts[row + i] = parts[row + i] + hit_out[row + i];
}

int fail(int code, const std::string& m) { return xs::set_error(code, m); }

int launched(void* stream, const char* what) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && !stream) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return fail(XS_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
    return XS_OK;
}

bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" {

int xs_wait_flag_ge(const uint32_t* flag, uint32_t value, int64_t limit_us, int32_t* status, void* stream) {
    if (!flag) return fail(XS_EINVAL, "wait_flag_ge: no flag");
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess ||
        khz <= 0)
        khz = 100000;
    const long long us = limit_us > 0 ? (limit_us < 3600000000ll ? (long long)limit_us : 3600000000ll) : 10000000ll;
    const long long ticks = us * (long long)khz / 1000;
    hipLaunchKernelGGL(wait_flag_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, flag, value, ticks, status);
    return launched(stream, "wait_flag_ge");
}

int xs_copy_i32_from_mapped(int32_t* dst, const int32_t* src, int64_t n, void* stream) {
    if (n <= 0) return XS_OK;
    if (!dst || !src) return fail(XS_EINVAL, "copy_i32_from_mapped: no buffer");
    const int vec = a16(dst) && a16(src);
    const int64_t units = vec ? (n + 3) / 4 : n;
    const int groups = (int)std::min<int64_t>(std::max<int64_t>((units + 255) / 256, 1), 64);
    hipLaunchKernelGGL(copy_i32_mapped_kernel, dim3(groups), dim3(256), 0, (hipStream_t)stream, dst, src, n, vec);
    return launched(stream, "copy_i32_from_mapped");
}

int xs_copy_rows_from_mapped(float* dst, const float* src, int64_t rows, int64_t width, const int32_t* hit_rows,
                             const int32_t* count, void* stream) {
    if (rows <= 0) return XS_OK;
    if ((width & 3) != 0 || !a16(dst) || !a16(src) || width <= 0)
        return fail(XS_EINVAL, "copy_rows_from_mapped: width must be a multiple of 4 and both pointers 16-byte aligned");
    if (!hit_rows || !count) return fail(XS_EINVAL, "copy_rows_from_mapped: no hit rows or count");
    if (rows > 0x7fffffff) return fail(XS_EINVAL, "copy_rows_from_mapped: too many rows");
    hipLaunchKernelGGL(copy_rows_mapped_kernel, dim3((unsigned)rows), dim3(128), 0, (hipStream_t)stream, dst, src, width,
                       hit_rows, count);
    return launched(stream, "copy_rows_from_mapped");
}

int xs_fetch_blobs(const unsigned long long* src, const int32_t* n, uint8_t* dst, int64_t blob_bytes, int cap,
                   void* stream) {
    if (cap <= 0) return XS_OK;
    if (blob_bytes <= 0 || blob_bytes % 16 != 0) return fail(XS_EINVAL, "fetch_blobs: blob size must be a multiple of 16");
    if (!src || !n || !a16(dst)) return fail(XS_EINVAL, "fetch_blobs: no source table or count, or dst not 16-byte aligned");
    if (cap > 65535) return fail(XS_EINVAL, "fetch_blobs: more than 65535 blobs");
    const long long per = blob_bytes / 16;
    // about 512 work-groups in all (two a CU), never more than a blob's words need
    const long long gx = std::max<long long>(1, std::min<long long>((per + 255) / 256, std::max(1, 512 / cap)));
    hipLaunchKernelGGL(fetch_blobs_kernel, dim3((unsigned)gx, (unsigned)cap), dim3(256), 0, (hipStream_t)stream, src, n,
                       (u32x4*)dst, per);
    return launched(stream, "fetch_blobs");
}

int xs_rebase_ptrs(unsigned long long* ptr, const int32_t* n, uint8_t* base, int64_t blob_bytes, void* stream) {
    if (!ptr || !n) return fail(XS_EINVAL, "rebase_ptrs: no table or count");
    hipLaunchKernelGGL(rebase_ptrs_kernel, dim3(1), dim3(128), 0, (hipStream_t)stream, ptr, n,
                       (unsigned long long)base, (unsigned long long)blob_bytes);
    return launched(stream, "rebase_ptrs");
}

int xs_moe_hit_add(float* parts, const float* hit_out, const int32_t* dst, const int32_t* count, int64_t cap,
                   int64_t n_embd, void* stream) {
    if (cap <= 0) return XS_OK;
    if (!parts || !hit_out || !dst || !count || n_embd <= 0) return fail(XS_EINVAL, "moe_hit_add: no buffer");
    if (cap > 65535) return fail(XS_EINVAL, "moe_hit_add: more than 65535 hits");
    const unsigned gx = (unsigned)std::min<int64_t>((n_embd + 255) / 256, 8);
    hipLaunchKernelGGL(hit_add_kernel, dim3(gx, (unsigned)cap), dim3(256), 0, (hipStream_t)stream, parts, hit_out, dst,
                       count, n_embd);
    return launched(stream, "moe_hit_add");
}

}  // extern "C"
