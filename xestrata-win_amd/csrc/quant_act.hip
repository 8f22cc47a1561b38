// xestrata-win_amd/csrc/quant_act.hip - activations to q8_1 with the canonical scale (reference
// src/kernels/xe/iq_kernels.cpp:1850-1879 and, for rows not a whole number of 256s, :1209-1223).
//
// Rows of whole 256s: one scale for each 256 values, stored in each of their eight q8_1 blocks; a block's fp16 sum is
// its four 8-value partial sums (each serial) combined by the xor-1 then xor-2 exchange.  Other rows: a scale and a
// xor-16..1 butterfly sum for each 32.  Both are the reference's bits.
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_route.h"

namespace xs {

// 8 values a lane, 32 lanes = 256 values; a wave64 holds two 256-value groups
__global__ void quantize_q8_1_256_kernel(const float* __restrict__ x, int64_t n8, uint8_t* __restrict__ y) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    q8_1_256_lane(x, j, j < n8, y);
}

// one lane a value, 32 lanes a block
__global__ void quantize_q8_1_32_kernel(const float* __restrict__ x, int64_t n, uint8_t* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const float xi = i < n ? x[i] : 0.0f;
    const float amax = group_max<32>(fabsf(xi));
    const float sum = group_sum<32>(xi);
    if (i >= n) return;
    const float d = q8_scale(amax);
    const int64_t ib = i / 32, iqs = i % 32;
    y[36 * ib + 4 + iqs] = (uint8_t)q8_value(xi, q8_inv(d));
    if (iqs == 0) {
        const uint32_t ds = (uint32_t)f2h(d) | ((uint32_t)f2h(q8_1_finite(sum)) << 16);
        *(uint32_t*)(y + 36 * ib) = ds;
    }
}

hipError_t launch_quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, void* y, hipStream_t s) {
    const int64_t n = n_rows * n_cols;
    if (n <= 0) return hipSuccess;
    if (n_cols % 256 == 0) {
        const int64_t n8 = n / 8;
        hipLaunchKernelGGL(quantize_q8_1_256_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, x, n8,
                           (uint8_t*)y);
    } else {
        hipLaunchKernelGGL(quantize_q8_1_32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n,
                           (uint8_t*)y);
    }
    return hipGetLastError();
}

}  // namespace xs
