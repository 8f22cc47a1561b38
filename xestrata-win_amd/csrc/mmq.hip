// xestrata-win_amd/csrc/mmq.hip - the prompt path's activation staging with the reference's int8 MMQ contract
// (include/strata/kernels/iq_mmq.hpp:33-50, src/kernels/xe/iq_mmq.cpp:1264-1341) and the small row kernels its
// prompt section calls between products (src/prefill/moe_mmq.cpp:128-140).
//
// Activation layout for `rows` rows of `oc` values (oc = cols, or 2 cols when every block is written twice):
//   int8  q[rows][oc]          the values, 32 a block
//   float d[rows][oc / 32]     the block scale amax / 127
//   float s[rows][oc / 32]     d * (sum of the block's q), written only when asked for
// A block: d = amax / 127 (IEEE division), id = 1 / d (0 for an all-zero block), q = round-half-away(v * id).
//
// Eight lanes take a block (a float4 each), so a wave quantizes 8 blocks at once: the block maximum and the code sum
// are three xor steps inside the eight lanes; a lane stores its four codes as one word and lane 0 of the eight the
// block's scale and sum.  The scatter form quantizes a token's row once and stores the block at each of the token's
// k_used rows (slot[t * k_used + j]).
#include "xs_device.h"
#include "xs_kernels.h"

namespace xs {

__device__ __forceinline__ float oct_max(float v) {   // over the 8 lanes of an aligned octet
    v = fmaxf(v, __shfl_xor(v, 1, 64));
    v = fmaxf(v, __shfl_xor(v, 2, 64));
    return fmaxf(v, __shfl_xor(v, 4, 64));
}
__device__ __forceinline__ int oct_sum(int v) {
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    return v + __shfl_xor(v, 4, 64);
}

__device__ __forceinline__ int round_away(float v) { return (int)roundf(v); }   // halves away from zero

// one thread per 4 values: item i covers values 4 (i % (8 nb)) .. of source row i / (8 nb)
template <bool SCATTER>
__global__ __launch_bounds__(256) void mmq_quantize_kernel(const float* __restrict__ x, const int32_t* __restrict__ map,
                                                           int8_t* __restrict__ q, float* __restrict__ d_out,
                                                           float* __restrict__ s_out, int64_t nb, int64_t ld,
                                                           int64_t n_src, int k_used, int rep, bool sums) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_row = nb * 8;
    const int64_t r = i / per_row, within = i - r * per_row;
    const bool live = r < n_src;
    const int64_t b = within >> 3;
    const int part = (int)(within & 7);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (live) {
        const int64_t xr = SCATTER ? r : (map ? (int64_t)map[r] : r);
        v = *(const float4*)(x + xr * ld + b * 32 + 4 * part);
    }
    const float amax = oct_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float d = amax / 127.0f;
    const float id = amax > 0.0f ? 1.0f / d : 0.0f;
    const int q0 = round_away(v.x * id), q1 = round_away(v.y * id), q2 = round_away(v.z * id),
              q3 = round_away(v.w * id);
    const int sum = oct_sum(q0 + q1 + q2 + q3);
    if (!live) return;
    const uint32_t word = (uint32_t)(uint8_t)(int8_t)q0 | (uint32_t)(uint8_t)(int8_t)q1 << 8 |
                          (uint32_t)(uint8_t)(int8_t)q2 << 16 | (uint32_t)(uint8_t)(int8_t)q3 << 24;
    const int64_t onb = nb * rep, oc = onb * 32;
    const int n_dst = SCATTER ? k_used : 1;
    for (int j = 0; j < n_dst; ++j) {
        const int64_t row = SCATTER ? (int64_t)map[r * k_used + j] : r;
        for (int c = 0; c < rep; ++c) {
            const int64_t ob = b * rep + c;
            *(uint32_t*)(q + row * oc + ob * 32 + 4 * part) = word;
            if (part == 0) {
                d_out[row * onb + ob] = d;
                if (sums) s_out[row * onb + ob] = d * (float)sum;
            }
        }
    }
}

hipError_t launch_mmq_quantize(const float* x, const int32_t* map, void* xq, int64_t cols, int64_t ld, int64_t n_src,
                               int64_t rows, int k_used, bool scatter, bool sums, bool dup, hipStream_t s) {
    const int rep = dup ? 2 : 1;
    const int64_t nb = cols / 32, oc = cols * rep;
    int8_t* q = (int8_t*)xq;
    float* d_out = (float*)(q + rows * oc);
    float* s_out = d_out + rows * (oc / 32);
    const int64_t items = n_src * nb * 8;
    const dim3 grid((unsigned)((items + 255) / 256));
    if (scatter)
        hipLaunchKernelGGL(mmq_quantize_kernel<true>, grid, dim3(256), 0, s, x, map, q, d_out, s_out, nb, ld, n_src,
                           k_used, rep, sums);
    else
        hipLaunchKernelGGL(mmq_quantize_kernel<false>, grid, dim3(256), 0, s, x, map, q, d_out, s_out, nb, ld, n_src,
                           1, rep, sums);
    return hipGetLastError();
}

// h[r, j] = g / (1 + exp(-g)) * u over rows of 2 n_ff values: gate j and up j interleaved (2j, 2j + 1) or split
// (j, n_ff + j)
__global__ __launch_bounds__(256) void mmq_swiglu_kernel(const float* __restrict__ gu, float* __restrict__ h,
                                                         int64_t n, int64_t n_ff, bool interleaved) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / n_ff, j = i - r * n_ff;
    const float* row = gu + r * 2 * n_ff;
    const float g = interleaved ? row[2 * j] : row[j];
    const float u = interleaved ? row[2 * j + 1] : row[n_ff + j];
    h[i] = g / (1.0f + expf(-g)) * u;
}

hipError_t launch_mmq_swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, bool interleaved, hipStream_t s) {
    const int64_t n = rows * n_ff;
    hipLaunchKernelGGL(mmq_swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gu, h, n, n_ff,
                       interleaved);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void iota_kernel(int32_t* __restrict__ dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = (int32_t)i;
}

hipError_t launch_iota(int32_t* dst, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(iota_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst, n);
    return hipGetLastError();
}

}  // namespace xs
