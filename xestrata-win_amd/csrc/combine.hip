// xestrata-win_amd/csrc/combine.hip - the weighted combine of a token's expert outputs, back into the residual stream
// (reference src/kernels/xe/native_moe.cpp:36-58, and add_inplace at src/core/plain_model.cpp:987).
//
// out[t, c] = fl(p0 w0), then + fl(pj wj) for j = 1..k-1 in rank order (each product rounded: no fused multiply-add),
// then + shared[t, c] (scaled by 1 / (1 + exp(-gate[t])), that product rounded, when gated), then, when a residual is
// given, residual[t, c] + that.  A gather over the routing-order parts: no atomics, one thread a column.
#include "xs_device.h"
#include "xs_kernels.h"

#include <type_traits>

namespace xs {

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ parts, const float* __restrict__ weights,
                                                      const float* __restrict__ shared,
                                                      const float* __restrict__ shared_gate,
                                                      const float* __restrict__ residual, float* __restrict__ out,
                                                      int64_t n_embd, int k) {
    const int64_t t = blockIdx.y;
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n_embd) return;
    const float* p = parts + t * k * n_embd + c;
    const float* w = weights + t * k;
    float sum = p[0] * w[0];
    for (int e = 1; e < k; ++e) {
        const float prod = p[(int64_t)e * n_embd] * w[e];
        sum = sum + prod;
    }
    if (shared) {
        float sv = shared[t * n_embd + c];
        if (shared_gate) {
            const float gt = 1.0f / (1.0f + expf(-shared_gate[t]));
            sv = sv * gt;
        }
        sum += sv;
    }
    if (residual) sum = residual[t * n_embd + c] + sum;
    out[t * n_embd + c] = sum;
}

__global__ __launch_bounds__(256) void add_inplace_kernel(float* __restrict__ x, const float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

// The same sum over f16 parts (the prompt layer's, whose products are f16 MFMA results anyway), plus the residual:
// 4 columns a thread (8-byte part reads, 16-byte residual and output accesses).
// V columns a thread (8: 16-byte loads of the f16 parts, when n_embd allows; else 4); every column's sum in the same
// order either way
template <int V>
__global__ __launch_bounds__(256) void combine_h_kernel(const uint16_t* __restrict__ parts,
                                                        const float* __restrict__ weights,
                                                        const float* __restrict__ shared,
                                                        const float* __restrict__ shared_gate,
                                                        const float* __restrict__ residual, float* __restrict__ out,
                                                        int64_t n_embd, int k) {
    using PV = typename std::conditional<V == 8, uint4, uint2>::type;
    const int64_t t = blockIdx.y;
    const int64_t c = V * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (c >= n_embd) return;
    const uint16_t* p = parts + t * k * n_embd + c;
    const float* w = weights + t * k;
    float sum[V];
    for (int e = 0; e < k; ++e) {
        const PV v = *(const PV*)(p + (int64_t)e * n_embd);
        const uint32_t* vw = (const uint32_t*)&v;
        const float we = w[e];
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const float prod = h2f((uint16_t)(vw[i / 2] >> (16 * (i & 1)))) * we;
            sum[i] = e == 0 ? prod : sum[i] + prod;
        }
    }
    if (shared) {   // the shared expert's row, once, after the routed ones (times its gate's sigmoid)
        const float gs = shared_gate ? 1.0f / (1.0f + expf(-shared_gate[t])) : 1.0f;
#pragma unroll
        for (int i = 0; i < V; i += 4) {
            const float4 sv = *(const float4*)(shared + t * n_embd + c + i);
            sum[i] = sum[i] + (shared_gate ? sv.x * gs : sv.x);
            sum[i + 1] = sum[i + 1] + (shared_gate ? sv.y * gs : sv.y);
            sum[i + 2] = sum[i + 2] + (shared_gate ? sv.z * gs : sv.z);
            sum[i + 3] = sum[i + 3] + (shared_gate ? sv.w * gs : sv.w);
        }
    }
#pragma unroll
    for (int i = 0; i < V; i += 4) {
        const float4 r = *(const float4*)(residual + t * n_embd + c + i);
        *(float4*)(out + t * n_embd + c + i) =
            make_float4(r.x + sum[i], r.y + sum[i + 1], r.z + sum[i + 2], r.w + sum[i + 3]);
    }
}

// native_moe_combine_multi with moe_hit_add folded in (the reference's native_moe_combine_multi_hits,
// src/kernels/xe/native_moe.cpp:67-110): a work-group of token t marks which of its k entries are listed in
// dst[0, *count), and those read parts + hits (the sum moe_hit_add leaves in place) before their product
__global__ __launch_bounds__(256) void combine_hits_kernel(const float* __restrict__ parts, const float* __restrict__ hits,
                                                           const int32_t* __restrict__ dst,
                                                           const int32_t* __restrict__ count,
                                                           const float* __restrict__ weights,
                                                           const float* __restrict__ shared,
                                                           const float* __restrict__ shared_gate,
                                                           float* __restrict__ out, int64_t n_embd, int k) {
    __shared__ int hit[16];
    const int64_t t = blockIdx.y;
    const int tid = threadIdx.x;
    if (tid < 16) hit[tid] = 0;
    __syncthreads();
    const int n_hit = *count, lo = (int)(t * k);
    for (int i = tid; i < n_hit; i += blockDim.x) {
        const int e = dst[i] - lo;
        if (e >= 0 && e < k) hit[e] = 1;
    }
    __syncthreads();
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + tid;
    if (c >= n_embd) return;
    const float* p = parts + t * k * n_embd + c;
    const float* hp = hits + t * k * n_embd + c;
    const float* w = weights + t * k;
    float sum = 0.0f;
    for (int e = 0; e < k; ++e) {
        const float pe = hit[e] ? p[(int64_t)e * n_embd] + hp[(int64_t)e * n_embd] : p[(int64_t)e * n_embd];
        const float prod = pe * w[e];
        sum = e == 0 ? prod : sum + prod;
    }
    if (shared) {
        float sv = shared[t * n_embd + c];
        if (shared_gate) sv = sv * (1.0f / (1.0f + expf(-shared_gate[t])));
        sum = sum + sv;
    }
    out[t * n_embd + c] = sum;
}

hipError_t launch_combine_hits(const float* parts, const float* hits, const int32_t* dst, const int32_t* count,
                               const float* weights, const float* shared, const float* shared_gate, float* out,
                               int64_t n_embd, int k, int n_tok, hipStream_t s) {
    const dim3 grid((unsigned)((n_embd + 255) / 256), (unsigned)n_tok);
    hipLaunchKernelGGL(combine_hits_kernel, grid, dim3(256), 0, s, parts, hits, dst, count, weights, shared,
                       shared_gate, out, n_embd, k);
    return hipGetLastError();
}

hipError_t launch_combine_h(const uint16_t* parts, const float* weights, const float* shared,
                            const float* shared_gate, const float* residual, float* out, int64_t n_embd, int k,
                            int n_tok, hipStream_t s) {
    if (n_embd % 8 == 0) {
        const dim3 grid((unsigned)((n_embd / 8 + 255) / 256), (unsigned)n_tok);
        hipLaunchKernelGGL(combine_h_kernel<8>, grid, dim3(256), 0, s, parts, weights, shared, shared_gate, residual,
                           out, n_embd, k);
    } else {
        const dim3 grid((unsigned)((n_embd / 4 + 255) / 256), (unsigned)n_tok);
        hipLaunchKernelGGL(combine_h_kernel<4>, grid, dim3(256), 0, s, parts, weights, shared, shared_gate, residual,
                           out, n_embd, k);
    }
    return hipGetLastError();
}

hipError_t launch_combine(const float* parts, const float* weights, const float* shared, const float* shared_gate,
                          const float* residual, float* out, int64_t n_embd, int k, int n_tok, hipStream_t s) {
    const dim3 grid((unsigned)((n_embd + 255) / 256), (unsigned)n_tok);
    hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, s, parts, weights, shared, shared_gate, residual, out, n_embd,
                       k);
    return hipGetLastError();
}

hipError_t launch_add_inplace(float* x, const float* y, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(add_inplace_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

}  // namespace xs
