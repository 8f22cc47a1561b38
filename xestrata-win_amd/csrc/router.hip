// xestrata-win_amd/csrc/router.hip - MoE routing on the device: the reference's softmax top-k router, a DeepSeek-V3
// style grouped sigmoid router (absent from the reference), and the f32 router-logit GEMV feeding them.
#include "xs_device.h"
#include "xs_kernels.h"

namespace xs {

constexpr int kRouterMaxPer = 16;   // experts a lane: one wave covers up to 1024 experts

// the argmax order: the larger value wins, a tie keeps the lower index; NaN never wins (reference
// src/kernels/xe/router.cpp:32-36)
__device__ __forceinline__ void better(float& bv, int& bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

// Softmax top-k, bit for bit the reference's router_top10 (src/kernels/xe/router.cpp:59-145 and its fast form
// :146-276): mx = max l; ex = exp((double) l - (double) mx); inv = (float) (1 / sum ex) with the sum serial and
// ascending in double; p = (float) (ex * inv); k passes of argmax; renormalised in double by max(sum of the k,
// 2^-14).  One wave a token.  The serial sum is only run when a tree sum cannot decide inv: the serial and tree sums
// both lie within 2^-43 of the exact sum (every term is positive, the largest is exactly 1), so when the bracket
// tree * (1 -+ 2^-40) maps to one float inv, that float is the serial sum's.
__global__ __launch_bounds__(64) void router_topk_kernel(const float* __restrict__ logits, int n_expert, int k,
                                                         int32_t* __restrict__ ids, float* __restrict__ weights) {
    const int t = blockIdx.x, lane = threadIdx.x;
    const float* l = logits + (int64_t)t * n_expert;
    float lv[kRouterMaxPer];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRouterMaxPer; ++j) {
        const int x = lane + 64 * j;
        lv[j] = x < n_expert ? l[x] : -INFINITY;
        if (x < n_expert) mx = fmaxf(mx, lv[j]);
    }
    mx = group_max<64>(mx);
    double ex[kRouterMaxPer];
    double part = 0.0;
#pragma unroll
    for (int j = 0; j < kRouterMaxPer; ++j) {
        const int x = lane + 64 * j;
        ex[j] = x < n_expert ? exp((double)lv[j] - (double)mx) : 0.0;
        part += ex[j];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
    const double lo = part * (1.0 - 0x1p-40), hi = part * (1.0 + 0x1p-40);
    const float f_lo = (float)(1.0 / hi), f_hi = (float)(1.0 / lo);
    float inv;
    if (part >= 1.0 && hi < 1e300 && f_lo == f_hi) {
        inv = f_lo;
    } else {   // uniform over the wave: the serial ascending sum
        double sum = 0.0;
        for (int j = 0; j < kRouterMaxPer; ++j) {
            if (64 * j >= n_expert) break;
            for (int s = 0; s < 64 && 64 * j + s < n_expert; ++s) sum += __shfl(ex[j], s, 64);
        }
        inv = (float)(1.0 / sum);
    }
    float pv[kRouterMaxPer];
    uint32_t live = 0;
#pragma unroll
    for (int j = 0; j < kRouterMaxPer; ++j) {
        const int x = lane + 64 * j;
        pv[j] = -INFINITY;
        if (x < n_expert) { pv[j] = (float)(ex[j] * (double)inv); live |= 1u << j; }
    }
    float my_w = 0.0f;
    int my_id = 0, nsel = 0;
    for (int i = 0; i < k; ++i) {
        float bv = -INFINITY;
        int bi = n_expert;
#pragma unroll
        for (int j = 0; j < kRouterMaxPer; ++j)
            if (((live >> j) & 1u) && pv[j] > bv) { bv = pv[j]; bi = lane + 64 * j; }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) better(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
        if (bi >= n_expert) break;   // every p left is NaN: ranks i.. keep the buffer's contents
        if ((bi & 63) == lane) live &= ~(1u << (bi >> 6));
        if (lane == i) { my_w = bv; my_id = bi; }
        nsel = i + 1;
    }
    int32_t* id_row = ids + (int64_t)t * k;
    float* w_row = weights + (int64_t)t * k;
    if (nsel == k) {
        double s = 0.0;
        for (int i = 0; i < k; ++i) s += (double)__shfl(my_w, i, 64);
        const double sc = fmax(s, 6.103515625e-05);
        if (lane < k) {
            id_row[lane] = my_id;
            w_row[lane] = (float)((double)my_w / sc);
        }
    } else {
        if (lane < nsel) { id_row[lane] = my_id; w_row[lane] = my_w; }
        __threadfence_block();
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {
            double s = 0.0;
            for (int i = 0; i < k; ++i) s += (double)w_row[i];
            const double sc = fmax(s, 6.103515625e-05);
            for (int i = 0; i < k; ++i) w_row[i] = (float)((double)w_row[i] / sc);
        }
    }
}

// DeepSeek-V3 routing (its technical report: sigmoid affinities, a selection bias, group-limited top-k): s =
// sigmoid(l) with the canonical exp and reciprocal (the same bits on the host); selection score c = s + bias; a
// group's score is the sum of its two best c; the topk_group best groups, then the k best c inside them (ties: the
// lower index, NaN never wins); weights = s / (sum of the chosen s, in rank order) * routed_scale.  One wave a token.
__global__ __launch_bounds__(64) void router_grouped_sigmoid_kernel(const float* __restrict__ logits,
                                                                    const float* __restrict__ bias, int n_expert,
                                                                    int n_group, int topk_group, int k,
                                                                    float routed_scale, int32_t* __restrict__ ids,
                                                                    float* __restrict__ weights) {
    __shared__ float s_c[1024];
    __shared__ float s_s[1024];
    __shared__ float s_g[64];
    __shared__ int s_gsel[64];
    const int t = blockIdx.x, lane = threadIdx.x;
    const float* l = logits + (int64_t)t * n_expert;
    for (int e = lane; e < n_expert; e += 64) {
        const float s = canon_rcp(1.0f + canon_exp(-l[e]));
        s_s[e] = s;
        s_c[e] = s + (bias ? bias[e] : 0.0f);
    }
    __syncthreads();
    const int per = n_expert / n_group;
    if (lane < n_group) {
        float b1 = -INFINITY, b2 = -INFINITY;
        for (int j = 0; j < per; ++j) {
            const float v = s_c[lane * per + j];
            if (v > b1) { b2 = b1; b1 = v; }
            else if (v > b2) b2 = v;
        }
        s_g[lane] = b1 + b2;
        s_gsel[lane] = 0;
    }
    __syncthreads();
    for (int i = 0; i < topk_group; ++i) {
        float bv = -INFINITY;
        int bi = 1 << 30;
        if (lane < n_group && !s_gsel[lane]) { bv = s_g[lane]; bi = lane; }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) better(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
        if (lane == 0 && bi < n_group) s_gsel[bi] = 1;
        __syncthreads();
    }
    float my_w = 0.0f;
    int my_id = 0;
    for (int i = 0; i < k; ++i) {
        float bv = -INFINITY;
        int bi = 1 << 30;
        for (int e = lane; e < n_expert; e += 64)
            if (s_gsel[e / per]) better(bv, bi, s_c[e], e);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) better(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
        if (bi >= n_expert) break;
        if (lane == 0) s_c[bi] = -INFINITY;   // taken
        if (lane == i) { my_w = s_s[bi]; my_id = bi; }
        __syncthreads();
    }
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) sum += __shfl(my_w, i, 64);
    if (lane < k) {
        ids[(int64_t)t * k + lane] = my_id;
        weights[(int64_t)t * k + lane] = my_w / sum * routed_scale;
    }
}

// logits[t, e] = x[t] . w[e] in fp32 (the router GEMV, reference src/kernels/xe/bf16_gemv.cpp:495-517): a wave per
// (expert, token), lanes over the row, then a butterfly
__global__ __launch_bounds__(256) void logits_f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         float* __restrict__ logits, int n_tokens, int64_t n_embd,
                                                         int n_expert) {
    const int wave = (int)(blockIdx.x * 4 + (threadIdx.x >> 6)), lane = threadIdx.x & 63;
    if (wave >= n_expert * n_tokens) return;
    const int e = wave % n_expert, t = wave / n_expert;
    const float* wr = w + (int64_t)e * n_embd;
    const float* xr = x + (int64_t)t * n_embd;
    float acc = 0.0f;
    for (int64_t i = lane; i < n_embd; i += 64) acc = __builtin_fmaf(wr[i], xr[i], acc);
    acc = group_sum<64>(acc);
    if (lane == 0) logits[(int64_t)t * n_expert + e] = acc;
}

hipError_t launch_router_topk(const float* logits, int n_tokens, int n_expert, int k, int32_t* ids, float* weights,
                              hipStream_t s) {
    hipLaunchKernelGGL(router_topk_kernel, dim3((unsigned)n_tokens), dim3(64), 0, s, logits, n_expert, k, ids, weights);
    return hipGetLastError();
}

hipError_t launch_router_grouped_sigmoid(const float* logits, const float* bias, int n_tokens, int n_expert,
                                         int n_group, int topk_group, int k, float routed_scale, int32_t* ids,
                                         float* weights, hipStream_t s) {
    hipLaunchKernelGGL(router_grouped_sigmoid_kernel, dim3((unsigned)n_tokens), dim3(64), 0, s, logits, bias, n_expert,
                       n_group, topk_group, k, routed_scale, ids, weights);
    return hipGetLastError();
}

hipError_t launch_logits_f32(const float* x, const float* w, float* logits, int n_tokens, int64_t n_embd,
                             int n_expert, hipStream_t s) {
    const int64_t waves = (int64_t)n_tokens * n_expert;
    hipLaunchKernelGGL(logits_f32_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, w, logits, n_tokens,
                       n_embd, n_expert);
    return hipGetLastError();
}

}  // namespace xs
