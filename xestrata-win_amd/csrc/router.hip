// xestrata-win_amd/csrc/router.hip - MoE routing on the device: the reference's softmax top-k router, a DeepSeek-V3
// style grouped sigmoid router (absent from the reference), and the f32 router-logit GEMV feeding them.
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_route.h"

namespace xs {


// Softmax top-k (the reference's router_top10, src/kernels/xe/router.cpp:59-308): one wave a token, route_topk_wave
template <int PER>
__global__ __launch_bounds__(64) void router_topk_kernel(const float* __restrict__ logits, int n_expert, int k,
                                                         int32_t* __restrict__ ids, float* __restrict__ weights) {
    const int t = blockIdx.x;
    route_topk_wave<PER>(logits + (int64_t)t * n_expert, n_expert, k, ids + (int64_t)t * k, weights + (int64_t)t * k);
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

// The same routing with the experts in registers, for shapes whose groups fall on whole lanes: lane l holds experts
// l PER .. l PER + PER - 1, so a group of per = n_expert / n_group experts is lpg = per / PER adjacent lanes (a power
// of two).  A group's two best c: each lane's two best, merged over the group's lanes by a xor butterfly (the pair of
// largest values does not depend on the order they are met in); the groups' ranks by v_readlane (score, then the
// lower group); the k best c by k argmax passes over the wave (better(): the same total order as above, so the same
// picks, a taken expert's c set to -inf as above).  Four tokens a work-group, one a wave.
template <int PER>
__global__ __launch_bounds__(256) void router_grouped_sigmoid_wave_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int n_tokens, int n_expert, int n_group,
    int topk_group, int k, float routed_scale, int32_t* __restrict__ ids, float* __restrict__ weights) {
    const int lane = threadIdx.x & 63, t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (t >= n_tokens) return;
    int my_id;
    float my_w;
    route_grouped_sigmoid_wave<PER>(logits + (int64_t)t * n_expert, bias, n_expert, n_group, topk_group, k,
                                    routed_scale, my_id, my_w);
    if (lane < k) {
        ids[(int64_t)t * k + lane] = my_id;
        weights[(int64_t)t * k + lane] = my_w;
    }
}

hipError_t launch_router_topk(const float* logits, int n_tokens, int n_expert, int k, int32_t* ids, float* weights,
                              hipStream_t s) {
    const dim3 g((unsigned)n_tokens), b(64);
    if (n_expert <= 64) hipLaunchKernelGGL(router_topk_kernel<1>, g, b, 0, s, logits, n_expert, k, ids, weights);
    else if (n_expert <= 128) hipLaunchKernelGGL(router_topk_kernel<2>, g, b, 0, s, logits, n_expert, k, ids, weights);
    else if (n_expert <= 256) hipLaunchKernelGGL(router_topk_kernel<4>, g, b, 0, s, logits, n_expert, k, ids, weights);
    else if (n_expert <= 512) hipLaunchKernelGGL(router_topk_kernel<8>, g, b, 0, s, logits, n_expert, k, ids, weights);
    else hipLaunchKernelGGL(router_topk_kernel<16>, g, b, 0, s, logits, n_expert, k, ids, weights);
    return hipGetLastError();
}

hipError_t launch_router_grouped_sigmoid(const float* logits, const float* bias, int n_tokens, int n_expert,
                                         int n_group, int topk_group, int k, float routed_scale, int32_t* ids,
                                         float* weights, hipStream_t s) {
    // the register form where the groups fall on whole lanes (lanes a group a power of two), else the LDS form
    const int PER = n_expert <= 64 ? 1 : n_expert <= 128 ? 2 : n_expert <= 256 ? 4 : n_expert <= 512 ? 8 : 16;
    const int per = n_group > 0 ? n_expert / n_group : 0;
    const int lpg = per % PER == 0 ? per / PER : 0;
    if (n_expert <= 1024 && n_group > 0 && per * n_group == n_expert && lpg > 0 && (lpg & (lpg - 1)) == 0) {
        const dim3 g((unsigned)((n_tokens + 3) / 4)), b(256);
        const auto args = [&](auto kern) {
            hipLaunchKernelGGL(kern, g, b, 0, s, logits, bias, n_tokens, n_expert, n_group, topk_group, k, routed_scale,
                               ids, weights);
        };
        if (PER == 1) args(router_grouped_sigmoid_wave_kernel<1>);
        else if (PER == 2) args(router_grouped_sigmoid_wave_kernel<2>);
        else if (PER == 4) args(router_grouped_sigmoid_wave_kernel<4>);
        else if (PER == 8) args(router_grouped_sigmoid_wave_kernel<8>);
        else args(router_grouped_sigmoid_wave_kernel<16>);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(router_grouped_sigmoid_kernel, dim3((unsigned)n_tokens), dim3(64), 0, s, logits, bias, n_expert,
                       n_group, topk_group, k, routed_scale, ids, weights);
    return hipGetLastError();
}

}  // namespace xs
