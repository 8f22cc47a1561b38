// xestrata-win_amd/csrc/decode_layer.hip - the decode layer's routing in one launch: the tokens' q8_1 activations,
// the softmax top-k of every token and the plan over their routed entries.  Work-group 0 (16 waves) routes and plans;
// work-groups 1.. quantize the activations beside it, 1024-lane rounds each (in work-group 0 after its routing they
// took more than half the launch: 10.7 of 20 us at 8 tokens of hidden 4096).  The
// reference runs these as quantize_q8_1_rows, router_top10 and resident_plan (src/core/verify.cpp:1160-1360, the
// resident verify window) or routes on the device and plans on the host (src/core/moe_window.cpp:183-250); one launch
// here instead of three, on the same arithmetic (xs_route.h).
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_route.h"

namespace xs {

constexpr int kRouteThreads = 1024;

template <int PER>
__global__ __launch_bounds__(kRouteThreads) void decode_route_kernel(const float* __restrict__ logits,
                                                                     const float* __restrict__ x, int n_tok,
                                                                     int n_expert, int k, int64_t n_embd,
                                                                     int32_t* __restrict__ ids,
                                                                     float* __restrict__ weights,
                                                                     int32_t* __restrict__ plan, long long capx,
                                                                     uint32_t* skip, const uint8_t* arena, long long blob,
                                                                     uint8_t* __restrict__ xq) {
    extern __shared__ int16_t s_gid[];   // n_expert
    __shared__ int s_ids[kRouteThreads], s_ent[kRouteThreads], s_gsz[kRouteThreads + 1], s_gexp[kRouteThreads];
    const int tid = threadIdx.x, wave = tid >> 6;
    if (blockIdx.x > 0) {
        // the activations: 8 values a lane, one scale a 256 (whole 1024-lane rounds, so every wave's groups are whole)
        const int64_t n8 = (int64_t)n_tok * n_embd / 8;
        for (int64_t j0 = (int64_t)(blockIdx.x - 1) * kRouteThreads; j0 < n8; j0 += (int64_t)(gridDim.x - 1) * kRouteThreads)
            q8_1_256_lane(x, j0 + tid, j0 + tid < n8, xq);
        return;
    }
    // the router: a wave a token
    for (int t = wave; t < n_tok; t += kRouteThreads / 64)
        route_topk_wave<PER>(logits + (int64_t)t * n_expert, n_expert, k, ids + (int64_t)t * k,
                             weights + (int64_t)t * k);
    __syncthreads();
    const int n = n_tok * k;
    bool bad = false;
    if (tid < n) {
        const int ex = ids[tid];
        s_ids[tid] = ex;
        bad = ex < 0 || ex >= n_expert;
    }
    if (__syncthreads_or(bad)) {   // a rank left unwritten (NaN logits): no groups this call
        if (tid == 0) {
            plan[0] = 0;
            plan[4] = 0;
            *skip = 0u;
        }
        return;
    }
    write_decode_plan(s_ids, PlanLds{s_gid, s_ent, s_gsz, s_gexp}, n, k, n_expert, nullptr, arena, nullptr, blob, plan,
                      capx, skip, 1u);
}

hipError_t launch_decode_route(const float* logits, const float* x, int n_tok, int n_expert, int k, int64_t n_embd,
                               int32_t* ids, float* weights, int32_t* plan, long long capx, uint32_t* skip,
                               const uint8_t* arena, long long blob, void* xq, hipStream_t s) {
    const size_t lds = ((size_t)n_expert * sizeof(int16_t) + 3) & ~(size_t)3;
    const int64_t rounds = ((int64_t)n_tok * n_embd / 8 + kRouteThreads - 1) / kRouteThreads;
    const dim3 g((unsigned)(1 + (rounds < 64 ? rounds : 64))), b(kRouteThreads);
#define XS_ROUTE(PER)                                                                                                  \
    hipLaunchKernelGGL(decode_route_kernel<PER>, g, b, lds, s, logits, x, n_tok, n_expert, k, n_embd, ids, weights,    \
                       plan, capx, skip, arena, blob, (uint8_t*)xq)
    if (n_expert <= 64) XS_ROUTE(1);
    else if (n_expert <= 128) XS_ROUTE(2);
    else if (n_expert <= 256) XS_ROUTE(4);
    else if (n_expert <= 512) XS_ROUTE(8);
    else XS_ROUTE(16);
#undef XS_ROUTE
    return hipGetLastError();
}

}  // namespace xs
