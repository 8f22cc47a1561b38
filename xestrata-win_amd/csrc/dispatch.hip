// xestrata-win_amd/csrc/dispatch.hip - token-to-expert dispatch on the device.
//
//  * resident_plan: the decode / verify-window plan in the reference's host-pool layout (reference
//    src/kernels/xe/verify_kernels.cpp:819-890; layout include/strata/core/expert_source.hpp:219-243): groups are the
//    distinct experts in order of first occurrence, a group's entries ascending.  A leader (an expert's first entry)
//    is found with an LDS atomicMin, groups are numbered by one work-group exclusive scan of (entries << 16 | 1) over
//    the leaders, and an entry's place in its group is the count of earlier entries with its expert.
//  * prefill_route: the prompt path's permutation (reference src/prefill/plain_prompt.cpp:576-637, there on the
//    host after a blocking copy): histogram, experts ascending, exclusive prefix, and a STABLE fill.  Here one
//    work-group of 16 waves: each wave counts its own contiguous segment of entries into its own LDS histogram, the
//    per-(wave, expert) bases come from one scan, and each wave then walks its segment in order, ranking equal
//    experts inside a 64-entry step by a ballot match on the expert bits.  The rows come out in the host loop's order
//    exactly.
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_route.h"

namespace xs {

constexpr int kPlanThreads = 1024;

__global__ __launch_bounds__(kPlanThreads) void resident_plan_kernel(const int32_t* __restrict__ ids, int n, int k,
                                                                     const int32_t* __restrict__ res, int n_expert,
                                                                     const uint8_t* cache_base,
                                                                     const unsigned long long* __restrict__ slot_off,
                                                                     long long blob, int32_t* __restrict__ pl,
                                                                     long long capx, uint32_t* skip, uint32_t ring) {
    extern __shared__ int s_first[];   // n_expert
    __shared__ int s_ids[kPlanThreads];
    __shared__ int s_excl[kPlanThreads];
    __shared__ int s_wave[64];
    const int t = threadIdx.x;
    bool bad = false;
    if (t < n) {
        const int ex = ids[t];
        s_ids[t] = ex;
        bad = ex < 0 || ex >= n_expert || (res && res[ex] < 0);
    }
    if (__syncthreads_or(bad)) {   // a routed expert that is not resident: the plan is left alone
        if (t == 0) *skip = 0u;
        return;
    }
    build_plan(s_ids, s_first, s_excl, s_wave, n, k, res, n_expert, cache_base, slot_off, blob, pl, capx, skip, ring);
}

constexpr int kRouteWaves = 16;

__global__ __launch_bounds__(kRouteWaves * 64) void prefill_route_kernel(
    const int32_t* __restrict__ ids, int n, int k, int n_expert, int nbits, int32_t* __restrict__ src,
    int32_t* __restrict__ slot, int32_t* __restrict__ entry, int32_t* __restrict__ bounds,
    int32_t* __restrict__ experts, int32_t* __restrict__ n_groups, const uint8_t* cache_base, long long blob,
    unsigned long long* __restrict__ grp_ptr) {
    extern __shared__ int s_hist[];   // [kRouteWaves][n_expert]: counts, then bases
    __shared__ int s_wave[64];
    __shared__ int s_bad;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int seg = ((n + kRouteWaves - 1) / kRouteWaves + 63) & ~63;
    const int i0 = wave * seg, i1 = min(n, i0 + seg);
    for (int i = tid; i < kRouteWaves * n_expert; i += blockDim.x) s_hist[i] = 0;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    int* hist = s_hist + wave * n_expert;
    for (int i = i0 + lane; i < i1; i += 64) {
        const int e = ids[i];
        if (e < 0 || e >= n_expert) s_bad = 1;
        else atomicAdd(&hist[e], 1);
    }
    __syncthreads();
    if (s_bad) {
        if (tid == 0) *n_groups = -1;
        return;
    }
    // per expert: its total, the exclusive prefix over experts (start), the compacted group list, and each wave's base
    int carry = 0, gcarry = 0;
    for (int e0 = 0; e0 < n_expert; e0 += blockDim.x) {
        const int e = e0 + tid;
        int tot = 0;
        if (e < n_expert)
            for (int w = 0; w < kRouteWaves; ++w) tot += s_hist[w * n_expert + e];
        int sum_all, g_all;
        const int st = block_exclusive_scan(tot, s_wave, &sum_all) + carry;
        const int gi = block_exclusive_scan(tot > 0 ? 1 : 0, s_wave, &g_all) + gcarry;
        if (e < n_expert) {
            if (tot > 0) {
                experts[gi] = e;
                bounds[gi] = st;
                if (grp_ptr) grp_ptr[gi] = (unsigned long long)(uintptr_t)(cache_base + (size_t)e * (size_t)blob);
            }
            int b = st;
            for (int w = 0; w < kRouteWaves; ++w) {
                const int c = s_hist[w * n_expert + e];
                s_hist[w * n_expert + e] = b;
                b += c;
            }
        }
        carry += sum_all;
        gcarry += g_all;
    }
    if (tid == 0) {
        bounds[gcarry] = n;
        *n_groups = gcarry;
    }
    __syncthreads();
    // the stable fill: wave by wave over its own segment, 64 entries a step, in entry order
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = i0; base < i1; base += 64) {
        const int i = base + lane;
        const bool in = i < i1;
        const int e = in ? ids[i] : 0;
        uint64_t peers = __ballot(in);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = (e >> b) & 1;
            const uint64_t m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        if (in) {
            const int rank = __popcll(peers & below);
            const int row = hist[e] + rank;
            src[row] = i / k;
            slot[i] = row;
            entry[row] = i;
        }
        __builtin_amdgcn_wave_barrier();
        if (in && (peers & below) == 0) hist[e] += __popcll(peers);
        __builtin_amdgcn_wave_barrier();
    }
}

hipError_t launch_resident_plan(const int32_t* ids, int n, int k, const int32_t* res, int n_expert,
                                const uint8_t* cache_base, const unsigned long long* slot_off, long long blob,
                                int32_t* plan, long long capx, uint32_t* skip, uint32_t ring, hipStream_t s) {
    const size_t lds = (size_t)n_expert * sizeof(int);
    hipLaunchKernelGGL(resident_plan_kernel, dim3(1), dim3(kPlanThreads), lds, s, ids, n, k, res, n_expert, cache_base,
                       slot_off, blob, plan, capx, skip, ring);
    return hipGetLastError();
}

hipError_t launch_prefill_route(const int32_t* ids, int64_t n, int k, int n_expert, int32_t* src, int32_t* slot,
                                int32_t* entry, int32_t* bounds, int32_t* experts, int32_t* n_groups,
                                const uint8_t* cache_base, long long blob, unsigned long long* grp_ptr, hipStream_t s) {
    int nbits = 1;
    while ((1 << nbits) < n_expert) ++nbits;
    const size_t lds = (size_t)kRouteWaves * n_expert * sizeof(int);
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void*)prefill_route_kernel,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(prefill_route_kernel, dim3(1), dim3(kRouteWaves * 64), lds, s, ids, (int)n, k, n_expert, nbits,
                       src, slot, entry, bounds, experts, n_groups, cache_base, blob, grp_ptr);
    return hipGetLastError();
}

}  // namespace xs
