// xestrata-win_amd/csrc/dispatch.hip - token-to-expert dispatch on the device.
//
//  * resident_plan: the decode / verify-window plan in the engine's plan words (xs_plan.h; reference
//    src/kernels/xe/verify_kernels.cpp:819-890): groups are the distinct experts in order of first occurrence, a
//    group's entries ascending.  One wave walks the entries in order and numbers the groups as their experts first
//    appear (plan_groups_wave, xs_route.h); then every thread places its entry.
//  * prefill_route: the prompt path's permutation (reference src/prefill/plain_prompt.cpp:576-637, there on the
//    host after a blocking copy): histogram, experts ascending, exclusive prefix, and a STABLE fill.  Here one
//    work-group of 16 waves: each wave counts its own contiguous segment of entries into its own LDS histogram, the
//    per-(wave, expert) bases come from one scan, and each wave then walks its segment in order, ranking equal
//    experts inside a 64-entry step by a ballot match on the expert bits.  The rows come out in the host loop's order
//    exactly.
#include "xs_device.h"
#include "xs_f16.h"
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
    extern __shared__ int16_t s_gid[];   // n_expert
    __shared__ int s_ids[kPlanThreads], s_ent[kPlanThreads], s_gsz[kPlanThreads + 1], s_gexp[kPlanThreads];
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
    write_decode_plan(s_ids, PlanLds{s_gid, s_ent, s_gsz, s_gexp}, n, k, n_expert, res, cache_base, slot_off, blob, pl,
                      capx, skip, ring);
}

constexpr int kRouteWaves = 16;
constexpr int kBatch = 16;   // 64-entry steps of ids loaded together

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
    // the ids are read kBatch steps of 64 at a time, all loads in flight together (a step's latency once a batch)
    for (int base = i0; base < i1; base += 64 * kBatch) {
        int ev[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int i = base + 64 * u + lane;
            ev[u] = i < i1 ? ids[i] : 0;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (base + 64 * u + lane >= i1) continue;
            const int e = ev[u];
            if (e < 0 || e >= n_expert) s_bad = 1;
            else atomicAdd(&hist[e], 1);
        }
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
    for (int base0 = i0; base0 < i1; base0 += 64 * kBatch) {
        int ev[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int i = base0 + 64 * u + lane;
            ev[u] = i < i1 ? ids[i] : 0;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int i = base0 + 64 * u + lane;
            const bool in = i < i1;
            const int e = ev[u];
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
}

// ---------------------------------------------------------------- the permutation split over work-groups
// The single work-group above writes every row itself, and its scattered stores (one cache line a lane) bound it.
// The whole-layer path has a workspace, so it spreads the same permutation over blocks of kSeg entries: pass 1 counts
// each block's experts (and bad ids), pass 2 gives every block its bases - the experts' exclusive prefix plus the
// counts of the blocks before it - and ranks its entries as above, one 64-entry step a wave.  Rows, groups and
// bounds come out identical to the single work-group's.
constexpr int kSeg = 1024;

__global__ __launch_bounds__(256) void route_hist_kernel(const int32_t* __restrict__ ids, int n, int n_expert,
                                                         int32_t* __restrict__ ghist) {
    extern __shared__ int s_h[];   // [n_expert + 1]: counts, then bad ids
    const int tid = threadIdx.x;
    for (int e = tid; e <= n_expert; e += 256) s_h[e] = 0;
    __syncthreads();
    const int i0 = blockIdx.x * kSeg;
    int ev[kSeg / 256];
#pragma unroll
    for (int u = 0; u < kSeg / 256; ++u) {
        const int i = i0 + 256 * u + tid;
        ev[u] = i < n ? ids[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kSeg / 256; ++u) {
        if (i0 + 256 * u + tid >= n) continue;
        const int e = ev[u];
        atomicAdd(&s_h[(e < 0 || e >= n_expert) ? n_expert : e], 1);
    }
    __syncthreads();
    for (int e = tid; e <= n_expert; e += 256) ghist[(int64_t)blockIdx.x * (n_expert + 1) + e] = s_h[e];
}

__global__ __launch_bounds__(1024) void route_fill_kernel(
    const int32_t* __restrict__ ids, int n, int k, int n_expert, int nbits, const int32_t* __restrict__ ghist, int nblk,
    int32_t* __restrict__ src, int32_t* __restrict__ slot, int32_t* __restrict__ entry, int32_t* __restrict__ bounds,
    int32_t* __restrict__ experts, int32_t* __restrict__ n_groups, const uint8_t* cache_base, long long blob,
    unsigned long long* __restrict__ grp_ptr, int32_t* __restrict__ mtile, int cap_groups, int split, ToF16 conv) {
    extern __shared__ int s_w[];   // [16][n_expert]: each wave's counts, then its bases
    __shared__ int s_wave[128];    // (block_exclusive_scan_n<7>: 119)
    __shared__ int s_bad;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = n_expert, blk = blockIdx.x;
    if (blk >= nblk) {   // the f16 copy of x, beside the permutation (it needs none of it)
        const int64_t stride = (int64_t)(gridDim.x - nblk) * 1024;
        for (int64_t c = (int64_t)(blk - nblk) * 1024 + tid; c < conv.n_chunks; c += stride)
            to_f16_chunk(conv.x, conv.y, c, conv.err);
        return;
    }
    const int i = blk * kSeg + tid;
    const bool in = i < n;
    const int ev = in ? ids[i] : 0;
    if (tid == 0) s_bad = 0;
    for (int x = tid; x < 16 * E; x += 1024) s_w[x] = 0;
    __syncthreads();
    if (tid < nblk && ghist[(int64_t)tid * (E + 1) + E] != 0) s_bad = 1;
    __syncthreads();
    if (s_bad) {   // a bad id anywhere: n_groups = -1 and nothing else written, as the single work-group does
        if (blk == 0 && tid == 0) *n_groups = -1;
        return;
    }
    const int e = in ? ev : 0;
    uint64_t peers = __ballot(in);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (e >> b) & 1;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(peers & below);
    if (in && rank == 0) s_w[wave * E + e] = __popcll(peers);
    __syncthreads();
    int carry = 0, gcarry = 0, f128 = 0, p128 = 0, f64 = 0, p64 = 0, ftall = 0;
    const int64_t cap128 = tile_cap(n, 128, cap_groups), cap64 = tile_cap(n, 64, cap_groups);
    for (int e0 = 0; e0 < E; e0 += 1024) {
        const int ee = e0 + tid;
        int tot = 0, pre = 0;
        if (ee < E)
            for (int b0 = 0; b0 < nblk; b0 += 8) {   // 8 loads in flight at a time
                int c[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) c[u] = b0 + u < nblk ? ghist[(int64_t)(b0 + u) * (E + 1) + ee] : 0;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    tot += c[u];
                    if (b0 + u < blk) pre += c[u];
                }
            }
        int sum_all, st;
        if (blk != 0) {
            st = block_exclusive_scan(tot, s_wave, &sum_all) + carry;
        } else {   // the groups (experts ascending), and the m-tile table of 128- and 64-row tiles
            // (split: the group's whole 256-row tiles in the tall list, the maps over the rows past them); the seven
            // scans in one pass of barriers
            const int ntall = split ? tot / 256 : 0, rest = tot - 256 * ntall;
            const int sv[7] = {tot, tot > 0 ? 1 : 0, rest / 128, rest % 128 ? 1 : 0, rest / 64, rest % 64 ? 1 : 0, ntall};
            int ex[7], tt[7];
            block_exclusive_scan_n<7>(sv, s_wave, ex, tt);
            st = ex[0] + carry;
            sum_all = tt[0];
            const int g_all = tt[1], a0 = tt[2], a1 = tt[3], a2 = tt[4], a3 = tt[5], a4 = tt[6];
            const int gi = ex[1] + gcarry;
            const int b128 = ex[2] + f128, q128 = ex[3] + p128, b64 = ex[4] + f64, q64 = ex[5] + p64;
            const int bt = ex[6] + ftall;
            if (ee < E && tot > 0) {
                experts[gi] = ee;
                bounds[gi] = st;
                if (grp_ptr) grp_ptr[gi] = (unsigned long long)(uintptr_t)(cache_base + (size_t)ee * (size_t)blob);
                if (mtile && gi < cap_groups) {
                    const int rs = st + 256 * ntall;
                    write_group_tiles(tile_list(mtile, n, cap_groups, 128), gi, rs, rest, 128, b128, q128, cap128);
                    write_group_tiles(tile_list(mtile, n, cap_groups, 64), gi, rs, rest, 64, b64, q64, cap64);
                    int32_t* lt = tall_list(mtile, n, cap_groups);
                    for (int t = 0; t < ntall; ++t) {
                        lt[1 + 2 * (bt + t)] = gi;
                        lt[2 + 2 * (bt + t)] = st + 256 * t;
                    }
                }
            }
            gcarry += g_all;
            f128 += a0;
            p128 += a1;
            f64 += a2;
            p64 += a3;
            if (split) ftall += a4;
        }
        if (ee < E) {
            int b = st + pre;
            for (int w = 0; w < 16; ++w) {
                const int c = s_w[w * E + ee];
                s_w[w * E + ee] = b;
                b += c;
            }
        }
        carry += sum_all;
    }
    if (blk == 0 && tid == 0) {
        bounds[gcarry] = n;
        *n_groups = gcarry;
        if (mtile) {
            mtile[0] = f128;
            mtile[1] = p128;
            mtile[2] = f64;
            mtile[3] = p64;
            if (split) *tall_list(mtile, n, cap_groups) = ftall;
        }
    }
    __syncthreads();
    if (in) {
        const int row = s_w[wave * E + e] + rank;
        src[row] = i / k;
        slot[i] = row;
        entry[row] = i;
    }
}

hipError_t launch_prefill_route_split(const int32_t* ids, int64_t n, int k, int n_expert, int32_t* src, int32_t* slot,
                                      int32_t* entry, int32_t* bounds, int32_t* experts, int32_t* n_groups,
                                      const uint8_t* cache_base, long long blob, unsigned long long* grp_ptr,
                                      int32_t* ghist, int32_t* mtile, int cap_groups, hipStream_t s, bool split,
                                      const ToF16* conv) {
    int nbits = 1;
    while ((1 << nbits) < n_expert) ++nbits;
    const int nblk = (int)((n + kSeg - 1) / kSeg);
    hipLaunchKernelGGL(route_hist_kernel, dim3(nblk), dim3(256), (size_t)(n_expert + 1) * sizeof(int), s, ids, (int)n,
                       n_expert, ghist);
    // with conv, one thread a chunk past the permutation's work-groups (up to 2048 work-groups, then a stride)
    const ToF16 cv = conv ? *conv : ToF16{nullptr, nullptr, 0, nullptr};
    const int64_t ncb = (cv.n_chunks + 1023) / 1024;
    const int nconv = (int)(ncb < 2048 ? ncb : 2048);
    hipLaunchKernelGGL(route_fill_kernel, dim3(nblk + nconv), dim3(1024), (size_t)16 * n_expert * sizeof(int), s, ids,
                       (int)n, k, n_expert, nbits, ghist, nblk, src, slot, entry, bounds, experts, n_groups, cache_base,
                       blob, grp_ptr, mtile, cap_groups, split ? 1 : 0, cv);
    return hipGetLastError();
}

size_t prefill_route_split_scratch(int64_t n, int n_expert) {
    return (size_t)((n + kSeg - 1) / kSeg) * (size_t)(n_expert + 1) * sizeof(int32_t);
}

hipError_t launch_resident_plan(const int32_t* ids, int n, int k, const int32_t* res, int n_expert,
                                const uint8_t* cache_base, const unsigned long long* slot_off, long long blob,
                                int32_t* plan, long long capx, uint32_t* skip, uint32_t ring, hipStream_t s) {
    const size_t lds = ((size_t)n_expert * sizeof(int16_t) + 3) & ~(size_t)3;
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

// ---------------------------------------------------------------- one group (a shared expert)

__global__ void single_group_plan_kernel(unsigned long long* grp_ptr, int32_t* start, int32_t* n_groups, int32_t* idx,
                                         int n, const uint8_t* blob) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) idx[i] = i;
    if (i == 0) {
        grp_ptr[0] = (unsigned long long)blob;
        start[0] = 0;
        start[1] = n;
        *n_groups = 1;
    }
}

hipError_t launch_single_group_plan(unsigned long long* grp_ptr, int32_t* start, int32_t* n_groups, int32_t* idx,
                                    int n, const uint8_t* blob, hipStream_t s) {
    hipLaunchKernelGGL(single_group_plan_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, grp_ptr, start,
                       n_groups, idx, n, blob);
    return hipGetLastError();
}

}  // namespace xs
