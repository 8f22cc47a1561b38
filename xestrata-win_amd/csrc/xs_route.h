// xestrata-win_amd/csrc/xs_route.h - device building blocks of routing, shared by the standalone kernels (router.hip,
// dispatch.hip, quant_act.hip) and the fused decode route kernel (decode_layer.hip).
#pragma once

#include "xs_device.h"
#include "xs_plan.h"

namespace xs {

// the argmax order: the larger value wins, a tie keeps the lower index; NaN never wins (reference
// src/kernels/xe/router.cpp:32-36)
__device__ __forceinline__ void better(float& bv, int& bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

// Softmax top-k of one token on one wave, bit for bit the reference's router_top10 (src/kernels/xe/router.cpp:59-145
// and its fast form :146-276): mx = max l; ex = exp((double) l - (double) mx); inv = (float) (1 / sum ex) with the
// sum serial and ascending in double; p = (float) (ex * inv); k passes of argmax; renormalised in double by max(sum
// of the k, 2^-14).  The serial sum runs only when a tree sum cannot decide inv: the serial and tree sums both lie
// within 2^-43 of the exact sum (every term is positive, the largest exactly 1), so when the bracket tree * (1 -+
// 2^-40) maps to one float inv, that float is the serial sum's.  PER experts a lane (n_expert <= 64 PER).  A row whose
// ranks run out (NaN) leaves them as they were and renormalises the buffer (router.cpp:113-133).  Reductions move
// lanes with DPP and v_readlane (xs_device.h): the argmax is order-free (a strict total order), the tree sum only
// brackets inv, and the serial sums read lanes in order.  Every lane of the wave calls it.
template <int PER>
__device__ __forceinline__ void load_logits_wave(const float* __restrict__ l, int n_expert, float (&lv)[PER]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < PER; ++j) lv[j] = lane + 64 * j < n_expert ? l[lane + 64 * j] : -INFINITY;
}
// the same on logits already loaded (load_logits_wave)
template <int PER>
__device__ void route_topk_wave_lv(const float (&lv)[PER], int n_expert, int k, int32_t* id_row, float* w_row) {
    const int lane = threadIdx.x & 63;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j)
        if (lane + 64 * j < n_expert) mx = fmaxf(mx, lv[j]);
    mx = wave_max(mx);
    double ex[PER];
    double part = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int x = lane + 64 * j;
        ex[j] = x < n_expert ? exp((double)lv[j] - (double)mx) : 0.0;
        part += ex[j];
    }
    part = wave_sum_d(part);
    const double lo = part * (1.0 - 0x1p-40), hi = part * (1.0 + 0x1p-40);
    const float f_lo = (float)(1.0 / hi), f_hi = (float)(1.0 / lo);
    float inv;
    if (part >= 1.0 && hi < 1e300 && f_lo == f_hi) {
        inv = f_lo;
    } else {   // uniform over the wave: the serial ascending sum
        double sum = 0.0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            if (64 * j >= n_expert) break;
            for (int s = 0; s < 64 && 64 * j + s < n_expert; ++s) sum += readlane_d(ex[j], s);
        }
        inv = (float)(1.0 / sum);
    }
    // k argmax passes (the reference's order: the larger p wins, a tie goes to the lower index; NaN never wins).  A
    // candidate's p bits + 1 order as p does (p >= 0), 0 marks none; each pass is one 32-bit wave max and, for the
    // tie, the lowest lane of the lowest slot holding it (slot j holds experts 64 j + lane).
    uint32_t pv[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int x = lane + 64 * j;
        const float p = x < n_expert ? (float)(ex[j] * (double)inv) : __int_as_float(0x7FC00000);
        pv[j] = p == p ? __float_as_uint(p) + 1u : 0u;
    }
    constexpr int kEq = 32, kNe = 33, kUle = 37;   // llvm.amdgcn.icmp predicates: the compare's lane mask, straight
    float my_w = 0.0f;
    int my_id = 0, nsel = 0;
    // Fast path, the same keys in the same order without k dependent passes: each candidate's bucket is its distance
    // below the largest key in half binades (2^22 in the bits, 15 for all further down); the k-th smallest bucket v
    // (a 4-step bisection on ballot counts) bounds the k best, the M (<= 32) candidates in buckets <= v move to
    // lanes 0..M-1 (ds_permute), each one's rank is the count of candidate keys above its own, and the k best move to
    // the lanes of their ranks.  Otherwise (NaN p, k > 32, candidates too dense) the passes below.
    int nvalid = 0;
    uint32_t pm = 0u;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        nvalid += __popcll(__builtin_amdgcn_uicmp(pv[j], 0u, kNe));
        pm = pm > pv[j] ? pm : pv[j];
    }
    if (nvalid > k && k <= 32) {
        pm = wave_max_u32(pm);
        uint32_t d[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) d[j] = pv[j] == 0u ? 16u : min((pm - pv[j]) >> 22, 15u);
        uint32_t v = 0u;   // the smallest bucket with >= k candidates at or below it (all valid ones are at <= 15)
#pragma unroll
        for (int b = 3; b >= 0; --b) {
            const uint32_t c = v + (1u << b) - 1u;
            int n = 0;
#pragma unroll
            for (int j = 0; j < PER; ++j) n += __popcll(__builtin_amdgcn_uicmp(d[j], c, kUle));
            v = n < k ? v + (1u << b) : v;
        }
        int M = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) M += __popcll(__builtin_amdgcn_uicmp(d[j], v, kUle));
        if (M <= 32) {
            // candidate q of the ascending index order to lane q; lanes that are no candidate write lane 63
            uint32_t cp = 0u, cx = 0u;
            int base = 0;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const unsigned long long cm = __builtin_amdgcn_uicmp(d[j], v, kUle);
                const int nj = __popcll(cm);
                if (nj == 0) continue;   // uniform
                const uint32_t below =
                    __builtin_amdgcn_mbcnt_hi((uint32_t)(cm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)cm, 0u));
                const int to = d[j] <= v ? base + (int)below : 63;
                const uint32_t gp = (uint32_t)__builtin_amdgcn_ds_permute(4 * to, (int)pv[j]);
                const uint32_t gx = (uint32_t)__builtin_amdgcn_ds_permute(4 * to, lane + 64 * j);
                const bool mine = lane >= base && lane < base + nj;
                cp = mine ? gp : cp;
                cx = mine ? gx : cx;
                base += nj;
            }
            // rank = candidates whose key (p bits over the inverted index) is above this lane's
            const unsigned long long kq = ((unsigned long long)cp << 32) | (unsigned int)~cx;
            int rank = 0;
            for (int r = 0; r < M; ++r) {
                const uint32_t hr = __builtin_amdgcn_readlane((int)cp, r), xr = __builtin_amdgcn_readlane((int)cx, r);
                rank += (((unsigned long long)hr << 32) | (unsigned int)~xr) > kq ? 1 : 0;
            }
            const int to = lane < M && rank < k ? rank : 63;
            const uint32_t wp = (uint32_t)__builtin_amdgcn_ds_permute(4 * to, (int)cp);
            const uint32_t wx = (uint32_t)__builtin_amdgcn_ds_permute(4 * to, (int)cx);
            if (lane < k) {
                my_w = __uint_as_float(wp - 1u);
                my_id = (int)wx;
            }
            nsel = k;
        }
    }
    for (int i = nsel > 0 ? k : 0; i < k; ++i) {
        uint32_t m = pv[0];
#pragma unroll
        for (int j = 1; j < PER; ++j) m = m > pv[j] ? m : pv[j];
        const uint32_t best = wave_max_u32(m);
        if (best == 0u) break;   // no candidate left (NaN p): ranks i.. keep the buffer's contents
        // the lowest index holding it: the first slot with a lane at best, its lowest lane
        unsigned long long e = 0ull;
        int wj = 0;
#pragma unroll
        for (int j = PER - 1; j >= 0; --j) {
            const unsigned long long ej = __builtin_amdgcn_uicmp(pv[j], best, kEq);
            wj = ej ? j : wj;
            e = ej ? ej : e;
        }
        const int wl = __builtin_ctzll(e);
#pragma unroll
        for (int j = 0; j < PER; ++j) pv[j] = j == wj && lane == wl ? 0u : pv[j];
        if (lane == i) {
            my_w = __uint_as_float(best - 1u);
            my_id = wl + 64 * wj;
        }
        nsel = i + 1;
    }
    if (nsel == k) {
        // the sum of the k in rank order, in double.  With k <= 16 values within 2^25 of each other (all <= 1) every
        // partial sum is exact (it is a multiple of the smallest value's ulp below 2^53 of them), so a tree over the
        // lanes gives the serial sum bit for bit.
        double s = 0.0;
        if (k <= 16 && readlane_f(my_w, k - 1) >= readlane_f(my_w, 0) * 0x1p-25f) {
            double t = lane < k ? (double)my_w : 0.0;
            t += dpp_d<kDppXor1>(t);
            t += dpp_d<kDppXor2>(t);
            t += dpp_d<kDppRor4>(t);
            t += dpp_d<kDppRor8>(t);
            s = readlane_d(t, 0);
        } else {
            for (int i = 0; i < k; ++i) s += (double)readlane_f(my_w, i);
        }
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

template <int PER>
__device__ void route_topk_wave(const float* __restrict__ l, int n_expert, int k, int32_t* id_row, float* w_row) {
    float lv[PER];
    load_logits_wave<PER>(l, n_expert, lv);
    route_topk_wave_lv<PER>(lv, n_expert, k, id_row, w_row);
}

// exclusive scan of v over the work-group (blockDim.x threads, a multiple of 64, at most 1024); *total gets the sum
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wave, int* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(inc, o, 64);
        if (lane >= o) inc += y;
    }
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    if (wave == 0) {
        const int w = lane < nw ? s_wave[lane] : 0;
        int wi = w;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(wi, o, 64);
            if (lane >= o) wi += y;
        }
        if (lane < nw) s_wave[lane] = wi - w;   // exclusive over waves
        if (lane == nw - 1) s_wave[63] = wi;    // total (nw <= 16 leaves slot 63 free)
    }
    __syncthreads();
    const int r = s_wave[wave] + inc - v;
    *total = s_wave[63];
    __syncthreads();
    return r;
}

// the same for N values at once (one pass of barriers for all of them): ex[i] the exclusive scan of v[i], total[i] its
// sum; s_wave holds at least 17 N ints
template <int N>
__device__ __forceinline__ void block_exclusive_scan_n(const int (&v)[N], int* s_wave, int (&ex)[N], int (&total)[N]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int inc[N];
#pragma unroll
    for (int i = 0; i < N; ++i) inc[i] = v[i];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int y = __shfl_up(inc[i], o, 64);
            if (lane >= o) inc[i] += y;
        }
    }
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < N; ++i) s_wave[i * 16 + wave] = inc[i];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int w = lane < nw ? s_wave[i * 16 + lane] : 0;
            int wi = w;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const int y = __shfl_up(wi, o, 64);
                if (lane >= o) wi += y;
            }
            if (lane == nw - 1) s_wave[16 * N + i] = wi;   // the total
            if (lane < nw) s_wave[i * 16 + lane] = wi - w;   // exclusive over waves (after every lane read its slot)
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) {
        ex[i] = s_wave[i * 16 + wave] + inc[i] - v[i];
        total[i] = s_wave[16 * N + i];
    }
    __syncthreads();
}

// ---------------------------------------------------------------- the decode plan
// Groups are the distinct experts in order of first occurrence and a group's entries ascend: the order the engine's
// plan consumers expect (reference src/kernels/xe/verify_kernels.cpp:819-890, the host pool's plan
// src/core/expert_source.cpp:2193-2344).  Built by ONE wave that walks the entries in order, 64 at a time, with each
// expert's group number kept in LDS (-1 until its first entry):
//  * the lanes holding one expert inside a step find each other by a ballot match over the expert's bits; the lowest
//    of them (the step's head for that expert) acts for all;
//  * a head whose expert has no group yet opens one, numbered after the groups already open and the heads below it
//    that open one too (a popcount of the opening ballot): groups come out in first-occurrence order;
//  * an entry's place in its group is the group's size before the step plus its rank among its expert's lanes; the
//    head then adds the step's count to the size.
// The wave then turns the sizes into starts (a 64-group inclusive sum, carried from chunk to chunk).  No atomics and
// no work-group scan: 1024 entries are 16 steps of a few ballots.  The caller places the entries afterwards:
// slot = start[group] + place.
struct PlanLds {
    int16_t* gid;    // [n_expert]: the expert's group, -1 before its first entry
    int32_t* ent;    // [n]: the entry's group | its place in the group << 16
    int32_t* gsz;    // [n + 1]: a group's size, then its first slot; [groups] = n
    int32_t* gexp;   // [n]: the group's expert
};

// Every lane of one wave calls it, with s_ids[0..n) valid ids below n_expert (n <= 32768).  Returns the group count.
__device__ int plan_groups_wave(const int* s_ids, int n, int n_expert, const PlanLds& p) {
    const int lane = threadIdx.x & 63;
    for (int e = lane; e < n_expert; e += 64) p.gid[e] = -1;
    int nbits = 1;
    while ((1 << nbits) < n_expert) ++nbits;
    const uint64_t below = lane ? ~0ull >> (64 - lane) : 0ull;
    int groups = 0;
    for (int s = 0; s < n; s += 64) {
        const int i = s + lane;
        const bool in = i < n;
        const int ex = in ? s_ids[i] : 0;
        uint64_t same = __ballot(in);
        for (int b = 0; b < nbits; ++b) {
            const bool bit = (ex >> b) & 1;
            const uint64_t m = __ballot(bit);
            same &= bit ? m : ~m;
        }
        const int rank = __popcll(same & below);
        const bool head = in && rank == 0;
        const int prev = head ? (int)p.gid[ex] : -1;
        const bool opens = head && prev < 0;
        const uint64_t opening = __ballot(opens);
        const int g = opens ? groups + __popcll(opening & below) : prev;
        const int size0 = head && !opens ? p.gsz[g] : 0;
        const int hl = in ? __ffsll((long long)same) - 1 : lane;
        const int eg = __shfl(g, hl, 64), es = __shfl(size0, hl, 64);
        if (in) p.ent[i] = eg | (es + rank) << 16;
        if (head) {
            p.gsz[g] = size0 + __popcll(same);
            if (opens) {
                p.gid[ex] = (int16_t)g;
                p.gexp[g] = ex;
            }
        }
        groups += __popcll(opening);
        __builtin_amdgcn_wave_barrier();
    }
    int carry = 0;
    for (int g0 = 0; g0 < groups; g0 += 64) {
        const int g = g0 + lane;
        const int v = g < groups ? p.gsz[g] : 0;
        int inc = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(inc, o, 64);
            if (lane >= o) inc += y;
        }
        if (g < groups) p.gsz[g] = carry + inc - v;
        carry += __shfl(inc, 63, 64);
    }
    if (lane == 0) p.gsz[groups] = n;
    return groups;
}

// The plan of n entries into the engine's words (PlanWords): wave 0 groups them (plan_groups_wave), then every thread
// of the work-group places its entry and the group it heads.  A group's blob is slot_off[slot] past cache_base when
// the caller maps slots, else slot * blob, with slot = res[expert] (the resident layer's slot) or the expert itself.
// Every thread calls it (n <= blockDim.x).  The last store, after a fence, is *skip = ring.
__device__ __forceinline__ void write_decode_plan(const int* s_ids, const PlanLds& p, int n, int k, int n_expert,
                                                  const int32_t* __restrict__ res, const uint8_t* cache_base,
                                                  const unsigned long long* __restrict__ slot_off, long long blob,
                                                  int32_t* __restrict__ pl, long long cap, uint32_t* skip,
                                                  uint32_t ring) {
    const int t = threadIdx.x;
    __shared__ int s_groups;
    if (t < 64) {
        const int groups = plan_groups_wave(s_ids, n, n_expert, p);
        if (t == 0) s_groups = groups;
    }
    __syncthreads();
    const int groups = s_groups;
    const PlanWords w{cap};
    if (t < n) {
        const int e = p.ent[t];
        const int slot = p.gsz[e & 0xffff] + (e >> 16);
        pl[w.dst() + slot] = t;
        pl[w.tok() + slot] = t / k;
    }
    for (int g = t; g <= groups; g += blockDim.x) {
        pl[w.start() + g] = p.gsz[g];
        if (g == groups) continue;
        const int ex = p.gexp[g];
        const size_t at = res ? (size_t)res[ex] : (size_t)ex;
        const size_t off = slot_off ? (size_t)slot_off[at] : at * (size_t)blob;
        ((unsigned long long*)(pl + w.ptr()))[g] = (unsigned long long)(uintptr_t)(cache_base + off);
    }
    if (t == 0) {
        pl[w.counts() + 0] = groups;
        pl[w.counts() + 1] = n;
        pl[w.counts() + 2] = 0;   // no PCIe groups
        pl[w.start2()] = n;
    }
    __syncthreads();
    if (t == 0) {
        __threadfence();
        *skip = ring;
    }
}

// q8_1 of values 8j .. 8j + 7 of rows whose width is a whole number of 256s (reference iq_kernels.cpp:1850-1879):
// one scale for each 256 values (32 neighbouring lanes), stored in each of their eight blocks; a block's fp16 sum is
// its four 8-value serial sums combined by the xor-1 then xor-2 exchange.  Every lane of the wave calls it (lanes
// with j >= n8 pass in == false): the exchanges are DPP lane moves.
__device__ __forceinline__ void q8_1_256_lane(const float* __restrict__ x, int64_t j, bool in, uint8_t* __restrict__ y) {
    float v[8], a = 0.0f, sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = in ? x[8 * j + q] : 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        a = fmaxf(a, fabsf(v[q]));
        sum += v[q];
    }
    const float amax = group_max32(a);
    sum += dpp_f<kDppXor1>(sum);
    sum += dpp_f<kDppXor2>(sum);
    if (!in) return;
    const float d = q8_scale(amax), id = q8_inv(d);
    const int64_t ib = j / 4, o = 8 * (j % 4);
    uint8_t* blk = y + 36 * ib;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) w0 |= (uint32_t)(uint8_t)q8_value(v[q], id) << (8 * q);
#pragma unroll
    for (int q = 0; q < 4; ++q) w1 |= (uint32_t)(uint8_t)q8_value(v[4 + q], id) << (8 * q);
    ((uint32_t*)(blk + 4 + o))[0] = w0;
    ((uint32_t*)(blk + 4 + o))[1] = w1;
    if (o == 0) *(uint32_t*)blk = (uint32_t)f2h(d) | ((uint32_t)f2h(q8_1_finite(sum)) << 16);
}

// The group-limited sigmoid top-k of one token on one wave (router.hip's router_grouped_sigmoid_wave_kernel, and the
// persistent decode layer's routing stage): expert e = lane PER + j, the groups on whole lanes (n_expert / n_group a
// multiple of PER, lanes a group a power of two).  Lane i < k returns the i-th pick and its weight (s_i / sum of the
// k s, times routed_scale).  Every lane of the wave calls it.
template <int PER>
__device__ __forceinline__ void route_grouped_sigmoid_wave(const float* __restrict__ l, const float* __restrict__ bias,
                                                           int n_expert, int n_group, int topk_group, int k,
                                                           float routed_scale, int& id_out, float& w_out) {
    const int lane = threadIdx.x & 63;
    const int per = n_expert / n_group, lpg = per / PER, my_g = lane / lpg;
    float s[PER], c[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = lane * PER + j;
        const bool in = e < n_expert;
        s[j] = in ? canon_rcp(1.0f + canon_exp(-l[e])) : 0.0f;
        c[j] = in ? s[j] + (bias ? bias[e] : 0.0f) : -INFINITY;
    }
    float b1 = -INFINITY, b2 = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const float v = c[j];
        if (v > b1) { b2 = b1; b1 = v; }
        else if (v > b2) b2 = v;
    }
    for (int o = 1; o < lpg; o <<= 1) {
        const float o1 = __shfl_xor(b1, o, 64), o2 = __shfl_xor(b2, o, 64);
        const float n1 = fmaxf(b1, o1), n2 = fmaxf(fminf(b1, o1), fmaxf(b2, o2));
        b1 = n1;
        b2 = n2;
    }
    const float gs = b1 + b2;
    int rank = 0;
    for (int g = 0; g < n_group; ++g) {
        const float og = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gs), g * lpg));
        rank += og > gs || (og == gs && g < my_g) ? 1 : 0;
    }
    const bool chosen = my_g < n_group && rank < topk_group;
    if (!chosen) {
#pragma unroll
        for (int j = 0; j < PER; ++j) c[j] = -INFINITY;
    }
    // a pass: each lane's best candidate as an unsigned key of c (the float order; NaN and "none" 0, so never picked),
    // the wave's largest key by DPP, its lowest lane by ballot (the lower lane holds the lower experts, and a lane's
    // own ties keep its lower one): better()'s order
    float my_w = 0.0f;
    int my_id = 0;
    for (int i = 0; i < k; ++i) {
        uint32_t lk = 0u;
        int lj = 0;
        float ls = 0.0f;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const float v = c[j] + 0.0f;   // -0 as +0: equal floats, equal keys
            const uint32_t b = __float_as_uint(v);
            const uint32_t key = !chosen || lane * PER + j >= n_expert || v != v ? 0u
                                 : (b & 0x80000000u) ? ~b : (b | 0x80000000u);
            if (key > lk) { lk = key; lj = j; ls = s[j]; }
        }
        const uint32_t m = wave_max_u32(lk);
        if (m == 0u) break;
        const int owner = (int)__builtin_ctzll(__ballot(lk == m));
        const int bi = owner * PER + __builtin_amdgcn_readlane(lj, owner);
        const float sv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ls), owner));
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (lane == owner && j == lj) c[j] = -INFINITY;   // taken
        if (lane == i) { my_w = sv; my_id = bi; }
    }
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), i));
    id_out = my_id;
    w_out = my_w / sum * routed_scale;
}

}  // namespace xs
