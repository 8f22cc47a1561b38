// xestrata-win_amd/csrc/decode_t1.hip - the decode MoE layer for one token in one launch, built for latency.
//
// The same layer and the same arithmetic as the persistent kernel of decode_fused.hip (router -> gate/up -> SwiGLU ->
// q8_1 -> down -> weighted combine -> residual, bit for bit the oracle's canonical rows), arranged so that a token
// waits on as few memory round trips as possible.  One work-group of 1024 threads a CU:
//
//   1. Wave 0 of every work-group routes the token exactly (softmax over all experts in double, top-k, renormalised:
//      router.cpp:59-145's arithmetic, xs_route.h).  Meanwhile waves 1-6 take the top-k of the raw logits - the same
//      experts in the same order unless two probabilities round to one float - and at once issue the LDS DMA of the
//      work-group's gate/up rows for those experts; waves 8-11 quantize x to q8_1 (one scale a 256).  When the exact
//      routing disagrees with the speculation, the DMA is drained and issued again.  The down rows are fetched once
//      the gate/up rows are in (or right after routing by a work-group with no gate/up unit), so that the gate/up
//      rows, which every output waits on, have the memory system to themselves.
//   2. A gate/up unit is one expert's 32 SwiGLU outputs (32 gate rows + 32 up rows), fetched in two halves; each half
//      is computed as it lands.  For Q4_K the integer sums of a block are split over four lanes (exact), then the
//      block scales are applied in the canonical order and the canonical butterfly taken.  h = SwiGLU(gate, up) is
//      quantized per 32 (the canonical q8_1 of the SwiGLU pass, iq_kernels.cpp:2118-2133) and handed over as 9
//      tagged words (8 of four int8 codes, one of the scale), written to 4 replicas.
//   3. A down unit is RD rows of the output for ALL k experts.  Its rows arrived with the first DMA; while h is on its
//      way the Q6_K rows are decoded in LDS to one 6-bit code a byte.  The work-group polls the k experts' q8_1 h,
//      computes the k x RD row dots, and combines them itself in rank order - fl(p0 w0) + fl(p1 w1) + ... then the
//      residual (native_moe_combine_multi + add_inplace) - so no expert output crosses work-groups and there is no
//      separate combine step.
//
// One hand-over is left (h), written and read with device-scope relaxed atomics in 64-bit words whose upper half is
// the call's tag (decode_fused.hip's scheme: no cache maintenance, no word ever reset).  Every wait is bounded and
// points backwards (down units on gate/up units, which wait on nothing), and every work-group of the grid is resident.
// Instances exist for config 2's (Q4_K / Q6_K, hidden 2048, F 768), the same shape all Q4_K, and config 1's (Q8_0,
// 1024, 512) layers; other layouts run decode_fused.hip's kernel.
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_route.h"
#include "xs_units.h"

#include <mutex>
#include <vector>

namespace xs {

namespace {

constexpr int kT1 = 1024;          // threads a work-group: 16 waves, 4 a SIMD
constexpr int kT1Waves = kT1 / 64;
// waves 1..6: speculative routing and the weight DMA.  The issuing waves stall while the memory queues are full, so
// more of them put the rows in flight sooner: config 2's layer 13.40 us with 3, 13.45 with 4, 12.96 with 5, 12.91 with
// 6, 12.96 with 7, 13.13 with 8, 13.07 with 10 (config 1's: 8.98, 8.40, 8.30, 8.04, 8.07 us with 3 to 7)
constexpr int kSpecWaves = 6;
constexpr int kXWave0 = 8;         // waves 8..11: x to q8_1 (H / 8 chunks of 8 values, a thread each a round)
static_assert(kXWave0 > kSpecWaves && kXWave0 + 4 <= 15, "x's waves are neither routing, DMA nor store waves");
constexpr int kStoreWave = kT1Waves - 1;   // the wave that writes the hand-over words (and loads nothing after x)
constexpr int kDnWave0 = 4, kDnWaves = 4;   // waves 4..7: the DMA of the down rows (4..6 issue it after their
                                            // speculative gate/up DMA has drained) and the decode of the rows after it;
                                            // they neither poll nor write h
constexpr int kHWords = 9;         // tagged words a 32-value q8_1 block of h: 8 x four codes, 1 scale
constexpr int kFirstPollTicks = 140;   // wall-clock ticks (100 MHz) from a work-group's h store to its first h read
// Every work-group polls every block of h with device-scope loads, which go past the L2 to the memory channel that
// owns the line, and reads of one line queue there one after another: with the whole grid on each line a poll took
// ~3 us to see a store.  So every block is written kHRep times, replica r read by the work-groups b with b % kHRep
// == r, and the blocks of a replica lie t1_h_stride(k) words apart (other lines, mostly other channels).  The
// hand-over region holds 256 * n_ff words: kHRep replicas of k * n_ff / 32 blocks (k <= 64).  With the first reads
// timed from the work-group's own store (below), 4 replicas measured fastest: config 2's layer 13.46 -> 13.42 us and
// config 1's 9.11 -> 8.92 against 8, while 2 and 1 lose again (fewer stores, but more readers on each line).
constexpr int kHRep = 4;
__host__ __device__ constexpr int t1_h_stride(int k) { return 1024 / k < 16 ? 16 : 1024 / k; }
__host__ __device__ constexpr int t1_h_replica(int k, int F) { return 32 * F; }   // words between replicas
constexpr int kT1MaxK = 64;

__host__ __device__ constexpr int t1_up16(int v) { return (v + 15) & ~15; }
__host__ __device__ inline int t1_act_stride(int n) { return t1_up16(n + n / 8 + n / 4); }

// the gate/up activation's bytes between the int8 values of consecutive 256-value blocks: Q4_K's four lanes a block
// read 64-value pieces of eight blocks at once, so the blocks start 16 bytes apart in the LDS banks
template <int TG>
constexpr int t1_act_qs() { return TG == kQ4_K ? 272 : 256; }
__host__ __device__ inline int t1_act_bytes(int n, int qs) { return t1_up16(n / 256 * qs + n / 8 + n / 4); }
// a decoded Q6_K down row: F 6-bit codes (one a byte), F / 16 sub-block scales, F / 256 block scales (float)
__host__ __device__ constexpr int t1_dec_stride(int F) { return t1_up16(F + F / 16 + 4 * (F / 256)) + 16; }

struct T1Lds {
    int ids, w, spec, misc, gu, po, hq, part, act_x, slab_gu, slab_dn, act_d, total;
};
__host__ __device__ inline T1Lds t1_lds(int k, int H, int F, int gu_row, int d_row, int rd, int qs, bool decode) {
    T1Lds o;
    int at = 0;
    o.ids = at; at += t1_up16(kT1MaxK * 4);
    o.w = at; at += t1_up16(kT1MaxK * 4);
    o.spec = at; at += t1_up16(kT1MaxK * 4);
    o.misc = at; at += t1_up16(16 * 4);
    o.gu = at; at += t1_up16(64 * 4);
    o.po = at; at += t1_up16(k * rd * 4);
    o.hq = at; at += t1_up16(64);
    // gate/up's integer parts; in the down phase, the list of units to compute here (t1_help_unit)
    const int part = 32 * (H / 256) * 8, help = 4 * (1 + k * (F / 32));
    o.part = at; at += t1_up16(part > help ? part : help);
    o.act_x = at; at += t1_act_bytes(H, qs);
    o.slab_gu = at;   // the gate/up rows; then, decoded, the down rows
    const int gu = 64 * gu_row, dec = decode ? k * rd * t1_dec_stride(F) : 0;
    at += t1_up16(gu > dec ? gu : dec);
    o.slab_dn = at; at += t1_up16(k * rd * d_row);
    o.act_d = at; at += k * t1_act_stride(F);
    o.total = at;
    return o;
}

__device__ __forceinline__ void t1_st_tag(unsigned long long* p, uint32_t v, unsigned int tag) {
    __hip_atomic_store(p, ((unsigned long long)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long t1_ld_tag(const unsigned long long* p) {
    return __hip_atomic_load((unsigned long long*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void t1_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void t1_vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// wait until at most n of the wave's vector memory operations are outstanding (n wave-uniform; past 31, 31: a wait
// for more than asked, never less)
__device__ __forceinline__ void t1_vm_wait_le(int n) {
    switch (n < 31 ? n : 31) {
#define XS_T1_VMW(i) \
    case i: asm volatile("s_waitcnt vmcnt(" #i ")" ::: "memory"); break;
        XS_T1_VMW(0) XS_T1_VMW(1) XS_T1_VMW(2) XS_T1_VMW(3) XS_T1_VMW(4) XS_T1_VMW(5) XS_T1_VMW(6) XS_T1_VMW(7)
        XS_T1_VMW(8) XS_T1_VMW(9) XS_T1_VMW(10) XS_T1_VMW(11) XS_T1_VMW(12) XS_T1_VMW(13) XS_T1_VMW(14)
        XS_T1_VMW(15) XS_T1_VMW(16) XS_T1_VMW(17) XS_T1_VMW(18) XS_T1_VMW(19) XS_T1_VMW(20) XS_T1_VMW(21)
        XS_T1_VMW(22) XS_T1_VMW(23) XS_T1_VMW(24) XS_T1_VMW(25) XS_T1_VMW(26) XS_T1_VMW(27) XS_T1_VMW(28)
        XS_T1_VMW(29) XS_T1_VMW(30) XS_T1_VMW(31)
#undef XS_T1_VMW
        default: break;
    }
}

// n16 16-byte chunks to LDS dst[0 .. n16) by the DMA of waves W0 .. W0 + NW - 1 (global_load_lds_dwordx4: one
// instruction of a wave fills 64 consecutive chunks at a wave-uniform LDS address)
template <int W0, int NW, typename Src>
__device__ __forceinline__ void t1_dma(uint8_t* dst, int n16, Src src) {
    const int lane = threadIdx.x & 63, r = (threadIdx.x >> 6) - W0;
    for (int base = 64 * r; base < n16; base += 64 * NW) {
        const int i = base + lane;
        if (i < n16)
            __builtin_amdgcn_global_load_lds(src(i), (__attribute__((address_space(3))) void*)(dst + 16 * base), 16, 0,
                                             2 /* nt */);
    }
}
// the number of DMA instructions t1_dma<W0, NW> issues in this wave for n16 chunks
template <int W0, int NW>
__device__ __forceinline__ int t1_dma_count(int n16) {
    const int r = (threadIdx.x >> 6) - W0;
    return n16 > 64 * r ? (n16 - 64 * r + 64 * NW - 1) / (64 * NW) : 0;
}

// The top-k of the raw logits, in order (larger first, the lower index on a tie; NaN never wins): exp is monotone, so
// these are the exact routing's experts in its order unless two of their probabilities round to one float.  Lane i
// < k of the wave returns the i-th (-1 when fewer than k logits are numbers).
template <int PER>
__device__ __forceinline__ int spec_topk(const float (&lv)[PER], int n_expert, int k) {
    const int lane = threadIdx.x & 63;
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int x = lane + 64 * j;
        const uint32_t u = __float_as_uint(lv[j]);
        const uint32_t s = (u & 0x80000000u) ? ~u : (u | 0x80000000u);   // order-preserving, 0 below every number
        key[j] = x < n_expert && lv[j] == lv[j] ? (s == 0u ? 1u : s) : 0u;
    }
    int mine = -1;
    for (int i = 0; i < k; ++i) {
        uint32_t m = key[0];
#pragma unroll
        for (int j = 1; j < PER; ++j) m = m > key[j] ? m : key[j];
        const uint32_t best = wave_max_u32(m);
        if (best == 0u) break;
        unsigned long long e = 0ull;
        int wj = 0;
#pragma unroll
        for (int j = PER - 1; j >= 0; --j) {
            const unsigned long long ej = __builtin_amdgcn_uicmp(key[j], best, 32 /* eq */);
            wj = ej ? j : wj;
            e = ej ? ej : e;
        }
        const int wl = __builtin_ctzll(e);
#pragma unroll
        for (int j = 0; j < PER; ++j) key[j] = j == wj && lane == wl ? 0u : key[j];
        if (lane == i) mine = wl + 64 * wj;
    }
    return mine;
}

__device__ __forceinline__ unsigned long long t1_load_counter(const FusedArgs& a) {
    const int lane = threadIdx.x & 63;
    return lane < 16 ? __hip_atomic_load((unsigned long long*)(a.sync + 32 * lane), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT)
                     : 0ull;
}
// the call's tag, 1 .. 2^32 - 1 (decode_fused.hip's call_tag: the epoch mod 2^32 - 1, plus one; never 0)
__device__ __forceinline__ unsigned int t1_tag(unsigned long long c) {
    c += dpp_u64<kDppXor1, 0xF>(c);
    c += dpp_u64<kDppXor2, 0xF>(c);
    c += dpp_u64<kDppRor4, 0xF>(c);
    c += dpp_u64<kDppRor8, 0xF>(c);
    const unsigned int lo = __builtin_amdgcn_readlane((int)c, 0), hi = __builtin_amdgcn_readlane((int)(c >> 32), 0);
    const unsigned long long epoch = (((unsigned long long)hi << 32) | lo) >> 20;
    return (unsigned int)(epoch % 0xFFFFFFFFull) + 1u;
}
__device__ __forceinline__ void t1_done(const FusedArgs& a) {   // this work-group's share of the call's 2^20
    if (threadIdx.x != 0) return;
    const unsigned int G = gridDim.x, b = blockIdx.x;
    const unsigned long long share = (1ull << 20) / G + (b < (1u << 20) % G ? 1ull : 0ull);
    __hip_atomic_fetch_add((unsigned long long*)(a.sync + 32 * (b % 16)), share, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// A gate/up unit that a waiter found unmarked - its owner had not started 5 us into the wait (other work held the
// compute units its work-group needed) - computed by the waiting work-group itself from the rows in HBM: the 64
// canonical row dots (Unit::apply: the same sums the owner's own form gives, bit for bit), SwiGLU, the q8_1 block;
// into this work-group's down activation for expert rank e (block j) and, tagged, into every replica for the other
// waiters.  An owner that starts later computes and stores the same bits again.  Every thread calls it.  (Inlined: a
// call would give the kernel a stack - scratch memory every launch sets up - and twice the registers.)
template <int TG, int H, int F>
__device__ __forceinline__ void t1_help_unit(const uint8_t* arena, long long blob_bytes, long long up_off,
                                          unsigned long long* hx, int q, int k, unsigned int tag, const int* s_ids,
                                          Act ax, Act ad, float* s_gu) {
    using UG = Unit<TG, true, t1_act_qs<TG>() - 256>;   // (x's blocks lie t1_act_qs apart in LDS)
    constexpr int nu = F / 32, gu_row = (int)row_bytes(TG, H);
    constexpr int lprc = canon_lanes(H / UG::kUnit);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int e = q / nu, j = q - e * nu;
    const uint8_t* blob = arena + (size_t)s_ids[e] * (size_t)blob_bytes;
    const int c = lane & (lprc - 1);
    for (int rr = tid / lprc; rr < 64; rr += kT1 / lprc) {   // gate rows 0..31, then up rows 0..31 of unit j
        const uint8_t* row = rr < 32 ? blob + (size_t)(32 * j + rr) * gu_row
                                     : blob + up_off + (size_t)(32 * j + rr - 32) * gu_row;
        float acc[1] = {0.0f};
        const Act at[1] = {ax};
        for (int u = c; u < H / UG::kUnit; u += lprc) UG::template apply<1>(row, 0, u, at, 1, acc);
        const float sm = lane0_sum<lprc>(acc[0]);
        if (c == 0) s_gu[rr] = sm;
    }
    __syncthreads();
    if (wave == 0) {
        const float h = lane < 32 ? canon_silu_mul(s_gu[lane], s_gu[32 + lane]) : 0.0f;
        const float amax = group_max32(fabsf(h));   // lanes 0..31 hold the block
        const float d = q8_scale(amax), id = q8_inv(d);
        const uint32_t code = lane < 32 ? (uint32_t)(uint8_t)(int8_t)q8_value(h, id) : 0u;
        uint32_t word = 0;   // lane i < 8: codes 4 i .. 4 i + 3
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t cb = (uint32_t)__shfl((int)code, (4 * lane + b) & 63, 64);
            word |= cb << (8 * b);
        }
        const uint32_t dbits = (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(h2f(f2h(d))), 0);
        const uint32_t val = lane < 8 ? word : dbits;   // lane i < 9: word i of the block
        const int s4 = lane < 8 ? sdot4((int)word, 0x01010101, 0) : 0;
        const int s8 = s4 + __shfl_xor(s4, 1, 64);
        const int s16 = s8 + __shfl_xor(s8, 2, 64);   // lane 0: codes 0..15, lane 4: 16..31
        if (lane < 8) ((uint32_t*)(ad.q + 32 * j))[lane] = word;
        if (lane == 0) ((int*)ad.us16)[2 * j] = s16;
        if (lane == 4) ((int*)ad.us16)[2 * j + 1] = s16;
        if (lane == 8) ((float*)ad.d8)[j] = __uint_as_float(dbits);
        static_assert(kHRep * kHWords <= 128, "two stores a lane");
        const uint32_t v0 = (uint32_t)__shfl((int)val, lane % kHWords, 64);          // (every lane active)
        const uint32_t v1 = (uint32_t)__shfl((int)val, (lane + 64) % kHWords, 64);
        for (int li = lane; li < kHRep * kHWords; li += 64) {
            const int r = li / kHWords, i = li - r * kHWords;
            t1_st_tag(hx + (size_t)r * t1_h_replica(k, F) + (size_t)q * t1_h_stride(k) + i, li < 64 ? v0 : v1, tag);
        }
    }
    __syncthreads();
}

// One token, at a hidden size H, expert width F and RD down rows a unit known at compile time (every index below is
// then shifts and constants).  a.nu: gate/up units an expert (F / 32); a.nj: down units (H / RD).
template <int TG, int TD, int PER, int H, int F, int RD>
__global__ __launch_bounds__(kT1) void moe_decode_t1_kernel(FusedArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    using UG = Unit<TG, true>;
    using UD = Unit<TD, false>;
    constexpr bool kSplitGU = TG == kQ4_K;   // gate/up: four lanes a block, integer parts, the scales per row after
    constexpr bool kDecode = TD == kQ6_K;    // down: the rows decoded to 6-bit codes while h is on its way
    constexpr int QS = t1_act_qs<TG>();
    const ExpertLayout& L = a.L;
    constexpr int rd = RD, nu = F / 32;
    constexpr int gu_row = (int)row_bytes(TG, H), d_row = (int)row_bytes(TD, F);
    const int k = a.k, E = a.n_expert;
    const T1Lds o = t1_lds(k, H, F, gu_row, d_row, rd, QS, kDecode);
    int* s_ids = (int*)(lds + o.ids);
    float* s_w = (float*)(lds + o.w);
    int* s_spec = (int*)(lds + o.spec);
    int* s_misc = (int*)(lds + o.misc);   // [0] 0 good / -1 bad routing, [1] the call's tag, [2] down-row waves
                                          // drained, [3] units to compute here, [4] the h store's time (| 1)
    float* s_gu = (float*)(lds + o.gu);   // gate outputs 0..31, then up outputs 0..31
    float* s_po = (float*)(lds + o.po);
    uint8_t* s_hq = lds + o.hq;
    int2* s_part = (int2*)(lds + o.part);
    uint8_t* slab_gu = lds + o.slab_gu;
    uint8_t* slab_dn = lds + o.slab_dn;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, b = blockIdx.x;
    int8_t* qx = (int8_t*)(lds + o.act_x);
    constexpr int nbx = H / 256;
    const Act ax{qx, (const float*)(qx + nbx * QS), (const int*)(qx + nbx * QS + H / 8)};
    auto act_d = [&](int e) {
        int8_t* q = (int8_t*)(lds + o.act_d) + e * t1_act_stride(F);
        return Act{q, (const float*)(q + F), (const int*)(q + F + F / 8)};
    };
    const bool spec_wave = wave >= 1 && wave <= kSpecWaves;
    const bool dn_wave = wave >= kDnWave0 && wave < kDnWave0 + kDnWaves;
    const bool has_gu = b < k * nu;   // (the host makes the grid at least the unit counts)
    const int g_gu = has_gu ? b / nu : 0, j_gu = has_gu ? b - g_gu * nu : 0;
    const int j_dn = b;               // down unit: rows j_dn * rd .. + rd of every expert
    const bool has_dn = j_dn < a.nj;
    constexpr int n16_half = 32 * gu_row / 16, n16_dn = rd * d_row / 16;
    static_assert((16 * gu_row) % 16 == 0 && (rd * d_row) % 16 == 0, "16-byte DMA chunks");
    // this wave's DMA instructions of gate/up half B (wave-uniform)
    const int n_b = __builtin_amdgcn_readfirstlane(has_gu ? t1_dma_count<1, kSpecWaves>(n16_half) : 0);

    // the DMA of this work-group's rows for the experts id_of(0 .. k) (rank order; id_of(i) wave-uniform): the slab
    // holds half A (gate rows 0..15, up rows 0..15 of the unit's 32) then half B (rows 16..31 of each).  The down rows
    // are fetched apart (issue_dn), once the gate/up rows have landed: fetched together, the down rows' bytes share
    // the memory system with the gate/up rows that every output waits on, and all of them land late.
    auto issue = [&](auto id_of) {
        if (has_gu) {
            const uint8_t* blob = a.arena + (size_t)id_of(g_gu) * (size_t)a.blob;
            for (int hh = 0; hh < 2; ++hh) {
                const uint8_t* sg = blob + ((size_t)j_gu * 32 + 16 * hh) * gu_row;
                const uint8_t* su = blob + L.up_off + ((size_t)j_gu * 32 + 16 * hh) * gu_row;
                const int n16g = n16_half / 2;
                t1_dma<1, kSpecWaves>(slab_gu + hh * 32 * gu_row, n16_half, [&](int i) {
                    return (const void*)(i < n16g ? sg + 16 * (size_t)i : su + 16 * (size_t)(i - n16g));
                });
            }
        }
    };
    auto issue_dn = [&](auto id_of) {
        if (has_dn)
            for (int e = 0; e < k; ++e) {
                const uint8_t* sd =
                    a.arena + (size_t)id_of(e) * (size_t)a.blob + L.down_off + (size_t)j_dn * rd * d_row;
                t1_dma<kDnWave0, kDnWaves>(slab_dn + e * rd * d_row, n16_dn,
                                           [&](int i) { return (const void*)(sd + 16 * (size_t)i); });
            }
    };

    // the combine's operands that depend on no work of this call - the residual, the shared expert's row and its gate
    // logit - loaded now by the threads that combine (loaded at the end, their latency was the kernel's last step)
    static_assert(RD <= kT1, "a thread a combined row");
    const bool combiner = has_dn && tid < rd;
    float c_res = 0.0f, c_sh = 0.0f, c_gate = 0.0f;
    if (combiner) {
        const int64_t col = (int64_t)j_dn * rd + tid;
        c_res = a.residual[col];
        if (a.shared) c_sh = a.shared[col];
        if (a.shared && a.shared_gate) c_gate = a.shared_gate[0];
    }

    // ---- 1. routing (wave 0 exact; waves 1..6 speculate and fetch; waves 8..11 quantize x)
    if (wave == 0) {
        float lv[PER];
        load_logits_wave<PER>(a.logits, E, lv);
        const unsigned long long ctr = t1_load_counter(a);
        if (lane < k) {
            s_ids[lane] = -1;
            s_w[lane] = 0.0f;
        }
        route_topk_wave_lv<PER>(lv, E, k, s_ids, s_w);
        const unsigned int ep = t1_tag(ctr);
        const int ex = lane < k ? s_ids[lane] : 0;
        const bool bad = __ballot(lane < k && (ex < 0 || ex >= E)) != 0;
        if (lane == 0) {
            s_misc[0] = bad ? -1 : 0;
            s_misc[1] = (int)ep;
            s_misc[2] = 0;
            s_misc[3] = 0;
            s_misc[4] = 0;
        }
    } else if (spec_wave) {
        float lv[PER];
        load_logits_wave<PER>(a.logits, E, lv);
        const int sp = spec_topk<PER>(lv, E, k);
        const bool ok = __ballot(lane < k && (sp < 0 || sp >= E)) == 0;
        if (wave == 1 && lane < k) s_spec[lane] = ok ? sp : -1;
        if (ok) issue([&](int i) { return __builtin_amdgcn_readlane(sp, i); });   // lane i holds the i-th
    } else if (wave >= kXWave0 && wave < kXWave0 + 4) {
        for (int j8 = tid - 64 * kXWave0; j8 < H / 8; j8 += 256) {
            // q8_1 of values 8 j8 .. + 7, one scale a 256 (32 neighbouring lanes): quantize_q8_1_rows's values
            float v[8], am = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[i] = a.x[8 * j8 + i];
                am = fmaxf(am, fabsf(v[i]));
            }
            const float amax = group_max32(am);
            const float d = q8_scale(amax), id = q8_inv(d);
            uint32_t w0 = 0, w1 = 0;
            int sq = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q0 = q8_value(v[i], id), q1 = q8_value(v[4 + i], id);
                w0 |= (uint32_t)(uint8_t)q0 << (8 * i);
                w1 |= (uint32_t)(uint8_t)q1 << (8 * i);
                sq += q0 + q1;
            }
            *(uint2*)(qx + (j8 >> 5) * QS + 8 * (j8 & 31)) = make_uint2(w0, w1);
            const int s16 = sq + dpp_i<kDppXor1>(sq);
            if ((j8 & 1) == 0) ((int*)ax.us16)[j8 >> 1] = s16;
            if ((j8 & 3) == 0) ((float*)ax.d8)[j8 >> 2] = h2f(f2h(d));
        }
    }
    // routing, speculation and x are in LDS.  An LDS-only barrier: __syncthreads() would also make the DMA waves wait
    // for every load in flight (a work-group release); the DMA waits are explicit below.
    t1_lds_barrier();
    if (s_misc[0] < 0) {   // a rank left unwritten (NaN logits): no output this call
        if (tid == 0) atomicOr(a.err, 4);
        if (spec_wave) t1_vm_drain();
        t1_done(a);
        return;
    }
    const unsigned int tag = (unsigned int)s_misc[1];
    // this work-group runs its gate/up unit: the mark a waiter checks before it waits on the unit (the store wave
    // writes it; it loads nothing after x)
    if (has_gu && wave == kStoreWave && lane == 0)
        __hip_atomic_store(a.marks + 32 * (b & 31) + (b >> 5), tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool same = true;
    for (int i = 0; i < k; ++i) same = same && s_spec[i] == s_ids[i];
    if (!same && spec_wave) {   // the speculation missed: drain what it fetched, fetch the exact experts' rows
        t1_vm_drain();
        issue([&](int i) { return s_ids[i]; });
    }
    // a work-group with no gate/up unit fetches its down rows now; the others once their gate/up rows are in
    if (!has_gu && dn_wave) issue_dn([&](int i) { return s_ids[i]; });
    if (b == 0 && tid < k) {
        a.ids[tid] = s_ids[tid];
        a.weights[tid] = s_w[tid];
    }

    // ---- 2. the gate/up unit: 32 gate rows + 32 up rows of expert g_gu, SwiGLU, q8_1, handed over
    if (has_gu) {
        if constexpr (kSplitGU) {
            // per half: integer parts of each (row, block) on four lanes (the 64-value pieces p = 0..3 of the block,
            // Unit<Q4_K>'s s1 / s2, summed over the quad: exact), then a thread a row applies the block scales in
            // the canonical order (lane c's blocks c, c + L, ..: fma(d d8, s1), fma(-dmin d8, s2)) and the lanes'
            // butterfly (acc[c] += acc[c ^ o], o = L/2 .. 1)
            for (int hh = 0; hh < 2; ++hh) {
                if (spec_wave) t1_vm_wait_le(hh == 0 ? n_b : 0);
                t1_lds_barrier();
                const uint8_t* half = slab_gu + hh * 32 * gu_row;
                for (int t = tid; t < 32 * nbx * 4; t += kT1) {
                    const int p = t & 3, rb = t >> 2, blk = rb % nbx, row = rb / nbx;
                    const uint8_t* bp = half + row * gu_row + 144 * blk;
                    const uint4 hdr = *(const uint4*)bp;
                    int sc0, m0, sc1, m1;
                    q4k_sm(hdr.y, hdr.z, hdr.w, 2 * p, sc0, m0);
                    q4k_sm(hdr.y, hdr.z, hdr.w, 2 * p + 1, sc1, m1);
                    const uint4 w0 = *(const uint4*)(bp + 16 + 32 * p), w1 = *(const uint4*)(bp + 32 + 32 * p);
                    const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                    const int8_t* q = ax.q + blk * QS + 64 * p;
                    const uint4 l0 = *(const uint4*)q, l1 = *(const uint4*)(q + 16);
                    const uint4 h0 = *(const uint4*)(q + 32), h1 = *(const uint4*)(q + 48);
                    const uint32_t al[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
                    const uint32_t ah[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
                    int il = 0, ih = 0;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        il = sdot4((int)(w[i] & 0x0F0F0F0Fu), (int)al[i], il);
                        ih = sdot4((int)((w[i] >> 4) & 0x0F0F0F0Fu), (int)ah[i], ih);
                    }
                    int s1 = sc0 * il + sc1 * ih;
                    int s2 = m0 * us32(ax, 8 * blk + 2 * p) + m1 * us32(ax, 8 * blk + 2 * p + 1);
                    s1 += dpp_i<kDppXor1>(s1);
                    s1 += dpp_i<kDppXor2>(s1);
                    s2 += dpp_i<kDppXor1>(s2);
                    s2 += dpp_i<kDppXor2>(s2);
                    if (p == 0) s_part[row * nbx + blk] = make_int2(s1, s2);
                }
                t1_lds_barrier();
                // lane c of a row's lpr: the scales of blocks c, c + lpr, .. in order, then the canonical butterfly
                constexpr int lpr_c = canon_lanes(nbx);
                for (int t = tid; t < 32 * lpr_c; t += kT1) {
                    const int row = t / lpr_c, c = t % lpr_c;
                    const uint8_t* rp = half + row * gu_row;
                    float acc = 0.0f;
#pragma unroll
                    for (int blk = c; blk < nbx; blk += lpr_c) {
                        const uint32_t dd = *(const uint32_t*)(rp + 144 * blk);
                        const float d = h2f((uint16_t)(dd & 0xFFFFu)), dmin = h2f((uint16_t)(dd >> 16));
                        const float d8 = ax.d8[8 * blk];
                        const int2 sp = s_part[row * nbx + blk];
                        acc = __builtin_fmaf(d * d8, (float)sp.x, acc);
                        acc = __builtin_fmaf(-(dmin * d8), (float)sp.y, acc);
                    }
                    acc = lane0_sum<lpr_c>(acc);
                    const int out = 16 * hh + (row & 15);
                    if (c == 0) s_gu[(row < 16 ? 0 : 32) + out] = acc;
                }
            }
        } else {
            if (spec_wave) t1_vm_drain();   // the gate/up rows have landed
            t1_lds_barrier();
            constexpr int lprc = canon_lanes(H / UG::kUnit);
            const int c = lane & (lprc - 1);
            for (int rr = tid / lprc; rr < 64; rr += kT1 / lprc) {
                float acc[1] = {0.0f};
                const Act at[1] = {ax};
                for (int u = c; u < H / UG::kUnit; u += lprc)
                    UG::template apply<1>(slab_gu, rr * gu_row, u, at, 1, acc);
                const float sm = lane0_sum<lprc>(acc[0]);
                // slab row rr: half rr / 32, gate rows first in each half
                const int hh = rr >> 5, row = rr & 31, out = 16 * hh + (row & 15);
                if (c == 0) s_gu[(row < 16 ? 0 : 32) + out] = sm;
            }
        }
        t1_lds_barrier();
        if (dn_wave) issue_dn([&](int i) { return s_ids[i]; });   // the gate/up rows are in and done with
        if (wave == kStoreWave) {
            // lane i < 32: h_i = SwiGLU(gate_i, up_i); the block's scale from the 32 |h|; codes; 9 tagged words
            const float h = lane < 32 ? canon_silu_mul(s_gu[lane], s_gu[32 + lane]) : 0.0f;
            const float amax = group_max32(fabsf(h));   // lanes 0..31 hold the block
            const float d = q8_scale(amax), id = q8_inv(d);
            if (lane < 32) s_hq[lane] = (uint8_t)(int8_t)q8_value(h, id);
            __builtin_amdgcn_wave_barrier();
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            // lane 9 r + i (r < kHRep, i < 9): word i of replica r
            const uint32_t dbits = (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(h2f(f2h(d))), 0);   // lanes
                                                                          // 32..63 reduced a block of zeros
            for (int li = lane; li < kHRep * kHWords; li += 64) {
                const int r = li / kHWords, i = li - r * kHWords;
                unsigned long long* dst =
                    a.hx + (size_t)r * t1_h_replica(k, F) + (size_t)(g_gu * nu + j_gu) * t1_h_stride(k);
                t1_st_tag(dst + i, i < 8 ? ((const uint32_t*)s_hq)[i] : dbits, tag);
            }
            if (lane == 0)   // when this work-group's h was stored: the pollers time their first read from it
                __hip_atomic_store(&s_misc[4], (int)((uint32_t)wall_clock64() | 1u), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }

    // ---- 3. the down unit: rows j_dn * rd .. + rd of all k experts, combined in rank order, + residual
    if (has_dn) {
        int* s_help = (int*)s_part;   // [1 ..]: the units to compute here, s_misc[3] of them (s_part is free after
                                      // gate/up)
        if (dn_wave) {   // the down rows have landed: counted in LDS (no barrier: the pollers need not wait for them)
            t1_vm_drain();
            if (lane == 0) __hip_atomic_fetch_add(&s_misc[2], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        auto rows_in = [&]() {
            return __hip_atomic_load(&s_misc[2], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= kDnWaves;
        };
        uint8_t* dec = slab_gu;         // (the gate/up rows were done with at the barrier before the h hand-over)
        constexpr int dstr = t1_dec_stride(F);
        const int nblk = k * nu;
        // waves 0 .. kPollWaves - 1 poll h while the others decode the down rows
        constexpr int kPollWaves = 3, kDecThreads = kT1 - 64 * (kPollWaves + 1);
        const bool poller = wave < kPollWaves;
        const int dtid = tid - 64 * kPollWaves;
        // the k experts' q8_1 h: one block (9 words) a thread of the poller waves, read whole first; then the
        // block's scale word alone (9x fewer loads in flight across the grid) until it carries the tag, and the block
        // again.  (A word a lane, so that a wave's load reads a few lines, measured slower.)  The first read goes out
        // kFirstPollTicks after this work-group's own h store, or when its down rows have landed if that is sooner
        // (a work-group with no gate/up unit: when they land); a first read that misses waits for the down rows.
        // Reads issued earlier, while h is not yet visible and the down rows are in flight, slow both: a first read
        // at 0.6 or 1.0 us after the store took the layer from 13.7 to 15.1 or 14.6 us, at 1.4 us to 13.5 (config
        // 1: 9.2 -> 9.0 us); polling from the end of gate/up on, 19.3 us.
        if (poller)
            for (int q = tid; q < nblk; q += 64 * kPollWaves) {
                const int e = q / nu, j = q - e * nu;
                const unsigned long long* src =
                    a.hx + (size_t)(b % kHRep) * t1_h_replica(k, F) + (size_t)q * t1_h_stride(k);
                unsigned long long w[kHWords];
                auto poll = [&](unsigned long long (&v)[kHWords]) {
#pragma unroll
                    for (int i = 0; i < kHWords; ++i) v[i] = t1_ld_tag(src + i);
                };
                auto tagged = [&](const unsigned long long (&v)[kHWords]) {
                    bool ok = true;
#pragma unroll
                    for (int i = 0; i < kHWords; ++i) ok = ok && (unsigned int)(v[i] >> 32) == tag;
                    return ok;
                };
                // (spin_ticks <= 0: the host forces every wait to expire at once - a test of the error path;
                // help_ticks < 0: every unit is computed here - a test of that path.)  Polled for help_ticks (5 us)
                // first; a block still not stored then is rare: its owner's mark is read - no mark, the owner has not
                // started (other work holds the compute units it needs), so the unit goes on this work-group's list
                // to be computed here after the polls; else the wait goes on for the rest of the bound.  So no wait
                // depends on a work-group that is not resident.
                // (every wait here ends: the store wave and the down-row waves are this work-group's own)
                if (has_gu) {
                    int st;
                    while ((st = __hip_atomic_load(&s_misc[4], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0)
                        __builtin_amdgcn_s_sleep(1);
                    while ((int)((uint32_t)wall_clock64() - (uint32_t)st) < kFirstPollTicks && !rows_in())
                        __builtin_amdgcn_s_sleep(1);
                } else {
                    while (!rows_in()) __builtin_amdgcn_s_sleep(1);
                }
                poll(w);
                bool good = a.spin_ticks > 0 && a.help_ticks >= 0 && tagged(w);
                if (!good)
                    while (!rows_in()) __builtin_amdgcn_s_sleep(1);
                long long t0 = wall_clock64();
                for (int it = 1; !good && a.spin_ticks > 0; ++it) {
                    const unsigned long long wd = t1_ld_tag(src + 8);
                    if ((unsigned int)(wd >> 32) == tag) {
                        poll(w);
                        if (tagged(w)) {
                            good = true;
                            break;
                        }
                    }
                    if ((it & 15) == 0 && wall_clock64() - t0 > a.help_ticks) break;
                    __builtin_amdgcn_s_sleep(8);
                }
                if (!good && a.spin_ticks > 0) {
                    if (a.help_ticks < 0 || __hip_atomic_load(a.marks + 32 * (q & 31) + (q >> 5), __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT) != tag) {
                        s_help[1 + atomicAdd(&s_misc[3], 1)] = q;
                        continue;
                    }
                    for (int it = 1; !good; ++it) {
                        const unsigned long long wd = t1_ld_tag(src + 8);
                        if ((unsigned int)(wd >> 32) == tag) {
                            poll(w);
                            good = tagged(w);
                        }
                        if (!good && (it & 15) == 0 && wall_clock64() - t0 > a.spin_ticks) break;
                        __builtin_amdgcn_s_sleep(8);
                    }
                }
                if (!good) {
                    atomicOr(a.err, 2);
#pragma unroll
                    for (int i = 0; i < kHWords; ++i) w[i] = 0ull;
                }
                const Act ad = act_d(e);
                uint32_t* qd = (uint32_t*)(ad.q + 32 * j);
                int s0 = 0, s1 = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    qd[i] = (uint32_t)w[i];
                    if (i < 4) s0 = sdot4((int)(uint32_t)w[i], 0x01010101, s0);
                    else s1 = sdot4((int)(uint32_t)w[i], 0x01010101, s1);
                }
                ((int*)ad.us16)[2 * j] = s0;
                ((int*)ad.us16)[2 * j + 1] = s1;
                ((float*)ad.d8)[j] = __uint_as_float((uint32_t)w[8]);
            }
        if (kDecode && !poller && wave != kStoreWave) {
            while (!rows_in()) __builtin_amdgcn_s_sleep(1);   // (their DMA waves drained and counted themselves)
            // each row's 6-bit codes, one a byte (ql | qh << 4, Unit<Q6_K>'s words), its sub-block and block scales:
            // the products after h arrives are then plain int8 dots
            // 16 values a task (half of a 32-value group): 16 ql bytes and 16 qh bytes as aligned words, realigned
            constexpr int cpr = F / 16;   // tasks a row
            for (int t = dtid; t < k * rd * cpr; t += kDecThreads) {
                const int rr = t / cpr, ch = t % cpr, g = ch >> 1, h16 = ch & 1;
                const int bb = g >> 3, gg = g & 7, hn = gg >> 2, sg = gg & 3;
                const int boff = rr * d_row + 210 * bb;
                uint32_t ql[4], qh[4];
                lds_words_a2<4>(slab_dn, boff + 64 * hn + 32 * (sg & 1) + 16 * h16, ql);
                lds_words_a2<4>(slab_dn, boff + 128 + 32 * hn + 16 * h16, qh);
                uint4 cw;
                cw.x = ((ql[0] >> (4 * (sg >> 1))) & 0x0F0F0F0Fu) | (((qh[0] >> (2 * sg)) & 0x03030303u) << 4);
                cw.y = ((ql[1] >> (4 * (sg >> 1))) & 0x0F0F0F0Fu) | (((qh[1] >> (2 * sg)) & 0x03030303u) << 4);
                cw.z = ((ql[2] >> (4 * (sg >> 1))) & 0x0F0F0F0Fu) | (((qh[2] >> (2 * sg)) & 0x03030303u) << 4);
                cw.w = ((ql[3] >> (4 * (sg >> 1))) & 0x0F0F0F0Fu) | (((qh[3] >> (2 * sg)) & 0x03030303u) << 4);
                *(uint4*)(dec + rr * dstr + 32 * g + 16 * h16) = cw;
            }
            for (int t = dtid; t < k * rd * (F / 256); t += kDecThreads) {   // the 16 sub-block scales and d of a block
                const int rr = t / (F / 256), bb = t % (F / 256);
                const int boff = rr * d_row + 210 * bb;
                uint32_t sc[5];
                lds_words_a2<5>(slab_dn, boff + 192, sc);
                uint8_t* dr = dec + rr * dstr;
                *(uint4*)(dr + F + 16 * bb) = make_uint4(sc[0], sc[1], sc[2], sc[3]);
                ((float*)(dr + F + F / 16))[bb] = h2f((uint16_t)(sc[4] & 0xFFFFu));
            }
        }
        t1_lds_barrier();
        // the units no owner ran (none when the grid was resident): computed here, one at a time
        const int nh = s_misc[3];
        if (__builtin_expect(nh > 0, 0))
        for (int i = 0; i < nh; ++i) {
            const int q = s_help[1 + i];
            t1_help_unit<TG, H, F>(a.arena, a.blob, L.up_off, a.hx, q, k, tag, s_ids, ax, act_d(q / nu), s_gu);
        }
        constexpr int lpd = canon_lanes(F / UD::kUnit);
        const int c = lane & (lpd - 1);
        for (int t = tid / lpd; t < k * rd; t += kT1 / lpd) {
            const int e = t / rd, r = t - e * rd;
            float acc[1] = {0.0f};
            const Act ad = act_d(e);
            if constexpr (kDecode) {
                // 32-value group g: S = sc_2g (codes . h - 32 sum h, values 0..15) + sc_2g+1 (.. 16..31); acc =
                // fma(d_block d8_g, S, acc) - Unit<Q6_K>'s integers and order on the decoded codes
                const uint8_t* dr = dec + (e * rd + r) * dstr;
                const int8_t* scs = (const int8_t*)(dr + F);
                const float* dbk = (const float*)(dr + F + F / 16);
                for (int g = c; g < F / 32; g += lpd) {
                    const uint4 c0 = *(const uint4*)(dr + 32 * g), c1 = *(const uint4*)(dr + 32 * g + 16);
                    const uint4 x0 = *(const uint4*)(ad.q + 32 * g), x1 = *(const uint4*)(ad.q + 32 * g + 16);
                    int i0 = 0, i1 = 0;
                    i0 = sdot4((int)c0.x, (int)x0.x, i0);
                    i0 = sdot4((int)c0.y, (int)x0.y, i0);
                    i0 = sdot4((int)c0.z, (int)x0.z, i0);
                    i0 = sdot4((int)c0.w, (int)x0.w, i0);
                    i1 = sdot4((int)c1.x, (int)x1.x, i1);
                    i1 = sdot4((int)c1.y, (int)x1.y, i1);
                    i1 = sdot4((int)c1.z, (int)x1.z, i1);
                    i1 = sdot4((int)c1.w, (int)x1.w, i1);
                    i0 -= 32 * ad.us16[2 * g];
                    i1 -= 32 * ad.us16[2 * g + 1];
                    const int S = (int)scs[2 * g] * i0 + (int)scs[2 * g + 1] * i1;
                    acc[0] = __builtin_fmaf(dbk[g >> 3] * ad.d8[g], (float)S, acc[0]);
                }
            } else {
                const Act at[1] = {ad};
                for (int u = c; u < F / UD::kUnit; u += lpd)
                    UD::template apply<1>(slab_dn, (e * rd + r) * d_row, u, at, 1, acc);
            }
            const float sm = lane0_sum<lpd>(acc[0]);
            if (c == 0) s_po[t] = sm;
        }
        t1_lds_barrier();
        if (combiner) {
            const int r = tid;
            const int64_t col = (int64_t)j_dn * rd + r;
            float sum = 0.0f;
            for (int e = 0; e < k; ++e) {
                const float prod = s_po[e * rd + r] * s_w[e];
                sum = e == 0 ? prod : sum + prod;
            }
            if (a.shared) {   // the shared expert's row, once, after the routed ones (times its gate's sigmoid)
                float sv = c_sh;
                if (a.shared_gate) sv = sv * (1.0f / (1.0f + expf(-c_gate)));
                sum = sum + sv;
            }
            a.out[col] = c_res + sum;
        }
    } else if (spec_wave) {
        t1_vm_drain();
    }
    t1_done(a);
}

// ---------------------------------------------------------------- host side

namespace {

template <int TG, int TD, int H, int F, int RD>
const void* t1_pick(int n_expert) {
    return n_expert <= 64    ? (const void*)moe_decode_t1_kernel<TG, TD, 1, H, F, RD>
         : n_expert <= 128   ? (const void*)moe_decode_t1_kernel<TG, TD, 2, H, F, RD>
         : n_expert <= 256   ? (const void*)moe_decode_t1_kernel<TG, TD, 4, H, F, RD>
                             : nullptr;
}

// the instances: config 2's layer (Q4_K gate/up, Q6_K down, hidden 2048, F 768), the same shape with Q4_K down rows,
// and config 1's (Q8_0, 1024, 512), with as many down rows a unit as a 256-CU grid of one work-group a CU needs
struct T1Instance {
    int gu, d, H, F, rd;
    const void* (*pick)(int);
};
const T1Instance kT1Instances[] = {
    {kQ4_K, kQ6_K, 2048, 768, 8, t1_pick<kQ4_K, kQ6_K, 2048, 768, 8>},
    {kQ4_K, kQ4_K, 2048, 768, 8, t1_pick<kQ4_K, kQ4_K, 2048, 768, 8>},   // the same shape quantized all Q4_K
    {kQ8_0, kQ8_0, 1024, 512, 4, t1_pick<kQ8_0, kQ8_0, 1024, 512, 4>},
};

struct T1Shape {   // per device and kernel: the attribute set and the resident work-groups
    int dev;
    const void* kern;
    int lds, grid_max;
};
std::mutex g_t1_mu;
std::vector<T1Shape> g_t1_shapes;

hipError_t t1_resident(const void* kern, int lds, int* grid_max) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_t1_mu);
    for (const T1Shape& s : g_t1_shapes)
        if (s.dev == dev && s.kern == kern && s.lds == lds) {
            *grid_max = s.grid_max;
            return hipSuccess;
        }
    if (lds > 65536 && (e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds)) != hipSuccess)
        return e;
    int cus = 0, occ = 0;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, kT1, lds)) != hipSuccess) return e;
    if (occ < 1) return hipErrorInvalidConfiguration;
    *grid_max = cus * occ;
    g_t1_shapes.push_back(T1Shape{dev, kern, lds, *grid_max});
    return hipSuccess;
}

}  // namespace

hipError_t launch_decode_t1(const FusedArgs& a0, hipStream_t s, bool* used) {
    *used = false;
    const ExpertLayout& L = a0.L;
    const int H = (int)L.n_embd, F = (int)L.n_ff, k = a0.k;
    if (a0.n_tok != 1 || k > kT1MaxK || a0.pre_ids || a0.sig_group > 0 || mixed_gu(L))
        return hipSuccess;   // (softmax top-k only; one gate/up type)
    const T1Instance* inst = nullptr;
    for (const T1Instance& i : kT1Instances)
        if (i.gu == L.gu_type && i.d == L.d_type && i.H == H && i.F == F) inst = &i;
    if (!inst) return hipSuccess;
    const void* kern = inst->pick(a0.n_expert);
    if (!kern) return hipSuccess;
    const int qs = L.gu_type == kQ4_K ? t1_act_qs<kQ4_K>() : t1_act_qs<kQ8_0>();
    const int lds = t1_lds(k, H, F, (int)L.gu_row, (int)L.d_row, inst->rd, qs, L.d_type == kQ6_K).total;
    if (lds > 160 * 1024) return hipSuccess;
    int grid = 0;
    hipError_t e = t1_resident(kern, lds, &grid);
    if (e != hipSuccess) return e;
    const int nu = F / 32, nj = H / inst->rd;
    // a work-group a unit, the grid resident at once when nothing else runs (the kernel stays correct when it is not:
    // waiters compute units whose owners have not started), and a mark word a gate/up unit
    if (nj > grid || k * nu > grid || k * nu > kMarkWords) return hipSuccess;
    FusedArgs a = a0;
    a.rd = inst->rd;
    a.nu = nu;
    a.nj = nj;
    const int launch = nj > k * nu ? nj : k * nu;
    void* args[] = {(void*)&a};
    *used = true;
    return hipLaunchKernel(kern, dim3(launch), dim3(kT1), args, lds, s);
}

}  // namespace xs
