// xestrata-win_amd/csrc/decode_fused.hip - the whole decode MoE layer in one persistent launch.
//
// The reference runs a decode layer's MoE as a chain of launches with a host round trip (router_top10, the host or
// resident plan, quantize_q8_1_rows, native_expert_grouped's gate/up, SwiGLU and down launches, and
// native_moe_combine_multi + add_inplace: src/core/plain_model.cpp:951-988, src/core/moe_window.cpp:183-250).  At
// decode sizes every launch costs more than its work (a token's 8 experts are 24.5 MB of config-2 weights, 3 us of
// HBM time), so here one kernel does all of it, on the same arithmetic, bit for bit (xs_route.h, xs_units.h):
//
//   1. every work-group routes the tokens itself (softmax top-k, the plan, in LDS): no grid-wide wait before the
//      weights can be fetched;
//   2. gate/up units (a group, an h-slab of rh SwiGLU outputs = rh gate rows + rh up rows): the work-group fetches the
//      unit's rows and, with them, the rows of its first down unit, all in flight at once; quantizes its entries'
//      tokens to q8_1 in LDS; computes the rows; writes h = SwiGLU(gate, up) as tagged words;
//   3. down units (a group, a slab of rd down rows): gather the entries' h, polling each word until it carries this
//      call's tag, quantize it per 32 values in LDS, compute the rows into tagged `parts` words (routing order);
//   4. combines (a token, a down slab), after the work-group's down units: poll the slab's columns of the token's k
//      parts, add them in rank order, then a shared expert's row when given, add the residual
//      (native_moe_combine_multi + add_inplace).
// Waits only point backwards (down units on gate/up units, combines on down units, and a work-group finishes its
// gate/up units before its down units and those before its combines), every work-group of the grid is resident at
// once, and every wait is bounded: a wait past the bound sets the error word and moves on.
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_route.h"
#include "xs_units.h"

#include <mutex>
#include <vector>

namespace xs {

constexpr int kFT = 256;          // threads a work-group
// threads a work-group of the pipelined 4..16-token instance: its LDS (token table, two slabs) holds one work-group a
// CU, and with 256 threads that is one wave a SIMD, whose LDS and ALU latencies nothing hides; 512 give a down slab's
// rows a thread each (64 rows x 8 canonical lanes) and route two tokens a wave instead of four
constexpr int kFTPiped = 512;
__host__ __device__ constexpr int fused_threads(int ne, int mode) { return ne == 4 && mode == 1 ? kFTPiped : kFT; }
constexpr int kFMaxN = 256;       // routed entries (tokens x k) a call
constexpr int kLoadWaves = 4;     // the 256-thread instances: all four waves issue the global loads, wave 3 also every
                                  // tagged store (config 5 T=1 99.2-100.3 -> 98.2-98.3 us against three load waves,
                                  // config 4's stack unchanged); the pipelined instance: FusedArgs::load_waves, wave 7
                                  // the stores

struct FusedLds {                 // byte offsets in the dynamic LDS
    int ids, w, excl, wave, first, gexp, start, dst, tok, misc, gu, po, slab_gu, slab_dn, act_g, act_d, total;
};

__host__ __device__ inline int up16(int v) { return (v + 15) & ~15; }
// one entry's LDS activation of n values: int8 values | n / 32 fp32 scales | n / 16 int sums of 16
__host__ __device__ inline int act_stride(int n) { return up16(n + n / 8 + n / 4); }
// a gate/up activation (n a multiple of 256): the same with kGuPad bytes after each 256 int8 values (Unit's PAD)
constexpr int kGuPad = 16;
__host__ __device__ inline int act_q_bytes_g(int n) { return n + n / 256 * kGuPad; }
__host__ __device__ inline int act_stride_g(int n) { return up16(act_q_bytes_g(n) + n / 8 + n / 4); }

// ttab: tokens of the LDS activation table of the pipelined gate/up path (0: none; it then also has no second slab);
// alias: the down slab over the gate/up slab(s) - a work-group's down units follow all of its gate/up units, so the two
// are never live at once unless the first down rows are fetched early (which alias turns off)
template <int NE>
__host__ __device__ inline FusedLds fused_lds(int n_expert, int H, int F, int rh, int slab_gu, int slab_dn, int ttab,
                                              int alias) {
    FusedLds o;
    int at = 0;
    o.ids = at; at += up16(kFMaxN * 4);
    o.w = at; at += up16(kFMaxN * 4);
    o.excl = at; at += up16(kFMaxN * 4);
    o.wave = at; at += up16(64 * 4);
    o.first = at; at += up16(n_expert * 4);
    o.gexp = at; at += up16(kFMaxN * 4);
    o.start = at; at += up16((kFMaxN + 1) * 4);
    o.dst = at; at += up16(kFMaxN * 4);
    o.tok = at; at += up16(kFMaxN * 4);
    o.misc = at; at += up16(96 * 4);
    o.gu = at; at += up16(NE * 2 * rh * 4);
    o.po = at; at += up16(NE * 64 * 4);
    o.slab_gu = at; at += up16(slab_gu);
    if (ttab > 0) at += up16(slab_gu);   // a second gate/up slab: a unit is fetched while one computes
    if (alias) {
        o.slab_dn = o.slab_gu;
        if (at < o.slab_gu + up16(slab_dn)) at = o.slab_gu + up16(slab_dn);
    } else {
        o.slab_dn = at; at += up16(slab_dn);
    }
    o.act_g = at; at += (ttab > NE ? ttab : NE) * act_stride_g(H);   // the passes' activations, or the token table
    o.act_d = at; at += NE * act_stride(F);
    o.total = at;
    return o;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// q8_1 of values 8j .. 8j + 7 of one row (one scale a 256: 32 neighbouring lanes) straight into an LDS activation
// (int8 values, fp32 scale, sums of 16): the values quantize_q8_1_rows writes (q8_1_256_lane), as the grouped
// kernels read them back
__device__ __forceinline__ void q8_1_256_store(const float (&v)[8], int j, int8_t* q, float* d8, int* us16);
__device__ __forceinline__ void q8_1_256_to_act(const float* __restrict__ x, int j, int8_t* q, float* d8, int* us16) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = x[8 * j + i];
    q8_1_256_store(v, j, q, d8, us16);
}
// the same from values already loaded (values 8j .. 8j + 7; 32 neighbouring lanes hold a 256-value block)
__device__ __forceinline__ void q8_1_256_store(const float (&v)[8], int j, int8_t* q, float* d8, int* us16) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(v[i]));
    const float amax = group_max32(a);
    const float d = q8_scale(amax), id = q8_inv(d);
    uint32_t w0 = 0, w1 = 0;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q0 = q8_value(v[i], id), q1 = q8_value(v[4 + i], id);
        w0 |= (uint32_t)(uint8_t)q0 << (8 * i);
        w1 |= (uint32_t)(uint8_t)q1 << (8 * i);
        s += q0 + q1;
    }
    *(uint2*)(q + 8 * j + kGuPad * (j >> 5)) = make_uint2(w0, w1);   // (a gate/up activation: padded blocks)
    const int s16 = s + dpp_i<kDppXor1>(s);
    if ((j & 1) == 0) us16[j >> 1] = s16;
    if ((j & 3) == 0) d8[j >> 2] = h2f(f2h(d));
}

// Hand-over between work-groups without cache maintenance.  A release or acquire fence at device scope writes back or
// invalidates the whole L2 of the XCD (eight L2s are not coherent with each other for ordinary accesses), and with
// hundreds of work-groups those serialise into tens of microseconds; a producer that waits for its stores to be
// acknowledged before raising a flag waits behind the HBM write queue, which the weight stream starves.  So a value
// handed over travels in a 64-bit word with the call's tag in its upper half, written and read with device-scope
// relaxed atomics (coherent across XCDs by themselves: write-through stores, loads that refetch), and the reader
// polls the words it needs until every one carries the tag.  Tags come from a call counter in the workspace that
// every call advances by one epoch (done_call), so no word needs resetting and a stale word never matches.
__device__ __forceinline__ void st_tag(unsigned long long* p, float v, unsigned int tag) {
    __hip_atomic_store(p, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_tag(const unsigned long long* p) {
    return __hip_atomic_load((unsigned long long*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_ok(unsigned long long w, unsigned int tag) { return (unsigned int)(w >> 32) == tag; }
__device__ __forceinline__ float tag_val(unsigned long long w) { return __uint_as_float((unsigned int)w); }
__device__ __forceinline__ int add_dev(int32_t* p, int v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every vector memory access of a wave counts on one in-order counter (vmcnt): a wave that waits for a load also waits
// for the acknowledgement of every store it issued before, and stores are acknowledged late while the weight stream
// fills the memory queues.  So the waves that load never store a hand-over word: waves 0..2 fetch (weights by DMA,
// activations, polls), wave 3 writes h and parts from LDS.
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// (vm_wait_le: xs_device.h)

// A work-group barrier for LDS hand-overs.  __syncthreads() is also a work-group release, which makes every wave wait
// for all of its LDS DMA in flight (vmcnt(0)) - the next unit's rows fetched ahead on purpose included.  Where a wave
// needs DMA data it waits for it itself (vm_drain, vm_wait_le) before the barrier; LDS reads and writes are complete at
// lgkmcnt(0).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// n16 16-byte chunks to LDS dst[0 .. n16) by one wave's DMA: the store wave's fetch of the first down slab, issued
// once the gate/up slab is in (so it does not compete with it), complete at the store wave's vm_drain()
template <typename Src>
__device__ __forceinline__ void dma_wave_to_lds(uint8_t* dst, int n16, Src src) {
    const int lane = threadIdx.x & 63;
    for (int base = 0; base < n16; base += 64) {
        const int i = base + lane;
        if (i < n16)
            __builtin_amdgcn_global_load_lds(src(i), (__attribute__((address_space(3))) void*)(dst + 16 * base), 16, 0,
                                             2 /* nt */);
    }
}

// n16 16-byte chunks to LDS dst[0 .. n16) by DMA (global_load_lds_dwordx4: a wave's instruction fills 64 consecutive
// chunks at a wave-uniform LDS address), chunk i from src(i); issued by the lt / 64 load waves, complete at their
// vm_drain()
template <typename Src>
__device__ __forceinline__ void dma_to_lds(uint8_t* dst, int n16, Src src, int lt) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int base = 64 * wave; base < n16; base += lt) {
        const int i = base + lane;
        if (i < n16)
            __builtin_amdgcn_global_load_lds(src(i), (__attribute__((address_space(3))) void*)(dst + 16 * base), 16, 0,
                                             2 /* nt */);
    }
}

// N tagged words from p into v, polled until all carry the tag or the bound passes (then false, values undefined)
template <int N>
__device__ __forceinline__ bool gather_tagged(const unsigned long long* p, int n, unsigned int tag, long long ticks,
                                              float (&v)[N]) {
    if (ticks <= 0) return false;   // the host forces every wait to expire at once (a test of the error path)
    long long t0 = 0;
    for (int it = 0;; ++it) {
        unsigned long long w[N];
#pragma unroll
        for (int q = 0; q < N; ++q)
            if (q < n) w[q] = ld_tag(p + q);
        bool ok = true;
#pragma unroll
        for (int q = 0; q < N; ++q)
            if (q < n) {
                ok = ok && tag_ok(w[q], tag);
                v[q] = tag_val(w[q]);
            }
        if (ok) return true;
        if (it == 0) t0 = wall_clock64();
        else if (wall_clock64() - t0 > ticks) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

// the row-dot lane sum for a run-time lane count (lane 0 of each group gets it)
// f(EntriesC<M>()) with M = m, 1 <= m <= NE: a pass's entry count as a compile-time constant, so that the units' per-
// entry branches fold away and their LDS reads go out together (with the count at run time every entry's reads waited
// behind the branch before them)
template <int N>
struct EntriesC {
    static constexpr int value = N;
};
template <int NE, typename Fn>
__device__ __forceinline__ void with_entries(int m, Fn&& f) {
    if constexpr (NE >= 4) {
        if (m >= 4) return f(EntriesC<4>());
        if (m == 3) return f(EntriesC<3>());
    }
    if constexpr (NE >= 2)
        if (m == 2) return f(EntriesC<2>());
    f(EntriesC<1>());
}

__device__ __forceinline__ float lanes_sum(float v, int l) {
    return l == 8 ? lane0_sum<8>(v) : l == 4 ? lane0_sum<4>(v) : l == 2 ? lane0_sum<2>(v) : v;
}

// The work-group is done with the call: it adds its share of 2^20 to one of 16 64-bit call counters (the shares of a
// grid sum to 2^20 whatever its size; 16 counters, 128 bytes apart, keep the device atomics on one address few), and
// does not wait for the result.  The next call's epoch is (the counters' sum) >> 20: the kernel's end makes every
// addition visible to the next launch, and no work-group has to learn it was the last (that took three dependent
// device atomics at the end of every call).
constexpr int kCounters = 16, kCounterStride = 32;   // counters, ints apart
__device__ __forceinline__ void done_call(const FusedArgs& a, unsigned int) {
    if (threadIdx.x != 0) return;
    const unsigned int G = gridDim.x, b = blockIdx.x;
    const unsigned long long share = (1ull << 20) / G + (b < (1u << 20) % G ? 1ull : 0ull);
    __hip_atomic_fetch_add((unsigned long long*)(a.sync + kCounterStride * (b % kCounters)), share, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
// the epoch: lane i of a wave loads counter i (issued early, its latency behind the routing), and the wave's sum
// gives it (on every lane) once the routing is done
__device__ __forceinline__ unsigned long long load_counter(const FusedArgs& a) {
    const int lane = threadIdx.x & 63;
    return lane < kCounters ? __hip_atomic_load((unsigned long long*)(a.sync + kCounterStride * lane), __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : 0ull;
}
// The call's tag from its counters (lanes 0..15, row 0, summed by DPP, read from lane 0): the epoch (the sum >> 20, the
// calls before this one) mod 2^32 - 1, plus one.  Consecutive calls get different tags and no tag is 0, the value of a
// word that was never written (a zeroed workspace), so a poller never takes an unwritten word for a stored one.
__device__ __forceinline__ unsigned int call_tag(unsigned long long c) {
    static_assert(kCounters == 16, "one 16-lane row of counters");
    c += dpp_u64<kDppXor1, 0xF>(c);
    c += dpp_u64<kDppXor2, 0xF>(c);
    c += dpp_u64<kDppRor4, 0xF>(c);
    c += dpp_u64<kDppRor8, 0xF>(c);
    const unsigned int lo = __builtin_amdgcn_readlane((int)c, 0), hi = __builtin_amdgcn_readlane((int)(c >> 32), 0);
    const unsigned long long epoch = (((unsigned long long)hi << 32) | lo) >> 20;
    return (unsigned int)(epoch % 0xFFFFFFFFull) + 1u;
}

template <int TG, int TD>
constexpr bool kFusedSigmoid = TG == kQ4_K && TD == kQ4_K;
bool fused_sigmoid_layout(int gu_type, int d_type) { return gu_type == kQ4_K && d_type == kQ4_K; }

// SIG: the instance carries the group-limited sigmoid router's stage (only the Q4_K pair's instances: code an instance
// never runs still takes instruction-cache room - config 4's one-token layer 40.5 -> 41.3 us with it)
// after_loads() runs once the wave's first logits loads are out (loads issued there queue behind them, so the routing
// waits for its own loads only)
template <int PER, bool SIG, int NT, typename Fn>
__device__ __forceinline__ void route_tokens_wave(const FusedArgs& a, int T, int* s_ids, float* s_w,
                                                  unsigned long long& ctr, Fn&& after_loads) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, E = a.n_expert, k = a.k;
    if (a.pre_ids) {   // routed already (another router): the tokens' ids and weights as given
        ctr = load_counter(a);
        after_loads();
        for (int t = wave; t < T; t += NT / 64)
            if (lane < k) {
                s_ids[t * k + lane] = a.pre_ids[t * k + lane];
                s_w[t * k + lane] = a.pre_w[t * k + lane];
            }
        return;
    }
    if (SIG && a.sig_group > 0) {   // the group-limited sigmoid router, a wave a token
        ctr = load_counter(a);
        after_loads();
        for (int t = wave; t < T; t += NT / 64) {
            int id;
            float w;
            route_grouped_sigmoid_wave<PER>(a.logits + (int64_t)t * E, a.sig_bias, E, a.sig_group, a.sig_topk_group, k,
                                            a.sig_scale, id, w);
            if (lane < k) {
                s_ids[t * k + lane] = id;
                s_w[t * k + lane] = w;
            }
        }
        return;
    }
    float lv[PER], ln[PER];
    if (wave < T) load_logits_wave<PER>(a.logits + (int64_t)wave * E, E, lv);
    ctr = load_counter(a);
    after_loads();
    for (int t = wave; t < T; t += NT / 64) {
        // the wave's next token's logits are in flight while this one routes
        const int tn = t + NT / 64;
        if (tn < T) load_logits_wave<PER>(a.logits + (int64_t)tn * E, E, ln);
        if (lane < k) {   // ranks a NaN row leaves unwritten stay invalid
            s_ids[t * k + lane] = -1;
            s_w[t * k + lane] = 0.0f;
        }
        route_topk_wave_lv<PER>(lv, E, k, s_ids + t * k, s_w + t * k);
        if (tn < T)
#pragma unroll
            for (int i = 0; i < PER; ++i) lv[i] = ln[i];
    }
}

// NE = 1 is launched for one token only (the plan's ne: 1 token -> 1, 2-3 -> 2, 4+ -> 4), so T = 1 there is a
// constant and the multi-token planning and the pipelined gate/up path fold away; MODE 1 is, for one token, the direct
// form (no slabs) and, for 4+ tokens, the pipelined gate/up path (its token table in use), each without the other
// path's code; MODE 0 otherwise.  Each instance carries only its own paths: the kernel's code is large, and what an
// instance does not run still costs instruction-cache room.
template <int TG, int TD, int NE, int MODE, int PER>
__global__ __launch_bounds__(fused_threads(NE, MODE)) void moe_decode_fused_kernel(FusedArgs a) {
    constexpr bool DIRECT = NE == 1 && MODE == 1;
    constexpr int NT = fused_threads(NE, MODE);
    constexpr bool PIPED = NE == 4 && MODE == 1;   // the pipelined 4..16-token path (token table, two slabs)
    extern __shared__ __align__(16) uint8_t lds[];
    using UG = Unit<TG, true, kGuPad>;
    using UD = Unit<TD, false>;
    const ExpertLayout& L = a.L;
    const int H = (int)L.n_embd, F = (int)L.n_ff, k = a.k, T = NE == 1 ? 1 : a.n_tok, n = T * k, E = a.n_expert;
    const int rh = a.rh, rd = a.rd, nu = a.nu, nj = a.nj;
    const FusedLds o = fused_lds<NE>(E, H, F, rh, a.slab_gu_bytes, a.slab_dn_bytes, a.ttab, a.slab_alias);
    int* s_ids = (int*)(lds + o.ids);
    float* s_w = (float*)(lds + o.w);
    int* s_excl = (int*)(lds + o.excl);
    int* s_first = (int*)(lds + o.first);
    int* s_gexp = (int*)(lds + o.gexp);
    int* s_start = (int*)(lds + o.start);
    int* s_dst = (int*)(lds + o.dst);
    int* s_tok = (int*)(lds + o.tok);
    int* s_misc = (int*)(lds + o.misc);   // [0] groups (-1: bad routing), [3] the epoch
    float* s_gu = (float*)(lds + o.gu);
    uint8_t* slab_gu = lds + o.slab_gu;
    uint8_t* slab_dn = lds + o.slab_dn;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    Act actg[NE], actd[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
        int8_t* qg = (int8_t*)(lds + o.act_g) + e * act_stride_g(H);
        actg[e] = Act{qg, (const float*)(qg + act_q_bytes_g(H)), (const int*)(qg + act_q_bytes_g(H) + H / 8)};
        int8_t* qd = (int8_t*)(lds + o.act_d) + e * act_stride(F);
        actd[e] = Act{qd, (const float*)(qd + F), (const int*)(qd + F + F / 8)};
    }

    // ---- 1. routing, in every work-group (router.cpp:59-308 and verify_kernels.cpp:819-890's order, in LDS): a wave a
    // token, waves t, t + 4, ...  The logits loads go out first; the call counters' loads follow, summed only after
    // the routing, so their latency hides behind it.  With one token, waves 1..3 meanwhile quantize its activation
    // (the gate/up units' q8_1 input, one scale a 256) into LDS, and wave 0 plans the call itself.
    unsigned long long ctr = 0;
    const bool x_early = T == 1 && a.ttab == 0;
    if (x_early && wave > 0) {
        int8_t* q = (int8_t*)(lds + o.act_g);
        // every chunk of the thread loaded first, then quantized: the loads share one round trip instead of one a
        // chunk (a chunk's quantization waits for its 32-lane block's amax, so a load-then-quantize loop exposes each
        // load); up to kXEarly chunks a thread, past that the loop
        constexpr int kXEarly = 8;
        const int step = NT - 64;
        if (H / 8 <= kXEarly * step) {
            float v[kXEarly][8];
#pragma unroll
            for (int it = 0; it < kXEarly; ++it) {
                const int j8 = tid - 64 + it * step;
                if (j8 < H / 8)
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[it][i] = a.x[8 * j8 + i];
            }
#pragma unroll
            for (int it = 0; it < kXEarly; ++it) {
                const int j8 = tid - 64 + it * step;
                if (j8 < H / 8)
                    q8_1_256_store(v[it], j8, q, (float*)(q + act_q_bytes_g(H)), (int*)(q + act_q_bytes_g(H) + H / 8));
            }
        } else {
            for (int j8 = tid - 64; j8 < H / 8; j8 += step)
                q8_1_256_to_act(a.x, j8, q, (float*)(q + act_q_bytes_g(H)), (int*)(q + act_q_bytes_g(H) + H / 8));
        }
    }
    // the pipelined path's token table: its first 8 chunks a thread (chunk i = 8 values of token i / (H / 8)) are
    // loaded beside the routing's logits (x does not depend on it); quantized into the table after the plan
    constexpr int kXPre = PIPED ? 8 : 1;
    float xv[kXPre][8];
    auto load_x = [&]() {
        if constexpr (PIPED) {
            const int nch = H / 8, total = T * nch;
#pragma unroll
            for (int b = 0; b < kXPre; ++b) {
                const int i = b * NT + tid;
                if (i < total) {
                    const int t = i / nch, j8 = i - t * nch;
                    const float4* xr = (const float4*)(a.x + (int64_t)t * H + 8 * j8);
                    const float4 u0 = xr[0], u1 = xr[1];
                    xv[b][0] = u0.x; xv[b][1] = u0.y; xv[b][2] = u0.z; xv[b][3] = u0.w;
                    xv[b][4] = u1.x; xv[b][5] = u1.y; xv[b][6] = u1.z; xv[b][7] = u1.w;
                }
            }
        }
    };
    route_tokens_wave<PER, kFusedSigmoid<TG, TD>, NT>(a, T, s_ids, s_w, ctr, load_x);   // PER = the experts a lane (64 PER >= E, chosen by the host)
    if (wave == 0) {
        const unsigned int ctag = call_tag(ctr);
        if (lane == 0) s_misc[3] = (int)ctag;
        if (T == 1) {   // one token: its k experts are distinct, each a group of one entry, in rank order
            const int ex = lane < k ? s_ids[lane] : 0;   // this lane's own rank (route_topk_wave_lv writes lane < k)
            if (__ballot(lane < k && (ex < 0 || ex >= E))) {
                if (lane == 0) s_misc[0] = -1;
            } else {
                if (lane < k) {
                    s_gexp[lane] = ex;
                    s_start[lane] = lane;
                    s_dst[lane] = lane;
                    s_tok[lane] = 0;
                }
                if (lane == 0) {
                    s_start[k] = k;
                    s_misc[0] = k;
                }
            }
        }
    }
    __syncthreads();
    // the plan: groups = distinct experts in order of first occurrence, a group's entries ascending (one token: planned
    // above).  Wave 0 numbers the groups (plan_groups_wave, xs_route.h: the expert ids' LDS group numbers, 16 bits,
    // over s_first; the entries' group | place over s_excl; the group sizes, then starts, in s_start); then every
    // thread places its entry.
    if (T > 1) {
        const int ex = tid < n ? s_ids[tid] : -1;
        if (__syncthreads_or(tid < n && (ex < 0 || ex >= E))) {
            if (tid == 0) s_misc[0] = -1;
        } else {
            const PlanLds pl{(int16_t*)s_first, s_excl, s_start, s_gexp};
            if (wave == 0) {
                const int groups = plan_groups_wave(s_ids, n, E, pl);
                if (lane == 0) s_misc[0] = groups;
            }
            __syncthreads();
            if (tid < n) {
                const int e = s_excl[tid];
                const int slot = s_start[e & 0xffff] + (e >> 16);
                s_dst[slot] = tid;
                s_tok[slot] = tid / k;
            }
        }
    }
    if (T > 1) __syncthreads();
    const unsigned int tag = (unsigned int)s_misc[3];
    if (s_misc[0] < 0) {   // a rank left unwritten (NaN logits): no output this call
        if (tid == 0) atomicOr(a.err, 4);
        done_call(a, tag);
        return;
    }
    if (blockIdx.x == 0 && tid < n) {
        a.ids[tid] = s_ids[tid];
        a.weights[tid] = s_w[tid];
    }
    const int ng = s_misc[0];
    const int wg = blockIdx.x;
    const int n_gu = ng * nu, n_dn = ng * nj;
    const int lpr_g = canon_lanes(H / UG::kUnit), lpr_d = canon_lanes(F / UD::kUnit);

    // ---- 2. gate/up units
    const int n16a = rh * (int)L.gu_row / 16, n16d = rd * (int)L.d_row / 16;
    float* s_po = (float*)(lds + o.po);
    // the waves that issue every global load.  The issuing waves stall while the memory queues are full, so the
    // pipelined instance issues from more of them: from 6 where one work-group fills a CU (config 2 at 16 tokens:
    // 130.4 us with 3, 127.5 with 4, 124.8 with 5, 123.0 with 6), from 4 where two do (8 tokens: 75.5 with 3, 74.4 with
    // 4, 74.9 with 5, 76.2 with 6; 4 tokens: 43.6, 43.3, 43.2, 44.1) - same box, alternating builds, bit for bit
    const int LW = NT > 256 ? a.load_waves : kLoadWaves, LT = 64 * LW;
    const bool loader = wave < LW;
    // the one wave that writes tagged words (with 256 threads also a load wave); with 512 threads, wave 7,
    // which has no rows of a gate/up slab (32 rows x 8 lanes fill waves 0..3) and issues no loads, so its SwiGLU and
    // stores overlap them
    const bool storer = wave == (NT > 256 ? 7 : kLoadWaves - 1);
    // with at most one gate/up unit a work-group, the store wave fetches the work-group's first down rows once the
    // gate/up slab is in: they then land while the gate/up products run and h travels
    const bool piped = NE == 4 && MODE == 1;   // the pipelined gate/up path below (4..16 tokens, the table in use)
    // down units: with one token and more units than work-groups, a work-group takes a run of consecutive ones
    // (mostly one expert's), so its entry's h is gathered and quantized once for the run rather than once a unit; so
    // too on the pipelined path below 8 tokens when most groups hold one entry (config 2 at 4 tokens, uniform
    // routing: 62.4 -> 60.3 us a layer).  Otherwise a unit's cost is its group's entry count and runs load the
    // work-groups unevenly (16 tokens: 170 -> 178 us a call; config 3's Zipf-routed verify: 55.9 -> 58.8 us a layer),
    // so the units go round the work-groups.
    const int G = (int)gridDim.x;
    const bool runs = (T == 1 || (PIPED && T < 8 && 4 * ng >= 3 * n)) && n_dn > G;
    const int dq = n_dn / G, dr = n_dn - dq * G;
    // Round robin: when the gate/up units do not divide evenly, the work-groups that took one more of them (the first
    // n_gu % G) take the down units from the other end (work-group wg starts at G - 1 - wg), so they are the ones with
    // one down unit fewer: config 3's Zipf verify 51.2 -> 50.2 us, 8 tokens 83.0 -> 80.3, 16 tokens 133.7 -> 131.3.
    const int d_begin0 = runs ? wg * dq + min(wg, dr) : (n_gu % G != 0 ? G - 1 - wg : wg);
    const int d_end0 = runs ? d_begin0 + dq + (wg < dr ? 1 : 0) : n_dn;
    const int d_step0 = runs ? 1 : G;
    // The direct form with fewer gate/up units than work-groups (config 5's routed experts at one token: 512 units,
    // 1024 work-groups): no runs; the down units go round in the order the work-groups come free - those without a
    // gate/up unit, then the others (a CU's later work-groups finish their units last) - while the units come in
    // routing rank, the order in which the experts' h is complete.  In runs, work-groups still streaming gate/up rows
    // held down units whose h was long in: config 5 T=1 107.3 -> 105.1 us.  (A constant false elsewhere: config 4's
    // slab instance lost 3% to code that changed its register allocation though it never takes this path.)
    const bool by_free = DIRECT && n_gu < G;
    const int d_begin = by_free ? (wg >= n_gu ? wg - n_gu : G - n_gu + wg) : d_begin0;
    const int d_end = by_free ? n_dn : d_end0;
    const int d_step = by_free ? G : d_step0;
    const bool dn_early = !piped && !DIRECT && !a.slab_alias && n_gu <= G && wg < n_gu && d_begin < d_end;
    if (piped) {
        // 4..16 tokens, several units a work-group: every token's q8_1 activation once, into an LDS table, then the
        // units' slabs double-buffered - unit i + 1's DMA flies while unit i computes.  The load waves issue nothing
        // but those DMAs meanwhile, so waiting for unit i is vmcnt <= (unit i + 1's DMA instructions of the wave).
        int8_t* ttab = (int8_t*)(lds + o.act_g);
        uint8_t* slab2[2] = {slab_gu, slab_gu + up16(a.slab_gu_bytes)};
        const int per_wave = loader && 2 * n16a > 64 * wave ? (2 * n16a - 64 * wave + LT - 1) / LT : 0;
        auto dma_unit = [&](int u, uint8_t* dst) {
            const int g = u / nu, j = u - g * nu;
            const uint8_t* blob = a.arena + (size_t)s_gexp[g] * (size_t)a.blob;
            const uint8_t* srcg = blob + (size_t)j * rh * L.gu_row;
            const uint8_t* srcu = blob + L.up_off + (size_t)j * rh * L.gu_row;
            dma_to_lds(dst, 2 * n16a, [&](int i) {
                return (const void*)(i < n16a ? srcg + 16 * (size_t)i : srcu + 16 * (size_t)(i - n16a));
            }, LT);
        };
        // the first unit's DMA goes out before the table, so that its rows land while the table is built
        if (loader && wg < n_gu) dma_unit(wg, slab2[0]);
        // the table: chunk i = (token, 8 values) of every token, four chunks a thread with their loads in flight at
        // once (a token at a time, every token's loads waited out a round trip of their own: ~1 us a token).  Chunks
        // come 32 to a 256-value block, and the token rows are multiples of 32 chunks, so each 32-lane group is whole.
        {
            const int nch = H / 8, total = T * nch;
#pragma unroll
            for (int b = 0; b < kXPre; ++b) {   // the chunks loaded at the kernel's start
                const int i = b * NT + tid;
                if (i < total) {
                    const int t = i / nch, j8 = i - t * nch;
                    int8_t* q = ttab + t * act_stride_g(H);
                    q8_1_256_store(xv[b], j8, q, (float*)(q + act_q_bytes_g(H)), (int*)(q + act_q_bytes_g(H) + H / 8));
                }
            }
            for (int i0 = kXPre * NT; i0 < total; i0 += 4 * NT) {
                float v[4][8];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int i = i0 + b * NT + tid;
                    if (i < total) {
                        const int t = i / nch, j8 = i - t * nch;
                        const float4* xr = (const float4*)(a.x + (int64_t)t * H + 8 * j8);
                        const float4 u0 = xr[0], u1 = xr[1];
                        v[b][0] = u0.x; v[b][1] = u0.y; v[b][2] = u0.z; v[b][3] = u0.w;
                        v[b][4] = u1.x; v[b][5] = u1.y; v[b][6] = u1.z; v[b][7] = u1.w;
                    }
                }
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int i = i0 + b * NT + tid;
                    if (i < total) {
                        const int t = i / nch, j8 = i - t * nch;
                        int8_t* q = ttab + t * act_stride_g(H);
                        q8_1_256_store(v[b], j8, q, (float*)(q + act_q_bytes_g(H)), (int*)(q + act_q_bytes_g(H) + H / 8));
                    }
                }
            }
        }
        // the store wave's last h value of a pass (one a lane), written once the next unit's slab is in: its SwiGLU
        // and store then run beside the next unit's products instead of before the next unit's first barrier
        float pg = 0.0f, pu = 0.0f;
        unsigned long long* pdst = nullptr;
        auto flush_h = [&]() {
            if (pdst) st_tag(pdst, canon_silu_mul(pg, pu), tag);
            pdst = nullptr;
        };
        int it = 0;
        for (int u1 = wg; u1 < n_gu; u1 += gridDim.x, ++it) {
            const int g = u1 / nu, j = u1 - g * nu, next = u1 + (int)gridDim.x;
            uint8_t* slab = slab2[it & 1];
            lds_barrier();   // the previous unit's readers of the other slab and of s_gu are done
            if (loader) {
                if (next < n_gu) {
                    dma_unit(next, slab2[(it + 1) & 1]);
                    vm_wait_le(per_wave);
                } else {
                    vm_drain();
                }
            }
            lds_barrier();   // this unit's slab is in
            if (storer) flush_h();
            const int e0 = s_start[g], e1 = s_start[g + 1];
            for (int p = e0; p < e1; p += NE) {
                const int m = min(NE, e1 - p);
                if (p > e0) lds_barrier();   // the previous pass's stores have read s_gu
                Act at[NE];
#pragma unroll
                for (int e = 0; e < NE; ++e) {
                    int8_t* q = ttab + (e < m ? s_tok[p + e] : 0) * act_stride_g(H);
                    at[e] = Act{q, (const float*)(q + act_q_bytes_g(H)), (const int*)(q + act_q_bytes_g(H) + H / 8)};
                }
                const int c = lane & (lpr_g - 1);
                with_entries<NE>(m, [&](auto mc) {
                    constexpr int M = decltype(mc)::value;
                    Act am[M];
#pragma unroll
                    for (int e = 0; e < M; ++e) am[e] = at[e];
                    for (int rr = tid / lpr_g; rr < 2 * rh; rr += NT / lpr_g) {
                        float acc[M];
#pragma unroll
                        for (int e = 0; e < M; ++e) acc[e] = 0.0f;
                        for (int u = c; u < H / UG::kUnit; u += lpr_g)
                            UG::template apply<M>(slab, rr * (int)L.gu_row, u, am, M, acc);
#pragma unroll
                        for (int e = 0; e < M; ++e) acc[e] = lanes_sum(acc[e], lpr_g);
                        if (c == 0) {
#pragma unroll
                            for (int e = 0; e < M; ++e) s_gu[e * 2 * rh + rr] = acc[e];
                        }
                    }
                });
                lds_barrier();
                if (storer) {
                    flush_h();   // (a group of more than NE entries: the previous pass's)
                    for (int i = lane; i < m * rh; i += 64) {
                        const int e = i / rh, r = i - e * rh;
                        unsigned long long* dst = a.hx + (int64_t)(p + e) * F + j * rh + r;
                        if (i + 64 < m * rh) {
                            st_tag(dst, canon_silu_mul(s_gu[e * 2 * rh + r], s_gu[e * 2 * rh + rh + r]), tag);
                        } else {
                            pg = s_gu[e * 2 * rh + r];
                            pu = s_gu[e * 2 * rh + rh + r];
                            pdst = dst;
                        }
                    }
                }
            }
        }
        if (storer) flush_h();
    } else
    for (int u1 = wg; u1 < n_gu; u1 += gridDim.x) {
        const int g = u1 / nu, j = u1 - g * nu;
        const uint8_t* blob = a.arena + (size_t)s_gexp[g] * (size_t)a.blob;
        const uint8_t* srcg = blob + (size_t)j * rh * L.gu_row;
        const uint8_t* srcu = blob + L.up_off + (size_t)j * rh * L.gu_row;
        __syncthreads();   // the previous unit's readers of the slab are done
        if (loader && !DIRECT)
            dma_to_lds(slab_gu, 2 * n16a, [&](int i) {
                return (const void*)(i < n16a ? srcg + 16 * (size_t)i : srcu + 16 * (size_t)(i - n16a));
            }, LT);
        const int e0 = s_start[g], e1 = s_start[g + 1];
        for (int p = e0; p < e1; p += NE) {
            const int m = min(NE, e1 - p);
            if (p > e0) lds_barrier();   // the previous pass's readers of the activations are done
            if (loader) {
                for (int e = 0; e < (x_early ? 0 : m); ++e) {    // the entries' tokens to q8_1, one scale a 256
                    const float* xr = a.x + (int64_t)s_tok[p + e] * H;
                    int8_t* q = (int8_t*)(lds + o.act_g) + e * act_stride_g(H);
                    for (int j8 = tid; j8 < H / 8; j8 += LT)
                        q8_1_256_to_act(xr, j8, q, (float*)(q + act_q_bytes_g(H)), (int*)(q + act_q_bytes_g(H) + H / 8));
                }
                vm_drain();   // the slab and the activations have landed
            }
            __syncthreads();
            if (dn_early && storer && u1 == wg && p == e0) {
                const int gd = d_begin / nj, jd = d_begin - gd * nj;
                const uint8_t* srcd =
                    a.arena + (size_t)s_gexp[gd] * (size_t)a.blob + L.down_off + (size_t)jd * rd * L.d_row;
                dma_wave_to_lds(slab_dn, n16d, [&](int i) { return (const void*)(srcd + 16 * (size_t)i); });
            }
            const int c = lane & (lpr_g - 1);
            // the rows from the slab (LDS reads), or in the direct form from the blob (global reads): two loops, so
            // that each one's loads have a known address space
            auto gu_rows = [&](auto row_base) {
                for (int rr = tid / lpr_g; rr < 2 * rh; rr += NT / lpr_g) {
                    float acc[NE];
#pragma unroll
                    for (int e = 0; e < NE; ++e) acc[e] = 0.0f;
                    const uint8_t* rb = row_base(rr);
                    for (int u = c; u < H / UG::kUnit; u += lpr_g)
                        UG::template apply<NE>(rb, rr * (int)L.gu_row, u, actg, m, acc);
#pragma unroll
                    for (int e = 0; e < NE; ++e) acc[e] = lanes_sum(acc[e], lpr_g);
                    if (c == 0) {
#pragma unroll
                        for (int e = 0; e < NE; ++e)
                            if (e < m) s_gu[e * 2 * rh + rr] = acc[e];
                    }
                }
            };
            if (DIRECT)   // gate rows, then up rows
                gu_rows([&](int rr) { return rr < rh ? srcg : srcu - (size_t)rh * L.gu_row; });
            else
                gu_rows([&](int) { return (const uint8_t*)slab_gu; });
            lds_barrier();
            if (storer)
                for (int i = lane; i < m * rh; i += 64) {
                    const int e = i / rh, r = i - e * rh;
                    st_tag(a.hx + (int64_t)(p + e) * F + j * rh + r,
                           canon_silu_mul(s_gu[e * 2 * rh + r], s_gu[e * 2 * rh + rh + r]), tag);
                }
        }
    }

    // ---- 3. down units; the first one's rows are fetched once the gate/up rows are in (they go first)
    int prev_g = -1;
    for (int u2 = d_begin; u2 < d_end; u2 += d_step) {
        const int g = u2 / nj, j = u2 - g * nj;
        const uint8_t* srcd = a.arena + (size_t)s_gexp[g] * (size_t)a.blob + L.down_off + (size_t)j * rd * L.d_row;
        lds_barrier();   // the previous unit's readers of the slab are done
        const bool fetched = dn_early && u2 == d_begin;
        if (loader && !fetched && !DIRECT)
            dma_to_lds(slab_dn, n16d, [&](int i) { return (const void*)(srcd + 16 * (size_t)i); }, LT);
        const int e0 = s_start[g], e1 = s_start[g + 1];
        for (int p = e0; p < e1; p += NE) {
            const int m = min(NE, e1 - p);
            if (p > e0) __syncthreads();
            // h of the entries (polled until the gate/up units have written it) per 32 values to canonical q8_1
            // (iq_kernels.cpp:2118-2133): 8 values a lane, a block on 4 neighbouring lanes.  The previous unit's, when
            // it was the same group's single pass: act_d holds it still.
            const bool h_kept = g == prev_g && e1 - e0 <= NE;
            if (loader && h_kept) {
                vm_drain();   // the slab has landed
            } else if (loader) {
                const int c8n = F / 8;
                for (int i0 = 0; i0 < m * c8n; i0 += LT) {
                    const int i = i0 + tid;
                    const bool in = i < m * c8n;
                    const int e = in ? i / c8n : 0, c8 = in ? i - e * c8n : 0;
                    float v[8];
                    if (!in || !gather_tagged<8>(a.hx + (int64_t)(p + e) * F + 8 * c8, 8, tag, a.spin_ticks, v)) {
                        if (in) atomicOr(a.err, 2);
#pragma unroll
                        for (int q = 0; q < 8; ++q) v[q] = 0.0f;
                    }
                    float amax = 0.0f;
#pragma unroll
                    for (int q = 0; q < 8; ++q) amax = fmaxf(amax, fabsf(v[q]));
                    amax = fmaxf(amax, dpp_f<kDppXor1>(amax));
                    amax = fmaxf(amax, dpp_f<kDppXor2>(amax));
                    const float d = q8_scale(amax), id = q8_inv(d);
                    uint32_t w0 = 0, w1 = 0;
                    int sq = 0;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int q0 = q8_value(v[q], id), q1 = q8_value(v[4 + q], id);
                        w0 |= (uint32_t)(uint8_t)q0 << (8 * q);
                        w1 |= (uint32_t)(uint8_t)q1 << (8 * q);
                        sq += q0 + q1;
                    }
                    const int s16 = sq + dpp_i<kDppXor1>(sq);
                    if (in) {
                        int8_t* qd = (int8_t*)(lds + o.act_d) + e * act_stride(F);
                        *(uint2*)(qd + 8 * c8) = make_uint2(w0, w1);
                        if ((c8 & 1) == 0) ((int*)(qd + F + F / 8))[c8 >> 1] = s16;
                        if ((c8 & 3) == 0) ((float*)(qd + F))[c8 >> 2] = h2f(f2h(d));
                    }
                }
                vm_drain();   // the slab has landed
            } else if (fetched && p == e0) {
                vm_drain();   // the store wave's fetch of the slab has landed
            }
            __syncthreads();
            const int c = lane & (lpr_d - 1);
            auto dn_rows = [&](const uint8_t* rb) {   // (the slab or, direct, the blob: as above, two instances)
                with_entries<NE>(m, [&](auto mc) {
                    constexpr int M = decltype(mc)::value;
                    Act am[M];
#pragma unroll
                    for (int e = 0; e < M; ++e) am[e] = actd[e];
                    for (int rr = tid / lpr_d; rr < rd; rr += NT / lpr_d) {
                        float acc[M];
#pragma unroll
                        for (int e = 0; e < M; ++e) acc[e] = 0.0f;
                        for (int u = c; u < F / UD::kUnit; u += lpr_d)
                            UD::template apply<M>(rb, rr * (int)L.d_row, u, am, M, acc);
#pragma unroll
                        for (int e = 0; e < M; ++e) acc[e] = lanes_sum(acc[e], lpr_d);
                        if (c == 0) {
#pragma unroll
                            for (int e = 0; e < M; ++e) s_po[e * rd + rr] = acc[e];
                        }
                    }
                });
            };
            if (DIRECT) dn_rows(srcd);
            else dn_rows(slab_dn);
            __syncthreads();
            if (storer)
                for (int i = lane; i < m * rd; i += 64) {
                    const int e = i / rd, r = i - e * rd;
                    st_tag(a.px + (int64_t)s_dst[p + e] * H + j * rd + r, s_po[e * rd + r], tag);
                }
        }
        prev_g = g;
    }

    // ---- 4. combines: (token t, down slab j), the slab's columns of the token's k parts in rank order + residual
    // rd <= 64 threads a task (a column each), NT / rd tasks of a work-group at once (their polls overlap)
    const int tg = NT / rd;
    for (int c = wg + (tid / rd) * (int)gridDim.x; tid < tg * rd && c < T * nj; c += tg * (int)gridDim.x) {
        const int t = c / nj, j = c - t * nj;
        for (int r = tid % rd; r < rd; r += NT) {
            const int64_t col = (int64_t)j * rd + r;
            const unsigned long long* pp = a.px + (int64_t)t * k * H + col;
            const float* ww = s_w + t * k;
            // (in flight while the parts are polled; no residual: the combined row alone)
            const float res = a.residual ? a.residual[(int64_t)t * H + col] : 0.0f;
            // the shared expert's row and gate logit, also in flight while the parts are polled
            const float shv = a.shared ? a.shared[(int64_t)t * H + col] : 0.0f;
            const float shg = a.shared && a.shared_gate ? a.shared_gate[t] : 0.0f;
            float sum = 0.0f;
            bool good = true;
            for (int e0 = 0; e0 < k; e0 += 16) {   // 16 parts in flight at once
                float pv[16];
                unsigned long long w[16];
                const int ne = min(16, k - e0);
                long long t0 = 0;
                for (int it = 0;; ++it) {
                    bool ok = true;
#pragma unroll
                    for (int q = 0; q < 16; ++q)
                        if (q < ne) w[q] = ld_tag(pp + (int64_t)(e0 + q) * H);
#pragma unroll
                    for (int q = 0; q < 16; ++q)
                        if (q < ne) {
                            ok = ok && tag_ok(w[q], tag);
                            pv[q] = tag_val(w[q]);
                        }
                    if (a.spin_ticks <= 0) {   // every wait forced to expire at once (the host's test of the path)
                        good = false;
                        break;
                    }
                    if (ok) break;
                    if (it == 0) t0 = wall_clock64();
                    else if (wall_clock64() - t0 > a.spin_ticks) {
                        good = false;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    if (q < ne) {
                        const float prod = pv[q] * ww[e0 + q];
                        sum = e0 + q == 0 ? prod : sum + prod;
                    }
            }
            if (!good) atomicOr(a.err, 2);
            if (a.shared) {   // the shared expert's row, once, after the routed ones (times its gate's sigmoid)
                float sv = shv;
                if (a.shared_gate) sv = sv * (1.0f / (1.0f + expf(-shg)));
                sum = sum + sv;
            }
            a.out[(int64_t)t * H + col] = a.residual ? res + sum : sum;
        }
    }
    done_call(a, tag);
}

// ---------------------------------------------------------------- host side

// compute units of the current device (cached per device)
static int device_cus() {
    static std::mutex mu;
    static std::vector<std::pair<int, int>> seen;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& s : seen)
        if (s.first == dev) return s.second;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    seen.emplace_back(dev, cus);
    return cus;
}

bool fused_decode_plan(const ExpertLayout& L, int n_expert, int k, int n_tok, FusedPlan* P) {
    const int H = (int)L.n_embd, F = (int)L.n_ff, n = n_tok * k;
    if (n > kFMaxN || n_expert > 1024 || k > 64 || n_tok > 64 || mixed_gu(L)) return false;   // (one gate/up type)
    const bool pair = (L.gu_type == kQ4_K && L.d_type == kQ6_K) || (L.gu_type == kQ8_0 && L.d_type == kQ8_0) ||
                      (L.gu_type == kIQ4_XS && L.d_type == kIQ4_XS) || (L.gu_type == kQ4_K && L.d_type == kQ4_K);
    if (!pair || H % 256 || F % 32) return false;
    // h-slab rows: about 36 KB of gate + up rows, a multiple of 8 dividing n_ff (of 4 for one token, below)
    int rh = (int)((36864 / (2 * L.gu_row)) & ~7ll);
    if (rh < 8) rh = 8;
    while (rh > 8 && F % rh) rh -= 8;
    if (F % rh) return false;
    // 4-8 tokens: 8-row h-slabs and (below) a token table for the call's tokens, so that two 512-thread work-groups
    // fit a CU (~65 KB of LDS at 4 tokens, ~78 KB at 8; 16-row slabs and a 16-token table took ~135 KB, one a CU):
    // config 2 T=4 54.6 -> 46.3 us, config 3's Zipf verify 49.4 -> 43.1, T=8 79.3 -> 75.5 (bit for bit).  At 16
    // tokens the table alone is 47 KB: 4-row h-slabs and 16-row down slabs fit two a CU but took 207 against 130 us.
    if (n_tok >= 4 && n_tok <= 8 && rh > 8 && F % 8 == 0) rh = 8;
    // one token: its k groups' gate/up units as close to one a resident work-group (two a CU) as the slab allows -
    // smaller slabs spread the weight stream over more CUs, and each work-group then also fetches its down rows
    // while its gate/up products run
    if (n_tok == 1) {
        const int target = 2 * device_cus();
        for (int r = 4; r < rh; r += 4)
            if (F % r == 0 && (int64_t)k * (F / r) <= target) {
                rh = r;
                break;
            }
    }
    // down-slab rows: about 20 KB of down rows at 2-3 tokens; 40 KB for one token (config 4's IQ4_XS rows: 32 rows,
    // two down units a work-group of the grid: 46.6 -> 40.3 us a layer; 64 rows, one a work-group: 55.3 us) and from 4
    // tokens on (config 2 at 16 tokens: 198.2 -> 195.3 us; at 4 tokens, with two work-groups a CU: 46.2 -> 43.7 us,
    // config 3's Zipf verify 43.0 -> 40.6 - with one a CU the same slabs had cost the verify 59.7 -> 63.0; 16 rows at
    // 4 tokens 54.3 us, 32 rows at 8 tokens 75.5 -> 82.3)
    int rd = (int)(((n_tok == 1 || n_tok >= 4 ? 40960 : 20480) / L.d_row) & ~7ll);
    if (rd < 8) rd = 8;
    if (rd > 64) rd = 64;
    while (rd > 8 && H % rd) rd -= 8;
    if (H % rd) return false;
    // one token with at least as many gate/up units as two work-groups a CU (large experts: config 5's routed layer):
    // the direct form - a unit's rows fill the work-group's lanes (each row's canonical lanes, 256 in all), every lane
    // reads its blocks from HBM itself, and without slabs the LDS holds up to four work-groups a CU, whose loads hide
    // each other's latency
    // (only with at least 4 gate/up units a lane: fewer, and each lane's few dependent loads leave it idle - measured
    // slower at hidden 4096, 2 a lane)
    P->direct = 0;
    const int ug = H / (L.gu_type == kQ8_0 ? 32 : 256);
    if (n_tok == 1 && n_expert == 1 && (int64_t)k * (F / rh) >= 2 * device_cus() && ug / canon_lanes(ug) >= 4) {
        // a one-expert layer (a shared expert as its own layer) that large stays in slabs: its rows, 8 canonical lanes
        // each, fill only two waves a CU in the direct form, each lane reading scattered 34- or 144-byte blocks, while
        // a slab's DMA streams whole rows; ~72 KB down slabs (config 5's Q8_0 shared expert: 32 rows, one down unit a
        // work-group).  Config 5 T=1: direct 105.3 us; slabs with 16-row down slabs 101.3, 32 rows 99.1; 2 or 8 gate
        // rows a gate/up unit instead of 4: 111 and 117 us (bit for bit throughout)
        int rd1 = (int)((73728 / L.d_row) & ~7ll);
        while (rd1 > 8 && H % rd1) rd1 -= 8;
        if (rd1 >= 8 && H % rd1 == 0 && rd1 <= 64 &&
            fused_lds<1>(n_expert, H, F, rh, 2 * rh * (int)L.gu_row, rd1 * (int)L.d_row, 0, 0).total <= 160 * 1024)
            rd = rd1;
    } else if (n_tok == 1 && (int64_t)k * (F / rh) >= 2 * device_cus() && ug / canon_lanes(ug) >= 4) {
        const int lg = canon_lanes(ug), ld = canon_lanes(F / 32);
        // a gate/up unit fills the work-group's lanes; where that leaves fewer units than CUs, half as many rows a
        // unit, so that twice the CUs stream the rows with half of each work-group's lanes (measured on config 5's
        // shared expert when it took this form: 105.6 -> 104.3 us; halving the down units as well, 118 us)
        const int rh2 = (int64_t)k * (F / (128 / lg)) < device_cus() ? 64 / lg : 128 / lg;
        const int rd2 = 256 / ld;
        if (F % rh2 == 0 && H % rd2 == 0 && rd2 <= 64) {
            P->direct = 1;
            rh = rh2;
            rd = rd2;
        }
    }
    P->rh = rh;
    P->rd = rd;
    P->nu = F / rh;
    P->nj = H / rd;
    P->slab_gu = P->direct ? 0 : 2 * rh * (int)L.gu_row;
    P->slab_dn = P->direct ? 0 : rd * (int)L.d_row;
    P->ne = n_tok >= 4 ? 4 : n_tok >= 2 ? 2 : 1;
    auto lds_of = [&](int ttab) {
        return (P->ne == 1 ? fused_lds<1>(n_expert, H, F, rh, P->slab_gu, P->slab_dn, ttab, P->alias)
                : P->ne == 2 ? fused_lds<2>(n_expert, H, F, rh, P->slab_gu, P->slab_dn, ttab, P->alias)
                             : fused_lds<4>(n_expert, H, F, rh, P->slab_gu, P->slab_dn, ttab, P->alias)).total;
    };
    // 4..16 tokens: the pipelined gate/up path, if its token table and second slab fit
    P->ttab = 0;
    // from two tokens the down slab lies over the gate/up slabs (the early down fetch serves one token), so that the
    // pipelined path's table and second slab fit beside 40 KB down slabs (config 2 at 8 and 16 tokens: 115.7 -> 107.1
    // and 196.2 -> 177.3 us); without the table, two work-groups a CU measured no faster than one
    P->alias = n_tok >= 2;
    if (P->ne == 4 && n_tok <= 16 && lds_of(16) <= 160 * 1024) {
        const int tt = (n_tok + 3) & ~3;   // the table: the call's tokens (rounded up to 4), not 16
        const FusedLds o4 = fused_lds<4>(n_expert, H, F, rh, P->slab_gu, P->slab_dn, tt, P->alias);
        // the pipelined path plans in the LDS past its slab offset: E words for each 32 entries
        if ((int64_t)n_expert * ((kFMaxN + 31) / 32) * 4 <= o4.total - o4.slab_gu) P->ttab = tt;
    }
    P->lds = lds_of(P->ttab);
    return P->lds <= 160 * 1024;
}

template <int TG, int TD, int PER>
static void* pick_per(int ne, int mode) {
    return ne == 1 ? (mode ? (void*)moe_decode_fused_kernel<TG, TD, 1, 1, PER> : (void*)moe_decode_fused_kernel<TG, TD, 1, 0, PER>)
         : ne == 2 ? (void*)moe_decode_fused_kernel<TG, TD, 2, 0, PER>
                   : (mode ? (void*)moe_decode_fused_kernel<TG, TD, 4, 1, PER> : (void*)moe_decode_fused_kernel<TG, TD, 4, 0, PER>);
}
// the routing's experts a lane is a template parameter too: an instance holds one routing form, not five (they were
// two thirds of its code)
template <int TG, int TD>
static void* pick(int ne, int mode, int n_expert) {
    return n_expert <= 64    ? pick_per<TG, TD, 1>(ne, mode)
         : n_expert <= 128   ? pick_per<TG, TD, 2>(ne, mode)
         : n_expert <= 256   ? pick_per<TG, TD, 4>(ne, mode)
         : n_expert <= 512   ? pick_per<TG, TD, 8>(ne, mode)
                             : pick_per<TG, TD, 16>(ne, mode);
}

namespace {
struct LaunchShape {   // per device and kernel: the attribute set and the resident work-groups
    int dev;
    const void* kern;
    int lds, cap, grid_max;
};
std::mutex g_shape_mu;
std::vector<LaunchShape> g_shapes;
}  // namespace

static hipError_t resident_grid(const void* kern, int threads, int lds, int cap, int* grid_max) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_shape_mu);
    for (const LaunchShape& s : g_shapes)
        if (s.dev == dev && s.kern == kern && s.lds == lds && s.cap == cap) {
            *grid_max = s.grid_max;
            return hipSuccess;
        }
    if (lds > 65536 && (e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds)) != hipSuccess)
        return e;
    int cus = 0, occ = 0;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, threads, lds)) != hipSuccess) return e;
    if (occ < 1) return hipErrorInvalidConfiguration;
    *grid_max = cus * (occ > cap ? cap : occ);
    g_shapes.push_back(LaunchShape{dev, kern, lds, cap, *grid_max});
    return hipSuccess;
}

// the routing of a one-expert layer (a shared expert run through the persistent layer): every token's only entry is
// expert 0 with weight 1.0
#define XS_ONES8 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f
static __device__ int32_t g_one_ids[kOneExpertMaxTok];
static __device__ float g_one_w[kOneExpertMaxTok] = {XS_ONES8, XS_ONES8, XS_ONES8, XS_ONES8,
                                                     XS_ONES8, XS_ONES8, XS_ONES8, XS_ONES8};
#undef XS_ONES8
static_assert(kOneExpertMaxTok == 64, "the weights' initializer holds 64 ones");

hipError_t one_expert_routing(const int32_t** ids, const float** w) {
    static std::mutex mu;
    static std::vector<std::pair<int, std::pair<const int32_t*, const float*>>> seen;   // per device
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& d : seen)
        if (d.first == dev) {
            *ids = d.second.first;
            *w = d.second.second;
            return hipSuccess;
        }
    void *pi = nullptr, *pw = nullptr;
    if ((e = hipGetSymbolAddress(&pi, HIP_SYMBOL(g_one_ids))) != hipSuccess) return e;
    if ((e = hipGetSymbolAddress(&pw, HIP_SYMBOL(g_one_w))) != hipSuccess) return e;
    seen.push_back({dev, {(const int32_t*)pi, (const float*)pw}});
    *ids = (const int32_t*)pi;
    *w = (const float*)pw;
    return hipSuccess;
}

hipError_t launch_decode_fused(const FusedArgs& a, const FusedPlan& P, hipStream_t s) {
    void* kern = nullptr;
    // the instance's mode: one token, the direct form; 4+ tokens, the pipelined path when its table takes them all
    const int mode = P.ne == 1 ? (P.direct ? 1 : 0) : P.ne == 4 ? (P.ttab > 0 && a.n_tok <= P.ttab ? 1 : 0) : 0;
    const int E = a.n_expert;
    if (a.L.gu_type == kQ4_K && a.L.d_type == kQ6_K) kern = pick<kQ4_K, kQ6_K>(P.ne, mode, E);
    else if (a.L.gu_type == kQ8_0) kern = pick<kQ8_0, kQ8_0>(P.ne, mode, E);
    else if (a.L.gu_type == kIQ4_XS) kern = pick<kIQ4_XS, kIQ4_XS>(P.ne, mode, E);
    else kern = pick<kQ4_K, kQ4_K>(P.ne, mode, E);
    // every work-group resident at once: the down units wait on the gate/up units of others
    int grid = 0;
    const int threads = fused_threads(P.ne, mode);
    hipError_t e = resident_grid(kern, threads, P.lds, P.direct ? 4 : 2, &grid);
    if (e != hipSuccess) return e;
    const int cap = a.n_tok * a.k < a.n_expert ? a.n_tok * a.k : a.n_expert;
    const int need = cap * (P.nu > P.nj ? P.nu : P.nj);
    FusedArgs a2 = a;
    if (threads > kFT) a2.load_waves = grid > device_cus() ? 4 : 6;   // the pipelined instance: 4 load waves at two
                                                                       // work-groups a CU, 6 at one
    if (grid > need) grid = need;
    void* args[] = {(void*)&a2};
    return hipLaunchKernel(kern, dim3(grid), dim3(threads), args, P.lds, s);
}

}  // namespace xs
