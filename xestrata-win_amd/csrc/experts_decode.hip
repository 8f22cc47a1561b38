// xestrata-win_amd/csrc/experts_decode.hip - grouped expert products for decode and verify windows (1-16 tokens):
// the MI355X form of the reference's native_expert_grouped (src/kernels/xe/iq_kernels.cpp:2042-2178; gate/up rows
// :997-1031, the SwiGLU + q8_1 pass :2118-2133, down rows :1033-1063).
//
// Work split.  A work-group (4 waves) owns a slab of consecutive weight rows of one group's expert: gate and up rows
// are one matrix of 2 n_ff rows (the blob stores them back to back), down rows another of n_embd rows.  The slab is
// copied to LDS with 16-byte coalesced loads (the whole slab in flight at once), so the raw GGUF blocks are read from
// HBM exactly once whatever their alignment (Q6_K and Q8_0 blocks sit at 2-byte boundaries).  The group's entries
// (tokens routed to the expert) are applied to the staged rows kNE at a time, so each row is fetched once however
// many entries the group has.
//
// Inside a slab a row is a run of 32-value units; LPR lanes share a row (LPR divides the unit count), each taking
// every LPR-th unit.  A unit's integer products are exact (v_dot4_i32_i8 against the q8_1 activation), its scales
// are applied in fp32, and the LPR lanes reduce their partial sums with a xor butterfly.
//
// Activations are q8_1 rows: for gate/up the caller's x_q8_1 (one scale per 256 values), for down the SwiGLU of the
// gate/up results quantized per 32 values, both with the reference's canonical arithmetic.  The down kernel forms
// that activation itself from the gate/up scratch (the reference's separate SwiGLU pass folded into its prologue);
// the q8_1 rows it builds are also written to scratch (hq), as the reference's pass leaves them.
#include "xs_device.h"
#include "xs_kernels.h"

namespace xs {

constexpr int kNE = 4;         // entries a pass over the staged rows (the reference's kEntriesPass)
constexpr int kThreads = 256;

__constant__ uint32_t kIq4Tab[4] = {0xBFAD9881u, 0xF6EADDCFu, 0x26190D01u, 0x71594535u};   // kvalues_iq4nl bytes

__device__ __forceinline__ int byte_at(uint32_t s0, uint32_t s1, uint32_t s2, int k) {
    const uint32_t w = k < 4 ? s0 : k < 8 ? s1 : s2;
    return (int)((w >> (8 * (k & 3))) & 0xFFu);
}
// the 6-bit scale and min of Q4_K sub-block s from the 12 scale bytes (reference dequant.hpp:181-190)
__device__ __forceinline__ void q4k_sm(uint32_t s0, uint32_t s1, uint32_t s2, int s, int& sc, int& m) {
    if (s < 4) {
        sc = byte_at(s0, s1, s2, s) & 63;
        m = byte_at(s0, s1, s2, s + 4) & 63;
    } else {
        const int hi = byte_at(s0, s1, s2, s + 4);
        sc = (hi & 0x0F) | ((byte_at(s0, s1, s2, s - 4) >> 6) << 4);
        m = (hi >> 4) | ((byte_at(s0, s1, s2, s) >> 6) << 4);
    }
}

__device__ __forceinline__ float lds_h(const uint8_t* p) { return h2f(*(const uint16_t*)p); }

template <int T>
struct Unit;

// Q4_K unit u: 16 bytes of qs = 16 low nibbles of sub-block 2p and 16 high nibbles of sub-block 2p + 1
template <>
struct Unit<kQ4_K> {
    struct W {
        uint32_t q[4];
        float d, dmin;
        int sca, ma, scb, mb, pa;
    };
    __device__ static __forceinline__ W load(const uint8_t* row, int u) {
        W w;
        const int b = u >> 3, j = u & 7, p = j >> 1;
        const uint8_t* blk = row + 144 * b;
        const uint4 hdr = *(const uint4*)blk;
        const uint4 qs = *(const uint4*)(blk + 16 + 16 * j);
        w.q[0] = qs.x; w.q[1] = qs.y; w.q[2] = qs.z; w.q[3] = qs.w;
        w.d = h2f((uint16_t)(hdr.x & 0xFFFFu));
        w.dmin = h2f((uint16_t)(hdr.x >> 16));
        q4k_sm(hdr.y, hdr.z, hdr.w, 2 * p, w.sca, w.ma);
        q4k_sm(hdr.y, hdr.z, hdr.w, 2 * p + 1, w.scb, w.mb);
        w.pa = 256 * b + 64 * p + 16 * (j & 1);
        return w;
    }
    __device__ static __forceinline__ float apply(const W& w, const int8_t* act, const float* d8, const int* us16) {
        const uint4 a = *(const uint4*)(act + w.pa);
        const uint4 bq = *(const uint4*)(act + w.pa + 32);
        int ia = 0, ib = 0;
        ia = sdot4((int)(w.q[0] & 0x0F0F0F0Fu), (int)a.x, ia);
        ia = sdot4((int)(w.q[1] & 0x0F0F0F0Fu), (int)a.y, ia);
        ia = sdot4((int)(w.q[2] & 0x0F0F0F0Fu), (int)a.z, ia);
        ia = sdot4((int)(w.q[3] & 0x0F0F0F0Fu), (int)a.w, ia);
        ib = sdot4((int)((w.q[0] >> 4) & 0x0F0F0F0Fu), (int)bq.x, ib);
        ib = sdot4((int)((w.q[1] >> 4) & 0x0F0F0F0Fu), (int)bq.y, ib);
        ib = sdot4((int)((w.q[2] >> 4) & 0x0F0F0F0Fu), (int)bq.z, ib);
        ib = sdot4((int)((w.q[3] >> 4) & 0x0F0F0F0Fu), (int)bq.w, ib);
        const int ua = us16[w.pa >> 4], ub = us16[(w.pa >> 4) + 2];
        const float fa = (float)(w.sca * ia) * w.d - (float)(w.ma * ua) * w.dmin;
        const float fb = (float)(w.scb * ib) * w.d - (float)(w.mb * ub) * w.dmin;
        return d8[w.pa >> 5] * fa + d8[(w.pa >> 5) + 1] * fb;
    }
};

// Q6_K unit u = (block b, half n, c): ql bytes [64n + 16c, +16) hold values 128n + 16c + i (low nibbles) and
// 128n + 64 + 16c + i (high); their 2 high bits are in qh[32n + 16(c & 1) + i] at shifts 2(c >> 1) and 4 + 2(c >> 1)
template <>
struct Unit<kQ6_K> {
    struct W {
        uint32_t lo[4], hi[4];
        float d;
        int scl, sch, pl;
    };
    __device__ static __forceinline__ W load(const uint8_t* row, int u) {
        W w;
        const int b = u >> 3, n = (u >> 2) & 1, c = u & 3;
        const uint8_t* blk = row + 210 * b;
        const uint8_t* ql = blk + 64 * n + 16 * c;
        const uint8_t* qh = blk + 128 + 32 * n + 16 * (c & 1);
        const int sh = 2 * (c >> 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t l = ld_u32_a2(ql + 4 * i), h = ld_u32_a2(qh + 4 * i);
            w.lo[i] = (l & 0x0F0F0F0Fu) | (((h >> sh) & 0x03030303u) << 4);
            w.hi[i] = ((l >> 4) & 0x0F0F0F0Fu) | (((h >> (4 + sh)) & 0x03030303u) << 4);
        }
        w.scl = (int)(int8_t)blk[192 + 8 * n + c];
        w.sch = (int)(int8_t)blk[192 + 8 * n + 4 + c];
        w.d = lds_h(blk + 208);
        w.pl = 256 * b + 128 * n + 16 * c;
        return w;
    }
    __device__ static __forceinline__ float apply(const W& w, const int8_t* act, const float* d8, const int* us16) {
        const uint4 a = *(const uint4*)(act + w.pl);
        const uint4 h = *(const uint4*)(act + w.pl + 64);
        int il = 0, ih = 0;
        il = sdot4((int)w.lo[0], (int)a.x, il);
        il = sdot4((int)w.lo[1], (int)a.y, il);
        il = sdot4((int)w.lo[2], (int)a.z, il);
        il = sdot4((int)w.lo[3], (int)a.w, il);
        ih = sdot4((int)w.hi[0], (int)h.x, ih);
        ih = sdot4((int)w.hi[1], (int)h.y, ih);
        ih = sdot4((int)w.hi[2], (int)h.z, ih);
        ih = sdot4((int)w.hi[3], (int)h.w, ih);
        il -= 32 * us16[w.pl >> 4];              // the codes are q + 32
        ih -= 32 * us16[(w.pl >> 4) + 4];
        return w.d * (d8[w.pl >> 5] * (float)(w.scl * il) + d8[(w.pl >> 5) + 2] * (float)(w.sch * ih));
    }
};

// Q8_0 unit u = block u
template <>
struct Unit<kQ8_0> {
    struct W {
        uint32_t q[8];
        float d;
        int u;
    };
    __device__ static __forceinline__ W load(const uint8_t* row, int u) {
        W w;
        const uint8_t* blk = row + 34 * u;
        w.d = lds_h(blk);
#pragma unroll
        for (int i = 0; i < 8; ++i) w.q[i] = ld_u32_a2(blk + 2 + 4 * i);
        w.u = u;
        return w;
    }
    __device__ static __forceinline__ float apply(const W& w, const int8_t* act, const float* d8, const int*) {
        const uint4 a0 = *(const uint4*)(act + 32 * w.u);
        const uint4 a1 = *(const uint4*)(act + 32 * w.u + 16);
        int s = 0;
        s = sdot4((int)w.q[0], (int)a0.x, s);
        s = sdot4((int)w.q[1], (int)a0.y, s);
        s = sdot4((int)w.q[2], (int)a0.z, s);
        s = sdot4((int)w.q[3], (int)a0.w, s);
        s = sdot4((int)w.q[4], (int)a1.x, s);
        s = sdot4((int)w.q[5], (int)a1.y, s);
        s = sdot4((int)w.q[6], (int)a1.z, s);
        s = sdot4((int)w.q[7], (int)a1.w, s);
        return (w.d * d8[w.u]) * (float)s;
    }
};

// IQ4_XS unit u = sub-block s of block b: 16 qs bytes, low nibbles values 0..15, high nibbles 16..31
template <>
struct Unit<kIQ4_XS> {
    struct W {
        int lo[4], hi[4];
        float d;
        int ls, p;
    };
    __device__ static __forceinline__ W load(const uint8_t* row, int u) {
        W w;
        const int b = u >> 3, s = u & 7;
        const uint8_t* blk = row + 136 * b;
        const uint2 hdr = *(const uint2*)blk;
        const uint2 q0 = *(const uint2*)(blk + 8 + 16 * s), q1 = *(const uint2*)(blk + 16 + 16 * s);
        const uint32_t qw[4] = {q0.x, q0.y, q1.x, q1.y};
        const uint32_t t0 = kIq4Tab[0], t1 = kIq4Tab[1], t2 = kIq4Tab[2], t3 = kIq4Tab[3];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w.lo[i] = table16_lookup(qw[i] & 0x0F0F0F0Fu, t0, t1, t2, t3);
            w.hi[i] = table16_lookup((qw[i] >> 4) & 0x0F0F0F0Fu, t0, t1, t2, t3);
        }
        w.d = h2f((uint16_t)(hdr.x & 0xFFFFu));
        const uint32_t scales_h = hdr.x >> 16;
        const uint32_t sl = (hdr.y >> (8 * (s >> 1))) & 0xFFu;
        w.ls = (int)(((sl >> (4 * (s & 1))) & 0x0Fu) | (((scales_h >> (2 * s)) & 3u) << 4)) - 32;
        w.p = 256 * b + 32 * s;
        return w;
    }
    __device__ static __forceinline__ float apply(const W& w, const int8_t* act, const float* d8, const int*) {
        const uint4 a0 = *(const uint4*)(act + w.p);
        const uint4 a1 = *(const uint4*)(act + w.p + 16);
        int s = 0;
        s = sdot4(w.lo[0], (int)a0.x, s);
        s = sdot4(w.lo[1], (int)a0.y, s);
        s = sdot4(w.lo[2], (int)a0.z, s);
        s = sdot4(w.lo[3], (int)a0.w, s);
        s = sdot4(w.hi[0], (int)a1.x, s);
        s = sdot4(w.hi[1], (int)a1.y, s);
        s = sdot4(w.hi[2], (int)a1.z, s);
        s = sdot4(w.hi[3], (int)a1.w, s);
        return (w.d * d8[w.p >> 5]) * (float)(s * w.ls);
    }
};

// the slab: n16 16-byte chunks, all of a thread's loads issued before its stores
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void stage_slab(const uint8_t* __restrict__ src, uint8_t* dst, int n16) {
    const int tid = threadIdx.x;
    for (int i0 = 0; i0 < n16; i0 += kThreads * 8) {
        u32x4_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j * kThreads + tid;
            if (i < n16) v[j] = __builtin_nontemporal_load((const u32x4_t*)src + i);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j * kThreads + tid;
            if (i < n16) ((u32x4_t*)dst)[i] = v[j];
        }
    }
}

template <int T, int LPR, bool DOWN>
__global__ __launch_bounds__(kThreads) void grouped_kernel(ExpertLayout L, GroupedArgs a, int rows_total, int slab_rows,
                                                           int64_t mat_off, int64_t rb) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int n_in = DOWN ? (int)L.n_ff : (int)L.n_embd;
    const int U = n_in >> 5;
    const int64_t slab_bytes = (int64_t)slab_rows * rb;
    uint8_t* slab = lds;
    int8_t* act = (int8_t*)(lds + slab_bytes);
    float* d8 = (float*)(act + kNE * n_in);
    int* us16 = (int*)(d8 + kNE * (n_in >> 5));
    const int tid = threadIdx.x, lane = tid & 63;
    const int r0 = blockIdx.x * slab_rows;
    const int nrows = min(slab_rows, rows_total - r0);
    const int ngroups = *a.n_groups;
    const int F = (int)L.n_ff, H = (int)L.n_embd;
    for (int g = blockIdx.y; g < ngroups; g += gridDim.y) {
        const uint8_t* blob = (const uint8_t*)a.grp_ptr[g];
        if (((uintptr_t)blob & 15u) != 0) {
            if (tid == 0) atomicOr(a.err, 1);
            continue;
        }
        __syncthreads();   // the previous group's readers of the slab are done
        stage_slab(blob + mat_off + (int64_t)r0 * rb, slab, (int)(((int64_t)nrows * rb) >> 4));
        const int e0 = a.grp_start[g], e1 = a.grp_start[g + 1];
        for (int p = e0; p < e1; p += kNE) {
            const int n = min(kNE, e1 - p);
            __syncthreads();   // the previous pass's readers of the activations are done
            if (!DOWN) {
                // the entries' q8_1 rows: int8 values, fp32 scales, sums of 16
                const int nb = n_in >> 5;
                for (int i = tid; i < n * nb; i += kThreads) {
                    const int e = i / nb, bi = i - e * nb;
                    const uint32_t* blk =
                        (const uint32_t*)((const uint8_t*)a.x_q8_1 + ((int64_t)a.ent_tok[p + e] * nb + bi) * 36);
                    uint32_t w[9];
#pragma unroll
                    for (int k = 0; k < 9; ++k) w[k] = blk[k];
                    uint4* dst = (uint4*)(act + e * n_in + 32 * bi);
                    dst[0] = make_uint4(w[1], w[2], w[3], w[4]);
                    dst[1] = make_uint4(w[5], w[6], w[7], w[8]);
                    d8[e * nb + bi] = h2f((uint16_t)(w[0] & 0xFFFFu));
                    int s0 = 0, s1 = 0;
#pragma unroll
                    for (int k = 1; k <= 4; ++k) s0 = sdot4((int)w[k], 0x01010101, s0);
#pragma unroll
                    for (int k = 5; k <= 8; ++k) s1 = sdot4((int)w[k], 0x01010101, s1);
                    us16[e * (n_in >> 4) + 2 * bi] = s0;
                    us16[e * (n_in >> 4) + 2 * bi + 1] = s1;
                }
            } else {
                // h = SwiGLU(gate, up) with the canonical arithmetic, then per-32 canonical q8_1 (reference
                // iq_kernels.cpp:2118-2133); 32 neighbouring lanes hold one block
                const bool write_hq = blockIdx.x == 0;
                for (int i = tid; i < n * F; i += kThreads) {
                    const int e = i / F, col = i - e * F;
                    const int64_t gi = (int64_t)(p + e) * F + col;
                    const float h = canon_silu_mul(a.gate[gi], a.up[gi]);
                    const float amax = group_max<32>(fabsf(h));
                    const float sum = group_sum<32>(h);
                    const float d = q8_scale(amax);
                    const int q = q8_value(h, q8_inv(d));
                    act[e * n_in + col] = (int8_t)q;
                    const uint16_t hd = f2h(d);
                    if ((col & 31) == 0) d8[e * (n_in >> 5) + (col >> 5)] = h2f(hd);
                    if (write_hq) {
                        uint8_t* blk = (uint8_t*)a.hq + ((int64_t)(p + e) * (F >> 5) + (col >> 5)) * 36;
                        blk[4 + (col & 31)] = (uint8_t)q;
                        if ((col & 31) == 0)
                            *(uint32_t*)blk = (uint32_t)hd | ((uint32_t)f2h(q8_1_finite(sum)) << 16);
                    }
                }
                __syncthreads();
                for (int i = tid; i < n * (n_in >> 4); i += kThreads) {
                    const uint4 v = *(const uint4*)(act + 16 * i);
                    int s = 0;
                    s = sdot4((int)v.x, 0x01010101, s);
                    s = sdot4((int)v.y, 0x01010101, s);
                    s = sdot4((int)v.z, 0x01010101, s);
                    s = sdot4((int)v.w, 0x01010101, s);
                    const int e = i / (n_in >> 4);
                    us16[i] = s;
                    (void)e;
                }
            }
            __syncthreads();
            const int c = lane & (LPR - 1);
            for (int rr = tid / LPR; rr < nrows; rr += kThreads / LPR) {
                const uint8_t* row = slab + (int64_t)rr * rb;
                float acc[kNE];
#pragma unroll
                for (int e = 0; e < kNE; ++e) acc[e] = 0.0f;
                for (int u = c; u < U; u += LPR) {
                    const typename Unit<T>::W w = Unit<T>::load(row, u);
#pragma unroll
                    for (int e = 0; e < kNE; ++e)
                        if (e < n)
                            acc[e] += Unit<T>::apply(w, act + e * n_in, d8 + e * (n_in >> 5), us16 + e * (n_in >> 4));
                }
#pragma unroll
                for (int e = 0; e < kNE; ++e) acc[e] = group_sum<LPR>(acc[e]);
                if (c == 0) {
                    const int r = r0 + rr;
                    for (int e = 0; e < n; ++e) {
                        if (DOWN) a.out[(int64_t)a.ent_dst[p + e] * H + r] = acc[e];
                        else if (r < F) a.gate[(int64_t)(p + e) * F + r] = acc[e];
                        else a.up[(int64_t)(p + e) * F + (r - F)] = acc[e];
                    }
                }
            }
        }
    }
}

static int lanes_per_row(int units) {
    int l = 64;
    while (l > 1 && units % l) l >>= 1;
    return l;
}

template <int T, bool DOWN>
static hipError_t launch_t(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s) {
    const int n_in = DOWN ? (int)L.n_ff : (int)L.n_embd;
    const int rows_total = DOWN ? (int)L.n_embd : (int)(2 * L.n_ff);
    const int64_t rb = DOWN ? L.d_row : L.gu_row;
    const int64_t mat_off = DOWN ? L.down_off : 0;
    const int lpr = lanes_per_row(n_in / 32);
    const int per_pass = kThreads / lpr;
    const int base = per_pass > 8 ? per_pass : 8;
    int64_t mult = 24576 / ((int64_t)base * rb);
    if (mult < 1) mult = 1;
    int slab_rows = (int)(base * mult);
    if (slab_rows > rows_total) slab_rows = rows_total;
    const size_t lds = (size_t)slab_rows * rb + (size_t)kNE * (n_in + (n_in / 32) * 4 + (n_in / 16) * 4);
    const int64_t gy = a.grid_groups > 0 && a.grid_groups < a.cap_groups ? a.grid_groups : a.cap_groups;
    const dim3 grid((unsigned)((rows_total + slab_rows - 1) / slab_rows), (unsigned)gy);
    void (*kern)(ExpertLayout, GroupedArgs, int, int, int64_t, int64_t) = nullptr;
    switch (lpr) {
        case 64: kern = grouped_kernel<T, 64, DOWN>; break;
        case 32: kern = grouped_kernel<T, 32, DOWN>; break;
        case 16: kern = grouped_kernel<T, 16, DOWN>; break;
        case 8: kern = grouped_kernel<T, 8, DOWN>; break;
        case 4: kern = grouped_kernel<T, 4, DOWN>; break;
        case 2: kern = grouped_kernel<T, 2, DOWN>; break;
        default: kern = grouped_kernel<T, 1, DOWN>; break;
    }
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), lds, s, L, a, rows_total, slab_rows, mat_off, rb);
    return hipGetLastError();
}

hipError_t launch_native_gu(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s) {
    switch (L.gu_type) {
        case kQ4_K: return launch_t<kQ4_K, false>(L, a, s);
        case kQ6_K: return launch_t<kQ6_K, false>(L, a, s);
        case kQ8_0: return launch_t<kQ8_0, false>(L, a, s);
        case kIQ4_XS: return launch_t<kIQ4_XS, false>(L, a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_native_down(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s) {
    switch (L.d_type) {
        case kQ4_K: return launch_t<kQ4_K, true>(L, a, s);
        case kQ6_K: return launch_t<kQ6_K, true>(L, a, s);
        case kQ8_0: return launch_t<kQ8_0, true>(L, a, s);
        case kIQ4_XS: return launch_t<kIQ4_XS, true>(L, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace xs
