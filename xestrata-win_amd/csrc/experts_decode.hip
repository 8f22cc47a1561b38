// xestrata-win_amd/csrc/experts_decode.hip - grouped expert products for decode and verify windows (1-16 tokens):
// the MI355X form of the reference's native_expert_grouped (src/kernels/xe/iq_kernels.cpp:2042-2178; gate/up rows
// :997-1031, the SwiGLU + q8_1 pass :2118-2133, down rows :1033-1063).
//
// Work split.  A work-group (2 waves) owns a slab of consecutive weight rows of one group's expert: the gate and up
// rows are one matrix of 2 n_ff rows (the blob stores them back to back), the down rows another of n_embd rows.  The
// slab is fetched with 16-byte coalesced loads, all of a thread's loads in flight at once together with the group's
// indices and activations, and parked in LDS, so the raw GGUF blocks are read from HBM once whatever their alignment
// (Q6_K and Q8_0 blocks sit at 2-byte boundaries).  The group's entries (the tokens routed to the expert) are applied
// to the staged rows kNE at a time.
//
// Arithmetic: the canonical row order (shared bit for bit with the CPU oracle).  A row is a run of units: a whole
// 256-value block when the activation has one scale for each 256 values (gate/up: quantize_q8_1_rows), else a
// 32-value group (down, and Q8_0).  A unit's products are exact integers (v_dot4_i32_i8 of the codes against the q8_1
// int8 values, the sub-block scales applied in integers); its scale enters once, acc = fma(d * d8, S, acc) (Q4_K's
// min term a second fma) - the reference's integer-first canonical rows (seg_dot_canon, iq_kernels.cpp:832-884)
// applied to every format.  L = min(8, the largest power of two dividing the unit count) lanes share a row, lane c
// taking units c, c + L, ..., then a xor butterfly over the L lanes.
//
// Activations: gate/up reads the caller's q8_1 rows; down forms its own from the gate/up scratch, h = SwiGLU(gate,
// up) quantized per 32 values, both with the reference's canonical arithmetic (the reference's separate SwiGLU pass
// folded into the down kernel's prologue); the q8_1 rows it builds are also written to scratch (hq).
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_units.h"

namespace xs {

constexpr int kNE = 4;          // the most entries a pass over the staged rows (the reference's kEntriesPass)
constexpr int kThreads = 128;   // two waves a work-group
constexpr int kSlabRegs = 10;   // 16-byte slab chunks a thread holds in flight

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// The whole grouped pass of one matrix (gate/up: DOWN false, down: DOWN true).
template <int T, int LPR, bool DOWN, int NE>
__global__ __launch_bounds__(kThreads) void grouped_kernel(ExpertLayout L, GroupedArgs a, int rows_total, int slab_rows,
                                                           int64_t mat_off, int64_t rb, int row0) {
    // gate/up: the staged rows carry kActPad bytes after every 256 int8 values (Unit's PAD), so that a row's lanes,
    // which read neighbouring 256-value blocks at once, hit distinct LDS banks
    constexpr int kPad = DOWN ? 0 : kActPad;
    using U = Unit<T, !DOWN, kPad>;
    extern __shared__ __align__(16) uint8_t lds[];
    const int n_in = DOWN ? (int)L.n_ff : (int)L.n_embd;
    const int rowq = act_rowq(n_in, kPad);   // a staged row's int8 bytes
    const int units = n_in / U::kUnit;
    const int64_t slab_bytes = (int64_t)slab_rows * rb;
    uint8_t* slab = lds;
    int8_t* actq = (int8_t*)(lds + slab_bytes);
    float* actd = (float*)(actq + NE * rowq);
    int* acts = (int*)(actd + NE * (n_in >> 5));
    const int tid = threadIdx.x, lane = tid & 63;
    const int r0 = blockIdx.x * slab_rows;
    const int nrows = min(slab_rows, rows_total - r0);
    const int n16 = (int)(((int64_t)nrows * rb) >> 4);
    const int ngroups = *a.n_groups;
    const int F = (int)L.n_ff, H = (int)L.n_embd;
    const int nb = n_in >> 5;
    Act act[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) act[e] = Act{actq + e * rowq, actd + e * nb, acts + e * (n_in >> 4)};

    for (int g = blockIdx.y; g < ngroups; g += gridDim.y) {
        const uint8_t* blob = (const uint8_t*)a.grp_ptr[g];
        const int e0 = a.grp_start[g], e1 = a.grp_start[g + 1];
        if (((uintptr_t)blob & 15u) != 0) {
            if (tid == 0) atomicOr(a.err, 1);
            continue;
        }
        const u32x4_t* src = (const u32x4_t*)(blob + mat_off + (int64_t)r0 * rb);
        __syncthreads();   // the previous group's readers of the slab are done
        for (int p = e0; p < e1; p += NE) {
            const int n = min(NE, e1 - p);
            if (p > e0) __syncthreads();   // the previous pass's readers of the activations are done
            // the slab (first pass only): every chunk of this thread in flight before any is stored
            u32x4_t v[kSlabRegs];
            if (p == e0) {
#pragma unroll
                for (int j = 0; j < kSlabRegs; ++j) {
                    const int i = j * kThreads + tid;
                    if (i < n16) v[j] = __builtin_nontemporal_load(src + i);
                }
            }
            if (!DOWN) {
                // the entries' q8_1 rows: int8 values, fp32 scales, sums of 16
                for (int i = tid; i < n * nb; i += kThreads) {
                    const int e = i / nb, bi = i - e * nb;
                    const uint32_t* blk =
                        (const uint32_t*)((const uint8_t*)a.x_q8_1 + ((int64_t)a.ent_tok[p + e] * nb + bi) * 36);
                    uint32_t w[9];
#pragma unroll
                    for (int k = 0; k < 9; ++k) w[k] = blk[k];
                    uint4* dst = (uint4*)(actq + e * rowq + 32 * bi + kPad * (bi >> 3));
                    dst[0] = make_uint4(w[1], w[2], w[3], w[4]);
                    dst[1] = make_uint4(w[5], w[6], w[7], w[8]);
                    actd[e * nb + bi] = h2f((uint16_t)(w[0] & 0xFFFFu));
                    int s0 = 0, s1 = 0;
#pragma unroll
                    for (int k = 1; k <= 4; ++k) s0 = sdot4((int)w[k], 0x01010101, s0);
#pragma unroll
                    for (int k = 5; k <= 8; ++k) s1 = sdot4((int)w[k], 0x01010101, s1);
                    acts[e * (n_in >> 4) + 2 * bi] = s0;
                    acts[e * (n_in >> 4) + 2 * bi + 1] = s1;
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
                    actq[e * n_in + col] = (int8_t)q;
                    const uint16_t hd = f2h(d);
                    if ((col & 31) == 0) actd[e * nb + (col >> 5)] = h2f(hd);
                    if (write_hq) {
                        uint8_t* blk = (uint8_t*)a.hq + ((int64_t)(p + e) * (F >> 5) + (col >> 5)) * 36;
                        blk[4 + (col & 31)] = (uint8_t)q;
                        if ((col & 31) == 0)
                            *(uint32_t*)blk = (uint32_t)hd | ((uint32_t)f2h(q8_1_finite(sum)) << 16);
                    }
                }
            }
            if (p == e0) {
#pragma unroll
                for (int j = 0; j < kSlabRegs; ++j) {
                    const int i = j * kThreads + tid;
                    if (i < n16) ((u32x4_t*)slab)[i] = v[j];
                }
                for (int i = kSlabRegs * kThreads + tid; i < n16; i += kThreads)   // a slab past the registers
                    ((u32x4_t*)slab)[i] = __builtin_nontemporal_load(src + i);
            }
            if (DOWN) {
                __syncthreads();
                for (int i = tid; i < n * (n_in >> 4); i += kThreads) {
                    const uint4 w = *(const uint4*)(actq + 16 * i);
                    int s = 0;
                    s = sdot4((int)w.x, 0x01010101, s);
                    s = sdot4((int)w.y, 0x01010101, s);
                    s = sdot4((int)w.z, 0x01010101, s);
                    s = sdot4((int)w.w, 0x01010101, s);
                    acts[i] = s;
                }
            }
            __syncthreads();
            const int c = lane & (LPR - 1);
            for (int rr = tid / LPR; rr < nrows; rr += kThreads / LPR) {
                const int roff = rr * (int)rb;
                float acc[NE];
#pragma unroll
                for (int e = 0; e < NE; ++e) acc[e] = 0.0f;
                for (int u = c; u < units; u += LPR) U::template apply<NE>(slab, roff, u, act, n, acc);
#pragma unroll
                for (int e = 0; e < NE; ++e) acc[e] = group_sum<LPR>(acc[e]);
                if (c == 0) {
                    const int r = row0 + r0 + rr;   // (gate/up: rows 0 .. F gate, F .. 2F up)
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

// part (gate/up only): 0 the gate and up rows as one matrix, 1 the gate rows alone, 2 the up rows alone (a mixed
// layer's two launches, each of its own type)
template <int T, bool DOWN>
static hipError_t launch_t(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s, int part = 0) {
    const int n_in = DOWN ? (int)L.n_ff : (int)L.n_embd;
    const int rows_total = DOWN ? (int)L.n_embd : (int)(part ? L.n_ff : 2 * L.n_ff);
    const int64_t rb = DOWN ? L.d_row : part == 2 ? L.up_row : L.gu_row;
    const int64_t mat_off = DOWN ? L.down_off : part == 2 ? L.up_off : 0;
    const int row0 = part == 2 ? (int)L.n_ff : 0;
    const int unit = Unit<T, !DOWN>::kUnit;
    const int lpr = canon_lanes(n_in / unit);
    const int per_pass = kThreads / lpr;
    int64_t rows = (20480 / rb) & ~(int64_t)7;               // about 20 KB of weights a work-group
    if (rows < 8) rows = 8;
    if (rows > 2 * per_pass) rows = 2 * per_pass;
    int slab_rows = (int)rows;
    if (slab_rows > rows_total) slab_rows = rows_total;
    // entries a pass: the most a group can hold (one per token), up to kNE
    const int ne = a.max_entries > 0 && a.max_entries < 4 ? (a.max_entries == 1 ? 1 : 2) : kNE;
    const size_t lds = (size_t)slab_rows * rb + (size_t)ne * (act_rowq(n_in, DOWN ? 0 : kActPad) + (n_in / 32) * 4 + (n_in / 16) * 4);
    const int64_t gy = a.grid_groups > 0 && a.grid_groups < a.cap_groups ? a.grid_groups : a.cap_groups;
    const dim3 grid((unsigned)((rows_total + slab_rows - 1) / slab_rows), (unsigned)gy);
    void (*kern)(ExpertLayout, GroupedArgs, int, int, int64_t, int64_t, int) = nullptr;
    switch (lpr * 8 + ne) {
        case 8 * 8 + 1: kern = grouped_kernel<T, 8, DOWN, 1>; break;
        case 8 * 8 + 2: kern = grouped_kernel<T, 8, DOWN, 2>; break;
        case 8 * 8 + 4: kern = grouped_kernel<T, 8, DOWN, 4>; break;
        case 4 * 8 + 1: kern = grouped_kernel<T, 4, DOWN, 1>; break;
        case 4 * 8 + 2: kern = grouped_kernel<T, 4, DOWN, 2>; break;
        case 4 * 8 + 4: kern = grouped_kernel<T, 4, DOWN, 4>; break;
        case 2 * 8 + 1: kern = grouped_kernel<T, 2, DOWN, 1>; break;
        case 2 * 8 + 2: kern = grouped_kernel<T, 2, DOWN, 2>; break;
        case 2 * 8 + 4: kern = grouped_kernel<T, 2, DOWN, 4>; break;
        case 1 * 8 + 1: kern = grouped_kernel<T, 1, DOWN, 1>; break;
        case 1 * 8 + 2: kern = grouped_kernel<T, 1, DOWN, 2>; break;
        default: kern = grouped_kernel<T, 1, DOWN, 4>; break;
    }
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), lds, s, L, a, rows_total, slab_rows, mat_off, rb, row0);
    return hipGetLastError();
}

static hipError_t launch_gu_part(int type, const ExpertLayout& L, const GroupedArgs& a, hipStream_t s, int part) {
    switch (type) {
        case kQ4_K: return launch_t<kQ4_K, false>(L, a, s, part);
        case kQ6_K: return launch_t<kQ6_K, false>(L, a, s, part);
        case kQ8_0: return launch_t<kQ8_0, false>(L, a, s, part);
        case kIQ4_XS: return launch_t<kIQ4_XS, false>(L, a, s, part);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_native_gu(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s) {
    if (!mixed_gu(L)) return launch_gu_part(L.gu_type, L, a, s, 0);
    // a mixed layer: the gate rows and the up rows as two matrices, each with its own type's unit and lanes
    const hipError_t e = launch_gu_part(L.gu_type, L, a, s, 1);
    return e != hipSuccess ? e : launch_gu_part(L.up_type, L, a, s, 2);
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
