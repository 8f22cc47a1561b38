// xestrata-win_amd/csrc/experts_prefill.hip - grouped expert products for prompt and verify batches: an f16 MFMA
// grouped GEMM over expert weights dequantized from the raw GGUF blocks (the MI355X replacement of the reference's
// int8 iq_mmq_grouped, src/kernels/xe/iq_mmq.cpp:483-943, and of its FP16 path dequant_f16 + xmx_gemm_grouped /
// Gemm::f16_groups, src/prefill/gemm.cpp:371-388, whose FP16 x FP16 -> FP32 arithmetic this follows).
//
// Rows are the routed rows in expert order (the permutation of src/prefill/plain_prompt.cpp:576-637).  Two launches:
//   gate/up: h[row, j] = SwiGLU(x[src[row]] . gate_j, x[src[row]] . up_j) in f16, a tile = 128 rows x 128 h columns
//            (their 128 gate and 128 up weight rows, so the SwiGLU is formed in registers);
//   down:    parts[entry[row], c] = h[row] . down_c in fp32, a tile = 128 rows x 256 output columns, written straight
//            into routing order for the combine.
//
// Why f16 and not bf16: the dequantization is the kernel's ALU cost, and gfx950 has packed f16 arithmetic
// (v_pk_fma_f16, two values an instruction) but none for bf16.  A 4-bit code q becomes an f16 with one v_and_or_b32
// that drops it into the mantissa of a constant (0x6400 | q = 1024 + q; 0x4C00 | q << 4 = 16 + q / 4), and one packed
// FMA with the sub-block scale and the exactly representable -1024 d (or -64 d) turns two of them into d q, rounded
// once; the Q4_K minimum is one packed add more.  The MFMA is v_mfma_f32_32x32x16_f16 (the bf16 rate).
//
// K order: in each step of 64 values, MFMA fragment slot p of both operands holds value 8 P[p / 8] + P[p % 8] with
// P = (0 2 1 3 4 6 5 7) - the order in which the bytes of a little-endian quant word come out in pairs (bytes 0 and 2,
// then 1 and 3).  The activations x and h are stored in that order (f16, saturated), so an activation fragment is one
// 16-byte LDS read and a weight fragment is built from two quant words with no shuffles.
//
// Work-group: 4 waves over a 128-row x 256-weight-row tile; wave w owns 64 weight rows (two 32-column MFMA tiles)
// and each lane dequantizes the fragments of its two weight rows in registers, one step ahead of their MFMAs.  Q6_K
// down weights take a 128-row x 128-weight-row tile, one weight row a lane: a dequantized fragment then feeds four
// MFMAs (against 64-row tiles' two), which halves the dequantization and the weight loads a product.  The
// tile's activation rows reach LDS by DMA (global_load_lds_dwordx4, gathered through src for gate/up) into a double
// buffer, chunk c of row r at slot c ^ swk(r) (a fragment read is free of bank conflicts).  Row tiles
// of 32 past the group's rows are skipped.  A work-group's m-tile comes from a flat index over every group's
// ceil(rows / 128) tiles (a prefix computed on the device).  Work-group b runs on XCD b % 8; an XCD takes every
// eighth m-tile and runs its n-tiles one after the other, so the m-tile's activations and its expert's weights are
// fetched into that XCD's L2 once and reused across the n-tiles.
#include "xs_device.h"
#include "xs_dequant.h"
#include "xs_f16.h"
#include "xs_kernels.h"
#include "xs_units.h"

namespace xs {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBN = 256, kBK = 64;
// the epilogue's staging tile in LDS: output rows of 128 values, 16 bytes of padding a row (the two half-waves write
// rows 4 apart, which the padding puts 16 banks apart); f16 rows take a whole 128-row tile, fp32 rows 64 at a time
constexpr int kStageF16 = 128 * 2 + 16, kStageF32 = 128 * 4 + 16;
constexpr int kStageBytes = 128 * kStageF16 > 64 * kStageF32 ? 128 * kStageF16 : 64 * kStageF32;
// bytes of LDS before the routing entries of a down tile: the A double buffer or the staging tile, the larger
__host__ __device__ constexpr int entry_offset(int bm) { return 2 * bm * 128 > kStageBytes ? 2 * bm * 128 : kStageBytes; }
// weight rows a lane dequantizes: one for Q6_K down weights (their raw words take the registers that a 128-row tile
// needs), two otherwise (gate/up pairs a gate row with its up row)
__host__ __device__ constexpr int lane_rows(bool down, int t) { return down && t == kQ6_K ? 1 : 2; }
// row tiles of 32 a work-group: 4 for Q4_K and Q8_0 weights and Q6_K down weights, 2 where the weight words of two
// rows a lane take more registers (Q6_K gate/up, other formats)
__host__ __device__ constexpr int row_tiles(bool down, int t) {
    return t == kQ4_K || t == kQ8_0 || (down && t == kQ6_K) ? 4 : 2;
}

// x [n, H] fp32 -> f16 in the step order: thread i writes chunk i (8 values)
__global__ __launch_bounds__(256) void to_f16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                     int64_t n_chunks, int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n_chunks) to_f16_chunk(x, y, i, err);
}

// the m-tile table (tile_list) of the groups in bounds: one work-group, the groups 1024 at a time; each thread
// writes its group's tiles of both maps
__global__ __launch_bounds__(1024) void tile_map_kernel(const int32_t* __restrict__ bounds,
                                                        const int32_t* __restrict__ n_groups, int32_t* __restrict__ mt,
                                                        int64_t rows, int cap_groups) {
    __shared__ int s_wave[16][4];
    __shared__ int s_carry[4];
    const int ng = min(*n_groups, cap_groups);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t cap128 = tile_cap(rows, 128, cap_groups), cap64 = tile_cap(rows, 64, cap_groups);
    int32_t* l128 = tile_list(mt, rows, cap_groups, 128);
    int32_t* l64 = tile_list(mt, rows, cap_groups, 64);
    if (tid < 4) s_carry[tid] = 0;
    __syncthreads();
    for (int g0 = 0; g0 < max(ng, 0); g0 += 1024) {
        const int g = g0 + tid;
        const int start = g < ng ? bounds[g] : 0, n = g < ng ? bounds[g + 1] - start : 0;
        int c[4] = {n / 128, n % 128 ? 1 : 0, n / 64, n % 64 ? 1 : 0}, inc[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {   // inclusive wave scans of the four counts
            inc[m] = c[m];
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(inc[m], o, 64);
                if (lane >= o) inc[m] += y;
            }
            if (lane == 63) s_wave[wave][m] = inc[m];
        }
        __syncthreads();
        int before[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            before[m] = s_carry[m] + inc[m] - c[m];
            for (int w = 0; w < wave; ++w) before[m] += s_wave[w][m];
        }
        if (g < ng) {
            write_group_tiles(l128, g, start, n, 128, before[0], before[1], cap128);
            write_group_tiles(l64, g, start, n, 64, before[2], before[3], cap64);
        }
        __syncthreads();
        if (tid == 1023)
#pragma unroll
            for (int m = 0; m < 4; ++m) s_carry[m] = before[m] + c[m];
        __syncthreads();
    }
    if (tid < 4) mt[tid] = s_carry[tid];
}

// Loads through a global-address-space pointer.  Blob addresses come from memory (the group table), so the compiler
// cannot prove them global and would emit FLAT loads, which also count on lgkmcnt (every wait for an LDS operand
// would then wait for the weight prefetch in flight).  Q6_K blocks are 210 bytes, so their words are only 2-byte
// aligned: global loads take unaligned addresses on gfx9 (the HSA memory model's unaligned mode).
typedef unsigned int g32x4_t __attribute__((ext_vector_type(4), aligned(2)));
typedef unsigned int g32x2_t __attribute__((ext_vector_type(2), aligned(2)));
__device__ __forceinline__ uint4 ldg16(const void* p) {
    const g32x4_t v = *(const __attribute__((address_space(1))) g32x4_t*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldg8(const void* p) {
    const g32x2_t v = *(const __attribute__((address_space(1))) g32x2_t*)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ldg_u16(const void* p) {
    return *(const __attribute__((address_space(1))) uint16_t*)p;
}
__device__ __forceinline__ uint32_t ldg_u32(const void* p) {
    return *(const __attribute__((address_space(1))) uint32_t*)p;
}

// The standalone product's m-tile mt: the groups' tiles one after another, ceil(rows / bm) a group, groups ascending,
// found from the bounds alone (no table, no scratch).  Every wave walks the groups 256 at a time - each lane's bounds
// loads for four chunks of 64 in flight together - and scans each chunk's tile counts; the chunk that holds tile mt
// names its group by a ballot.  Rows past total_rows are cut off.  False when mt is past the last tile.
__device__ bool walk_tiles(const int32_t* __restrict__ bounds, int n, int64_t total_rows, int bm, int mt, int& g,
                           int& nrows, int& r0) {
    const int lane = threadIdx.x & 63;
    int carry = 0;
    for (int g0 = 0; g0 < n; g0 += 256) {
        int lo[4], hi[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int gg = g0 + 64 * u + lane;
            lo[u] = gg < n ? bounds[gg] : 0;
            hi[u] = gg < n ? bounds[gg + 1] : 0;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int top = (int)min((int64_t)hi[u], total_rows);
            const int cnt = top > lo[u] ? (top - lo[u] + bm - 1) / bm : 0;
            int inc = cnt;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(inc, o, 64);
                if (lane >= o) inc += y;
            }
            const int total = __shfl(inc, 63, 64);
            if (mt < carry + total) {
                const int l = __ffsll((long long)__ballot(carry + inc > mt)) - 1;
                const int first = __shfl(carry + inc - cnt, l, 64);
                g = g0 + 64 * u + l;
                r0 = __shfl(lo[u], l, 64) + (mt - first) * bm;
                nrows = min(bm, __shfl(top, l, 64) - r0);
                return true;
            }
            carry += total;
        }
    }
    return false;
}

__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// A work-group barrier over LDS only: the wave's LDS operations are complete, its global loads may still be in flight.
// (__syncthreads() is a release fence too, so it would wait for every load in flight - the prefetch of the steps
// ahead - before the barrier.)
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int N>
struct IntC {
    static constexpr int value = N;
};

// The 16-byte slot of chunk c of row r in a row-major LDS slab of 128-byte rows: c ^ swk(r).  A fragment read takes
// one chunk of 32 consecutive rows, served 16 lanes at a time from 64 banks: rows of one parity share a half of the
// banks, so the 8 even (odd) rows among 16 consecutive ones need 8 different keys - swk is a bijection of bits 1..3
// of r.  Its low bit is bit 3 of r, so the 4 even rows among 8 consecutive ones have keys of distinct high bits: a
// lane pair writing chunks (c, c ^ 1) of each of those rows (the tall tile's weight stores) is also conflict-free.
__device__ __forceinline__ int swk(int r) { return (((r >> 1) & 3) << 1) | ((r >> 3) & 1); }
__device__ __forceinline__ int swz(int r, int c) { return r * 8 + (c ^ swk(r)); }   // in 16-byte units

__device__ __forceinline__ h2_t h2(uint32_t w) { return __builtin_bit_cast(h2_t, w); }
__device__ __forceinline__ uint32_t u32(h2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ h2_t h2b(float v) {   // v rounded to f16, in both halves
    const _Float16 h = (_Float16)v;
    return (h2_t){h, h};
}
// (a & m) | o as one v_and_or_b32: the empty asm pins the result, else the compiler regroups nested ones into v_and,
// v_and, v_or3_b32 (an instruction more)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r = (a & m) | o;
    asm("" : "+v"(r));
    return r;
}

// a constant held in a VGPR: gfx9's three-operand forms (v_and_or_b32) take no literal, and with the mask and the
// magic as literals the compiler splits every v_and_or_b32 into an AND and an OR
template <uint32_t C>
__device__ __forceinline__ uint32_t vreg() {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "n"(C));
    return r;
}
// the masks and magic words of the code unpacking: index 0 places a code at bits [5:0] of each half (f16 1024 + q),
// index 1 at bits [9:4] (f16 16 + q / 4)
struct QConst {
    uint32_t nib[2];   // 4-bit code: 0x000F000F, 0x00F000F0
    uint32_t two[2];   // Q6_K 2-bit high part: 0x00300030, 0x03000300
    uint32_t mag[2];   // 0x64006400 (f16 1024), 0x4C004C00 (f16 16)
    uint32_t byte;     // 8-bit code: 0x00FF00FF
};
__device__ __forceinline__ QConst make_qconst() {
    QConst c;
    c.nib[0] = vreg<0x000F000Fu>();
    c.nib[1] = vreg<0x00F000F0u>();
    c.two[0] = vreg<0x00300030u>();
    c.two[1] = vreg<0x03000300u>();
    c.mag[0] = vreg<0x64006400u>();
    c.mag[1] = vreg<0x4C004C00u>();
    c.byte = vreg<0x00FF00FFu>();
    return c;
}

// ---------------------------------------------------------------- Q4_K
// Lane l (half hf = l / 32) of weight row r, step p of a block (values 64 p .. 64 p + 63): the qs word run
// D = qs[32 p + 16 hf, +16).  Fragment kk: kk 0, 1 the low nibbles of words (0, 1) / (2, 3) - sub-block 2 p; kk 2, 3
// their high nibbles - sub-block 2 p + 1.
struct Q4Step {
    h2_t dlo, clo, mlo;   // d1, -1024 d1, -m1 of sub-block 2 p
    h2_t dhi, chi, mhi;   // 4 d1, -64 d1, -m1 of sub-block 2 p + 1
};
__device__ __forceinline__ Q4Step q4k_step(const uint4& hdr, int p) {
    const float d = h2f((uint16_t)(hdr.x & 0xFFFFu)), dmin = h2f((uint16_t)(hdr.x >> 16));
    int s0, m0, s1, m1;
    q4k_sm(hdr.y, hdr.z, hdr.w, 2 * p, s0, m0);
    q4k_sm(hdr.y, hdr.z, hdr.w, 2 * p + 1, s1, m1);
    Q4Step s;
    s.dlo = h2b(d * (float)s0);
    s.clo = s.dlo * (h2_t){-1024.0f16, -1024.0f16};
    s.mlo = -h2b(dmin * (float)m0);
    const h2_t d1 = h2b(d * (float)s1);
    s.dhi = d1 * (h2_t){4.0f16, 4.0f16};
    s.chi = d1 * (h2_t){-64.0f16, -64.0f16};
    s.mhi = -h2b(dmin * (float)m1);
    return s;
}
__device__ __forceinline__ f16x8_t q4k_frag(const uint4& D, int kk, const Q4Step& s, const QConst& qc) {
    const uint32_t w0 = (kk & 1) ? D.z : D.x, w1 = (kk & 1) ? D.w : D.y;
    const bool hi = kk >= 2;
    const uint32_t m = qc.nib[hi], o = qc.mag[hi];
    const h2_t sc = hi ? s.dhi : s.dlo, c = hi ? s.chi : s.clo, mn = hi ? s.mhi : s.mlo;
    const uint32_t v[4] = {and_or(w0, m, o), and_or(w0 >> 8, m, o), and_or(w1, m, o), and_or(w1 >> 8, m, o)};
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = u32(__builtin_elementwise_fma(h2(v[i]), sc, c) + mn);
    return __builtin_bit_cast(f16x8_t, make_uint4(r[0], r[1], r[2], r[3]));
}

// ---------------------------------------------------------------- Q6_K
// Half n of a block (values 128 n .. 128 n + 127) is two steps t.  Lane hf of weight row r loads, once a half,
// L0 = ql[64 n + 16 hf, +16), L1 = ql[64 n + 32 + 16 hf, +16), Hq = qh[32 n + 16 hf, +16) and the half's 8 scales.
// Fragment kk of step t: ql words (0, 1) / (2, 3) of L0 (kk < 2) or L1 (kk >= 2) - low nibbles at t = 0, high at
// t = 1 - and qh words (0, 1) / (2, 3) of Hq, bits 2 f .. 2 f + 1 of each byte with f = 2 t + kk / 2; its 16 values
// share scale 4 t + 2 (kk / 2) + hf of the half.
struct Q6Raw {
    uint4 l0, l1, hq;
    uint2 sc;
    uint32_t d;
};
__device__ __forceinline__ void q6k_load(const uint8_t* blk, int n, int hf, Q6Raw& r, bool scales = true) {
    r.l0 = ldg16(blk + 64 * n + 16 * hf);
    r.l1 = ldg16(blk + 64 * n + 32 + 16 * hf);
    r.hq = ldg16(blk + 128 + 32 * n + 16 * hf);
    if (scales) {
        r.sc = ldg8(blk + 192 + 8 * n);
        r.d = ldg_u16(blk + 208);
    }
}
__device__ __forceinline__ h2_t q6k_scale_of(uint2 sc, uint32_t dbits, int t, int kk, int hf) {
    const int i = 4 * t + 2 * (kk >> 1) + hf;
    const uint32_t w = i < 4 ? sc.x : sc.y;
    const float s = h2f((uint16_t)dbits) * (float)(int8_t)((w >> (8 * (i & 3))) & 0xFFu);
    const h2_t v = h2b(s);
    return t ? v * (h2_t){4.0f16, 4.0f16} : v;
}
__device__ __forceinline__ h2_t q6k_scale(const Q6Raw& r, int t, int kk, int hf) {
    return q6k_scale_of(r.sc, r.d, t, kk, hf);
}
__device__ __forceinline__ f16x8_t q6k_frag(const Q6Raw& r, int t, int kk, h2_t sc, const QConst& qc) {
    const uint4& L = kk < 2 ? r.l0 : r.l1;
    const uint32_t l0 = (kk & 1) ? L.z : L.x, l1 = (kk & 1) ? L.w : L.y;
    const uint32_t q0 = (kk & 1) ? r.hq.z : r.hq.x, q1 = (kk & 1) ? r.hq.w : r.hq.y;
    const int sl = (kk >> 1) ? 2 : 4, sr = (kk >> 1) ? 6 : 4;   // the qh field to bits [5:4] (t 0) or [9:8] (t 1)
    const uint32_t ml = qc.nib[t], mh = qc.two[t], o = qc.mag[t];
    const uint32_t v[4] = {and_or(l0, ml, and_or(q0 << sl, mh, o)), and_or(l0 >> 8, ml, and_or(q0 >> sr, mh, o)),
                           and_or(l1, ml, and_or(q1 << sl, mh, o)), and_or(l1 >> 8, ml, and_or(q1 >> sr, mh, o))};
    const h2_t off = t ? (h2_t){-24.0f16, -24.0f16} : (h2_t){-1056.0f16, -1056.0f16};   // (q - 32) / 4, q - 32
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = u32((h2(v[i]) + off) * sc);
    return __builtin_bit_cast(f16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
}

// ---------------------------------------------------------------- Q8_0
// Step ks (64 values) is blocks 2 ks, 2 ks + 1 of the row; lane hf takes codes 16 hf .. 16 hf + 15 of each (one
// 16-byte load, 2-byte aligned) and the block's scale.  Fragment kk: block kk / 2, words (0, 1) / (2, 3) for kk % 2.
// A code q becomes the f16 1152 + q (its byte with the sign bit flipped dropped into 0x6400), q = h - 1152 exactly,
// and d q is rounded once - the bits of the reference's q * d (dequant.hpp:84-89) taken to f16.
__device__ __forceinline__ f16x8_t q8_frag(const uint4& Q, int kk, uint32_t dbits, const QConst& qc) {
    const uint32_t w0 = ((kk & 1) ? Q.z : Q.x) ^ 0x80808080u, w1 = ((kk & 1) ? Q.w : Q.y) ^ 0x80808080u;
    const uint32_t m = qc.byte, o = qc.mag[0];
    const uint32_t v[4] = {and_or(w0, m, o), and_or(w0 >> 8, m, o), and_or(w1, m, o), and_or(w1 >> 8, m, o)};
    const h2_t d = h2((dbits & 0xFFFFu) * 0x10001u);
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = u32((h2(v[i]) + (h2_t){-1152.0f16, -1152.0f16}) * d);
    return __builtin_bit_cast(f16x8_t, make_uint4(r[0], r[1], r[2], r[3]));
}

// ---------------------------------------------------------------- other formats (IQ4_XS, and Q8_0 at other K)
// values [o, o + 8) of the 32-value group g of the block at b, as the reference's host dequantizers give them
// (dequant.hpp:84-89 Q8_0, 283-299 IQ4_XS)
__device__ __forceinline__ void dequant8(int type, const uint8_t* b, int g, int o, float (&y)[8]) {
    if (type == kQ8_0) {
        const float d = rd_h(b);
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = (float)(int8_t)b[2 + o + j] * d;
    } else if (type == kQ4_K) {   // (dequant32's arithmetic for values o .. o + 7 of group g)
        const float d = rd_h(b), dmin = rd_h(b + 2);
        const uint8_t* q = b + 4;
        int sc, m;
        if (g < 4) {
            sc = q[g] & 63;
            m = q[g + 4] & 63;
        } else {
            sc = (q[g + 4] & 0x0F) | ((q[g - 4] >> 6) << 4);
            m = (q[g + 4] >> 4) | ((q[g] >> 6) << 4);
        }
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        const uint8_t* qs = b + 16 + 32 * (g / 2) + o;
        const int sh = 4 * (g % 2);
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = d1 * (float)((qs[j] >> sh) & 0x0F) - m1;
    } else if (type == kQ6_K) {
        const float d = rd_h(b + 208);
        const int n = g / 4, s = g % 4;
        const uint8_t* ql = b + 64 * n + 32 * (s & 1) + o;
        const uint8_t* qh = b + 128 + 32 * n + o;
        const float sd = d * (float)((const int8_t*)(b + 192 + 8 * n))[2 * s + o / 16];   // (o .. o + 7: one scale)
        const int nsh = 4 * (s >> 1), hsh = 2 * s;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            y[j] = sd * (float)((int)(((ql[j] >> nsh) & 0x0F) | (((qh[j] >> hsh) & 3) << 4)) - 32);
    } else {
        const float d = rd_h(b);
        const unsigned scales_h = (unsigned)(b[2] | (b[3] << 8));
        const int ls = ((b[4 + g / 2] >> (4 * (g % 2))) & 0x0F) | (((scales_h >> (2 * g)) & 3) << 4);
        const float dl = d * (float)(ls - 32);
        const uint8_t* qs = b + 8 + 16 * g + (o & 15);
        const int sh = o >= 16 ? 4 : 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = dl * (float)iq4nl_value((qs[j] >> sh) & 0x0F);
    }
}
__device__ __forceinline__ f16x8_t generic_frag(const uint8_t* brow, int type, int k0, int kk, int hf) {
    const int qk = block_values(type), bs = block_bytes(type);
    const int kv = k0 + 32 * (kk >> 1);
    float v[8];
    dequant8(type, brow + (int64_t)(kv / qk) * bs, (kv % qk) / 32, 16 * hf + 8 * (kk & 1), v);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = sat_f16x2(v[perm8(2 * i)], v[perm8(2 * i + 1)]);
    return __builtin_bit_cast(f16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
}

// RT DMA instructions of a wave: instruction i copies 16 bytes at src[i] + off of each lane to LDS dst + 1024 i
// (global_load_lds_dwordx4; a function of its own: in a lambda the LDS address-space cast breaks the host pass)
template <int RT>
__device__ __forceinline__ void dma_rows(const uint8_t* const* src, size_t off, uint8_t* dst) {
#pragma unroll
    for (int i = 0; i < RT; ++i)
        __builtin_amdgcn_global_load_lds(src[i] + off, (__attribute__((address_space(3))) void*)(dst + i * 1024), 16, 0,
                                         0);
}

template <bool DOWN, int T, int RT, bool MMQ = false>
__global__ __launch_bounds__(256, 2) void grouped_mfma_kernel(ExpertLayout L, PrefillArgs a,
                                                              const int32_t* __restrict__ mtile, int mt_bound,
                                                              int n_tiles, int by_n) {
    constexpr int kBM = 32 * RT;
    constexpr int J = lane_rows(DOWN, T), BN = 128 * J;   // weight rows a lane; weight rows (output columns) a tile
    static_assert(DOWN || J == 2, "gate/up pairs a gate row with its up row in each lane");
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hf = lane >> 5;
    // work-group b runs on XCD x = b % 8.  With by_n (n-tiles a multiple of 8), XCD x takes n-tiles [x n8, x n8 + n8)
    // of every m-tile, m-tile by m-tile: the weight slice of its n-tiles is fetched into its L2 once an expert and
    // reused by the expert's m-tiles.  Otherwise XCD x takes m-tiles x, x + 8, ..., each with its n-tiles one after
    // the other, so the m-tile's activations are fetched into its L2 once (the better order where groups hold one or
    // two m-tiles, as the rows past the tall tiles do).
    const int c8 = (int)(blockIdx.x >> 3), xcd = (int)(blockIdx.x & 7);
    int mt, nt;
    if (by_n) {
        const int n8 = n_tiles >> 3;
        mt = c8 / n8;
        nt = xcd * n8 + c8 % n8;
    } else {
        mt = (c8 / n_tiles) * 8 + xcd;
        nt = c8 % n_tiles;
    }
    if (mt >= mt_bound) return;
    int g, nrows, r0;
    if constexpr (MMQ) {
        if (!walk_tiles(a.bounds, (int)a.cap_groups, a.n_tok, kBM, mt, g, nrows, r0)) return;
    } else {
        const int ng = *a.n_groups;
        const int nfull = mtile[kBM == 128 ? 0 : 2], npart = mtile[kBM == 128 ? 1 : 3];
        if (ng <= 0 || mt >= nfull + npart) return;
        const int64_t te = mt < nfull ? mt : mt_bound - 1 - (mt - nfull);   // the tile's entry (tile_list)
        const int32_t* tl = tile_list(const_cast<int32_t*>(mtile), a.rows, a.cap_groups, kBM) + 2 * te;
        g = tl[0] & 0xFFFF;
        nrows = tl[0] >> 16;
        r0 = tl[1];
    }
    const int nrt = (nrows + 31) >> 5;   // live 32-row tiles
    const int H = (int)L.n_embd, F = (int)L.n_ff;
    const int K = DOWN ? F : H;
    const int nk = K / kBK;
    const int n0 = nt * (DOWN ? BN : kBN / 2);
    const int64_t wrb = DOWN ? L.d_row : L.gu_row;

    // A by DMA: wave w fills rows [8 RT w, 8 RT (w + 1)) of the tile, 8 rows an instruction; lane l of instruction i
    // holds LDS slot swz(R, l & 7) of row R = 8 RT w + 8 i + l / 8, i.e. chunk (l & 7) ^ swk(R) of that row (rows
    // past the group's end read its first row)
    // (MMQ: the chunk's 8 int8 codes - values 8 perm8(c) .. + 8 of the step - and their block's scale instead)
    const uint8_t* asrc[RT];
    const uint8_t* adsc[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        const int R = 8 * RT * wave + 8 * i + (lane >> 3);
        const int rr = R < nrows ? R : 0;
        const int c = (lane & 7) ^ swk(R);
        if constexpr (MMQ) {
            asrc[i] = (const uint8_t*)(a.xq + (int64_t)(r0 + rr) * K) + 8 * perm8(c);
            adsc[i] = (const uint8_t*)((const float*)(a.xq + a.n_tok * K) + (int64_t)(r0 + rr) * (K / 32) + perm8(c) / 4);
        } else {
            asrc[i] = (const uint8_t*)(DOWN ? a.h + (int64_t)(r0 + rr) * F : a.xb + (int64_t)a.src[r0 + rr] * H) +
                      16 * c;
            adsc[i] = nullptr;
        }
    }
    // a chunk of A step ks as loaded (f16, or MMQ's codes and scale), and as written to LDS (f16: the codes times the
    // scale rounded to f16, saturated, in the slot order - the bits of a saturated f16 copy of xq)
    auto a_load = [&](int i, int ks) -> uint4 {
        if constexpr (MMQ) {
            const uint2 q = ldg8(asrc[i] + (size_t)ks * 64);
            return make_uint4(q.x, q.y, ldg_u32(adsc[i] + (size_t)ks * 8), 0u);
        } else {
            return ldg16(asrc[i] + (size_t)ks * 128);
        }
    };
    auto a_f16 = [&](const uint4& r) -> uint4 {
        if constexpr (MMQ) {
            const float d = __uint_as_float(r.z);
            float v[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = (float)(int8_t)(((t < 4 ? r.x : r.y) >> (8 * (t & 3))) & 0xFFu) * d;
            return make_uint4(sat_f16x2(v[0], v[2]), sat_f16x2(v[1], v[3]), sat_f16x2(v[4], v[6]),
                              sat_f16x2(v[5], v[7]));
        } else {
            return r;
        }
    };
    // down: the routing entry of each row, staged in LDS for the epilogue (visible after the first step's barrier)
    int32_t* const s_entry = (int32_t*)(lds + entry_offset(kBM));
    if (DOWN && tid < nrows) s_entry[tid] = a.entry[r0 + tid];
    // the A rows of step ks into buffer `buf`
    auto dma_a = [&](int ks, int buf) {
        dma_rows<RT>(asrc, (size_t)ks * 128, lds + buf * (kBM * 128) + wave * 8 * RT * 128);
    };
    // B: the lane's J weight rows (tile columns cb[j] + lane % 32); gate/up pairs a gate column with its up column
    int cb[J];
#pragma unroll
    for (int j = 0; j < J; ++j) cb[j] = DOWN ? 32 * J * wave + 32 * j : (j ? 128 + 32 * wave : 32 * wave);
    // (gate/up: a gate row at wrow * gu_row, an up row at up_off + wrow * up_row - the same place as row F + wrow of
    // one matrix when the up rows are of the gate's type; wtype[j] the row's type, which the generic path reads)
    const uint8_t* brow[J];
    int wtype[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int col = cb[j] + (lane & 31);
        const bool up = !DOWN && col >= kBN / 2;
        const int wrow = DOWN ? n0 + col : up ? n0 + (col - kBN / 2) : n0 + col;
        const uint8_t* wb;
        if constexpr (MMQ) wb = a.wtab ? a.wtab[g] + a.woff : a.wbase + (size_t)g * a.wstride;
        else wb = (const uint8_t*)a.wptr[g];
        brow[j] = DOWN ? wb + L.down_off + (int64_t)wrow * wrb
                       : up ? wb + L.up_off + (int64_t)wrow * (L.up_row ? L.up_row : wrb) : wb + (int64_t)wrow * wrb;
        wtype[j] = DOWN ? L.d_type : up && L.up_type >= 0 ? L.up_type : L.gu_type;
    }

    f32x16_t acc[RT][J];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

    // a step's start: its A rows and raw weights (issued a step before) have landed in every wave
    auto step_sync = [&]() {
        vm_drain();
        __syncthreads();
    };
    const QConst qc = make_qconst();

    // The K loop for NRT live row tiles, a compile-time count: a fragment's operand reads and MFMAs are then
    // straight-line code that the scheduler interleaves with the next fragment's dequantization.
    auto kloop = [&](auto nrt_c) {
        constexpr int NRT = decltype(nrt_c)::value;
        // down: a wave whose A rows hold no live row tile neither loads nor stages them (its share of the step's loads
        // was a fifth of a small tile's TA address cycles; for gate/up the same skip measured slower)
        const bool a_live = !DOWN || NRT == RT || RT * wave < 4 * NRT;
        // fragment kk of step ks: the B fragments fb[0 .. J) against the live row tiles of the step's A buffer
        auto mfma_step = [&](int ks, int kk, const f16x8_t (&fb)[J]) {
            const uint4* sA = (const uint4*)(lds + (ks & 1) * (kBM * 128));
            const int ch = 2 * kk + hf;
            f16x8_t fa[NRT];
#pragma unroll
            for (int i = 0; i < NRT; ++i) fa[i] = __builtin_bit_cast(f16x8_t, sA[swz(32 * i + (lane & 31), ch)]);
#pragma unroll
            for (int i = 0; i < NRT; ++i)
#pragma unroll
                for (int j = 0; j < J; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        };
        if (T == kQ4_K) {
            // The A rows of step ks + 1 go through registers (loaded at the start of step ks, written to LDS at its
            // end), not by LDS DMA: a DMA in flight makes the compiler wait for every load (vmcnt(0)) before the
            // step's first LDS read, which would serialise each step with its own prefetch.
            uint4 areg[RT];
            auto load_a = [&](int ks) {
                if (a_live)
#pragma unroll
                    for (int i = 0; i < RT; ++i) areg[i] = a_load(i, ks);
            };
            auto store_a = [&](int buf) {
                uint8_t* dst = lds + buf * (kBM * 128) + wave * 8 * RT * 128 + 16 * lane;
                if (a_live)
#pragma unroll
                    for (int i = 0; i < RT; ++i) *(uint4*)(dst + i * 1024) = a_f16(areg[i]);
            };
            const int nb = K / 256;
            uint4 hdr[J], q[2][J];   // header of the block; the qs run of steps (even, odd)
            load_a(0);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                hdr[j] = ldg16(brow[j]);
                q[0][j] = ldg16(brow[j] + 16 + 16 * hf);
            }
            store_a(0);
            for (int b = 0; b < nb; ++b) {
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int ks = 4 * b + p;
                    lds_sync();   // A(ks) is in buffer ks & 1; step ks - 1 is done with the other
                    // the step's scales first: at p = 3 the header registers then take the next block's header
                    Q4Step sj[J];
#pragma unroll
                    for (int j = 0; j < J; ++j) sj[j] = q4k_step(hdr[j], p);
                    // the next step's loads, with no branch (the last step reloads its own block and A rows): a branch
                    // around them would make the compiler's waits for the current words wait for these too
                    load_a(min(ks + 1, nk - 1));
                    const int bn = min(p == 3 ? b + 1 : b, nb - 1);   // the next step's block
#pragma unroll
                    for (int j = 0; j < J; ++j) {
                        const uint8_t* blk = brow[j] + 144 * bn;
                        if (p == 3) hdr[j] = ldg16(blk);
                        q[(p + 1) & 1][j] = ldg16(blk + 16 + 32 * ((p + 1) & 3) + 16 * hf);
                    }
                    __builtin_amdgcn_sched_barrier(0);   // the loads stay ahead of the step's products
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        f16x8_t fb[J];
#pragma unroll
                        for (int j = 0; j < J; ++j) fb[j] = q4k_frag(q[p & 1][j], kk, sj[j], qc);
                        mfma_step(ks, kk, fb);
                    }
                    store_a((ks + 1) & 1);   // after the last step no one reads it
                }
            }
        } else if (T == kQ6_K) {
            // K is short here (n_ff: 12 steps at 768), so the loads of a step must be in flight two steps ahead.  The
            // A tile goes through registers (loaded at the start of step ks - 2, written to LDS at the end of step
            // ks - 1) rather than by LDS DMA: the wait for a register load is the compiler's own and exact, while a
            // wait for "all but the newest n" on vmcnt cannot single out LDS DMA among ordinary loads.  The raw words of a half are loaded at the
            // first step of the half before.  With 3 blocks a row (n_ff 768) everything is straight-line code.
            uint4 areg[2][RT];   // A(ks) staging, slot ks & 1
            auto load_a = [&](int ks, int slot) {
                if (a_live)
#pragma unroll
                    for (int i = 0; i < RT; ++i) areg[slot][i] = a_load(i, ks);
            };
            auto store_a = [&](int slot, int buf) {
                uint8_t* dst = lds + buf * (kBM * 128) + wave * 8 * RT * 128 + 16 * lane;
                if (a_live)
#pragma unroll
                    for (int i = 0; i < RT; ++i) *(uint4*)(dst + i * 1024) = a_f16(areg[slot][i]);
            };
            auto q6loop = [&](auto nbc) {
                constexpr int NBC = decltype(nbc)::value;
                const int nb = NBC > 0 ? NBC : K / 256;
                Q6Raw r[2][J];   // the raw words of halves (even, odd), per row
                // with the block count known (fully unrolled), a block's 16 scales and d are loaded once (one 16-byte
                // and one 2-byte load a lane, slot block & 1) rather than a half's 8 scales and d with every half:
                // two fewer 32-row loads a block for the lanes' address path
                uint4 scb[2][J];
                uint32_t db[2][J];
                load_a(0, 0);
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    q6k_load(brow[j], 0, hf, r[0][j], NBC == 0);
                    if constexpr (NBC > 0) {
                        scb[0][j] = ldg16(brow[j] + 192);
                        db[0][j] = ldg_u16(brow[j] + 208);
                    }
                }
                load_a(1, 1);
                store_a(0, 0);
#pragma unroll
                for (int b = 0; b < nb; ++b) {
#pragma unroll
                    for (int n = 0; n < 2; ++n) {
#pragma unroll
                        for (int t = 0; t < 2; ++t) {
                            const int ks = 4 * b + 2 * n + t;
                            lds_sync();   // A(ks) is in buffer ks & 1; step ks - 1 is done with the other
                            if (ks + 2 < nk) load_a(ks + 2, ks & 1);   // (slot ks & 1 went to LDS last step)
                            if (t == 0 && 2 * b + n + 1 < 2 * nb) {   // the next half's words
                                const int h1 = 2 * b + n + 1;
#pragma unroll
                                for (int j = 0; j < J; ++j) {
                                    const uint8_t* blk = brow[j] + 210 * (h1 >> 1);
                                    q6k_load(blk, h1 & 1, hf, r[n ^ 1][j], NBC == 0);
                                    if constexpr (NBC > 0)
                                        if ((h1 & 1) == 0) {   // the next block's scales
                                            scb[(h1 >> 1) & 1][j] = ldg16(blk + 192);
                                            db[(h1 >> 1) & 1][j] = ldg_u16(blk + 208);
                                        }
                                }
                            }
#pragma unroll
                            for (int kk = 0; kk < 4; ++kk) {
                                f16x8_t fb[J];
#pragma unroll
                                for (int j = 0; j < J; ++j) {
                                    h2_t sc;
                                    if constexpr (NBC > 0) {
                                        const uint4& q = scb[b & 1][j];
                                        sc = q6k_scale_of(n ? make_uint2(q.z, q.w) : make_uint2(q.x, q.y), db[b & 1][j],
                                                          t, kk, hf);
                                    } else {
                                        sc = q6k_scale(r[n][j], t, kk, hf);
                                    }
                                    fb[j] = q6k_frag(r[n][j], t, kk, sc, qc);
                                }
                                mfma_step(ks, kk, fb);
                            }
                            // A(ks + 1), loaded a step ago, into the buffer step ks - 1 read: at the step's end, so
                            // that its loads have two steps to land
                            if (ks + 1 < nk) store_a((ks + 1) & 1, (ks + 1) & 1);
                        }
                    }
                }
            };
            if (K == 768) q6loop(IntC<3>{});
            else q6loop(IntC<0>{});
        } else if (T == kQ8_0) {
            // the Q4_K path's pipeline: A rows and raw words of step ks + 1 loaded at the start of step ks with no
            // branch, A written to LDS at its end; steps in pairs so the word registers are named statically
            uint4 areg[RT];
            auto load_a = [&](int ks) {
#pragma unroll
                for (int i = 0; i < RT; ++i) areg[i] = a_load(i, ks);
            };
            auto store_a = [&](int buf) {
                uint8_t* dst = lds + buf * (kBM * 128) + wave * 8 * RT * 128 + 16 * lane;
#pragma unroll
                for (int i = 0; i < RT; ++i) *(uint4*)(dst + i * 1024) = a_f16(areg[i]);
            };
            uint4 qv[2][2][J];       // codes of (step parity, block of the step, row)
            uint32_t dv[2][2][J];    // their blocks' scales (f16 bits)
            auto load_w = [&](int ks, auto slot_c) {
                constexpr int SL = decltype(slot_c)::value;
#pragma unroll
                for (int j = 0; j < J; ++j)
#pragma unroll
                    for (int bb = 0; bb < 2; ++bb) {
                        const uint8_t* blk = brow[j] + 34 * (2 * ks + bb);
                        qv[SL][bb][j] = ldg16(blk + 2 + 16 * hf);
                        dv[SL][bb][j] = ldg_u16(blk);
                    }
            };
            auto q8_step = [&](int ks, auto slot_c) {
                constexpr int SL = decltype(slot_c)::value;
                lds_sync();   // A(ks) is in buffer ks & 1; step ks - 1 is done with the other
                const int kn = min(ks + 1, nk - 1);
                load_a(kn);
                load_w(kn, IntC<SL ^ 1>{});
                __builtin_amdgcn_sched_barrier(0);   // the loads stay ahead of the step's products
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    f16x8_t fb[J];
#pragma unroll
                    for (int j = 0; j < J; ++j) fb[j] = q8_frag(qv[SL][kk >> 1][j], kk, dv[SL][kk >> 1][j], qc);
                    mfma_step(ks, kk, fb);
                }
                store_a((ks + 1) & 1);   // after the last step no one reads it
            };
            load_a(0);
            load_w(0, IntC<0>{});
            store_a(0);
            for (int ks = 0; ks < nk; ks += 2) {   // nk is even (K % 128 == 0 for this instance)
                q8_step(ks, IntC<0>{});
                q8_step(ks + 1, IntC<1>{});
            }
        } else if constexpr (MMQ) {
            // other formats over MMQ rows: each step's A chunks loaded, converted and written to LDS, then its products
            for (int ks = 0; ks < nk; ++ks) {
                uint4 r[RT];
#pragma unroll
                for (int i = 0; i < RT; ++i) r[i] = a_load(i, ks);
                uint8_t* dst = lds + (ks & 1) * (kBM * 128) + wave * 8 * RT * 128 + 16 * lane;
#pragma unroll
                for (int i = 0; i < RT; ++i) *(uint4*)(dst + i * 1024) = a_f16(r[i]);
                lds_sync();
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    f16x8_t fb[J];
#pragma unroll
                    for (int j = 0; j < J; ++j) fb[j] = generic_frag(brow[j], wtype[j], ks * kBK, kk, hf);
                    mfma_step(ks, kk, fb);
                }
            }
        } else {
            dma_a(0, 0);
            for (int ks = 0; ks < nk; ++ks) {
                step_sync();
                if (ks + 1 < nk) dma_a(ks + 1, (ks + 1) & 1);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    f16x8_t fb[J];
#pragma unroll
                    for (int j = 0; j < J; ++j) fb[j] = generic_frag(brow[j], wtype[j], ks * kBK, kk, hf);
                    mfma_step(ks, kk, fb);
                }
            }
        }
    };
    if (nrt >= RT) kloop(IntC<RT>{});
    else if (RT > 3 && nrt == 3) kloop(IntC<(RT > 3 ? 3 : 1)>{});
    else if (RT > 2 && nrt == 2) kloop(IntC<(RT > 2 ? 2 : 1)>{});
    else kloop(IntC<1>{});

    // Epilogue.  Lane holds C[32 i + 8 (q / 4) + 4 (lane / 32) + q % 4][cb[j] + lane % 32].  The values go through a
    // row-major staging tile in LDS, so that every global store is 16 contiguous bytes of an output row: down rows
    // scatter by routing entry, h rows are the tile's own.  Staging column sc = 32 wave + lane % 32 of pass j is
    // output column cb[j] + lane % 32 (down), or h column n0 + sc at its place in the step order (gate/up).
    lds_sync();   // every wave is done with the A buffers
    const bool f32out = DOWN && !a.parts_h;
    const int esz = f32out ? 4 : 2, stride = f32out ? kStageF32 : kStageF16, rpp = f32out ? 64 : 128;
    const int cpr = 128 * esz / 16;   // 16-byte chunks a staged row
    const int sc = 32 * wave + (lane & 31);
    const int spos = DOWN ? sc : (sc & ~63) + perm64(sc & 63);
    bool sat = false;   // a value saturated to the f16 range
#pragma unroll
    for (int j = 0; j < (DOWN ? J : 1); ++j) {
        for (int rb = 0; rb < 32 * nrt; rb += rpp) {
#pragma unroll
            for (int i = 0; i < RT; ++i) {
                if (i >= nrt || 32 * i < rb || 32 * i >= rb + rpp) continue;
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int row = 32 * i + 8 * (q >> 2) + 4 * hf + (q & 3);
                    uint8_t* dst = lds + (row - rb) * stride + spos * esz;
                    if (DOWN) {
                        const float v = acc[i][j][q];
                        if (f32out) {
                            *(float*)dst = v;
                        } else {
                            sat |= past_f16(v);
                            *(uint16_t*)dst = f2h(__builtin_fminf(__builtin_fmaxf(v, -65504.0f), 65504.0f));
                        }
                    } else {
                        // SwiGLU on the hardware exp2 and reciprocal (the f16 path's tolerance, not canon's bits)
                        const float gv = acc[i][0][q], uv = acc[i][J - 1][q];
                        const float e = __builtin_amdgcn_exp2f(-gv * 1.4426950408889634f);
                        float hv = gv * __builtin_amdgcn_rcpf(1.0f + e) * uv;
                        sat |= past_f16(hv);
                        hv = __builtin_fminf(__builtin_fmaxf(hv, -65504.0f), 65504.0f);
                        *(uint16_t*)dst = f2h(hv);
                    }
                }
            }
            lds_sync();
            const int nr = min(rpp, nrows - rb);
            for (int idx = tid; idx < nr * cpr; idx += 256) {
                const int r = idx / cpr, c = idx - r * cpr, row = rb + r;
                const uint4 v = *(const uint4*)(lds + r * stride + 16 * c);
                const int scol = c * (16 / esz);   // the chunk's first staged column
                if (DOWN) {
                    const int w = scol >> 5;
                    const int col = (J == 1 ? 32 * w : 64 * w + 32 * j) + (scol & 31);
                    const int64_t o = (int64_t)s_entry[row] * a.ld_parts + n0 + col;
                    if (f32out) *(uint4*)(a.parts + o) = v;
                    else *(uint4*)(a.parts_h + o) = v;
                } else {
                    *(uint4*)(a.h + (int64_t)(r0 + row) * F + n0 + scol) = v;
                }
            }
            lds_sync();   // the next pass writes the staging tile again
        }
    }
    if (sat && a.err) atomicOr(a.err, kSatBit);
}

// ---------------------------------------------------------------- tall tiles
// A whole 256-row tile of one group against BN weight rows (gate/up: BN / 2 gate rows and their up rows, so BN / 2 h
// columns; down: BN output columns), by 8 waves, two a SIMD.  Each K step (64 values) the
// work-group dequantizes the step's BN x 64 weight slab once into LDS (512 / BN threads a weight row, each a share of
// the row's 8 fragments) and stages the 256 x 64 activation slab, both double-buffered; wave w then multiplies rows
// [64 (w % 4), + 64) by BN / 2 weight rows of the tile (gate/up: BN / 4 gate rows and their up rows), so a dequantized
// fragment feeds 8 products (a 64-row tile's lane-held fragments feed 2 to 4).  The raw words of step ks + 2 and
// the activation rows of step ks + 1 are loaded at the start of step ks; step ks + 1 is dequantized and staged while
// step ks's products run (the A rows stored halfway, which frees their registers for the second half's products),
// one barrier a step.  Work-group b runs on XCD b % 8; XCD x takes tall tiles x, x + 8, ...
// and runs each one's n-tiles side by side, so the tile's activations reach its L2 once.
constexpr int kTallSlab = 256 * 128;   // one activation buffer: 256 rows x 64 f16 values
__host__ __device__ constexpr int tall_lds(int bn) { return 2 * kTallSlab + 2 * bn * 128; }

template <bool DOWN, int T, int BN>
__global__ __launch_bounds__(512) void tall_mfma_kernel(ExpertLayout L, PrefillArgs a, const int32_t* __restrict__ tall,
                                                        int n_tiles) {
    static_assert(T == kQ4_K || T == kQ6_K, "tall tiles take Q4_K and Q6_K weights");
    static_assert(BN == 128 || BN == 256, "a tile is 128 or 256 weight rows");
    constexpr int TPC = 512 / BN;     // threads a weight row
    constexpr int NF = 8 / TPC;       // fragments a thread dequantizes a step
    constexpr int JW = BN / 64;       // 32-column MFMA tiles a wave
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hf = lane >> 5;
    const int c8 = (int)(blockIdx.x >> 3), xcd = (int)(blockIdx.x & 7);
    const int mt = (c8 / n_tiles) * 8 + xcd, nt = c8 % n_tiles;
    if (*a.n_groups <= 0 || mt >= tall[0]) return;   // (no groups: the route refused the ids and wrote no table)
    const int g = tall[1 + 2 * mt], r0 = tall[2 + 2 * mt];
    if (g >= *a.n_groups || r0 < 0 || r0 + 256 > a.rows) return;
    const int H = (int)L.n_embd, F = (int)L.n_ff;
    const int K = DOWN ? F : H, nk = K / kBK;   // nk % 4 == 0 (K is whole 256-value blocks)
    const int n0 = nt * (DOWN ? BN : BN / 2);
    uint8_t* const sA = lds;
    uint8_t* const sB = lds + 2 * kTallSlab;
    int32_t* const s_entry = (int32_t*)(lds + tall_lds(BN));
    if (DOWN && tid < 256) s_entry[tid] = a.entry[r0 + tid];

    // A: thread t stages rows 64 i + t / 8 (i < 4), slot t % 8 of each: chunk (t % 8) ^ swk(row) of the row (byte
    // offsets from abase: the f16 activations are far below 4 GB)
    const uint8_t* const abase = (const uint8_t*)(DOWN ? a.h : a.xb);
    uint32_t aoff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int R = 64 * i + (tid >> 3);
        const int c = (tid & 7) ^ swk(R);
        aoff[i] = (uint32_t)(DOWN ? (r0 + R) * F : a.src[r0 + R] * H) * 2u + 16u * c;
    }
    // B: thread t dequantizes weight row cw = t / TPC of the tile, lane half hb = t % 2 of the raw words, and of the
    // row's fragments 2 kk + hb those with kk = 2 kp + f (f < NF; kp = t / 2 % 2 when TPC = 4, else kk = f)
    const int cw = tid / TPC, hb = tid & 1, kp = TPC == 4 ? (tid >> 1) & 1 : 0;
    const int wrow = DOWN ? n0 + cw : (cw < BN / 2 ? n0 + cw : F + n0 + (cw - BN / 2));
    const uint8_t* const brow = (const uint8_t*)a.wptr[g] + (DOWN ? L.down_off : 0) +
                                (int64_t)wrow * (DOWN ? L.d_row : L.gu_row);
    uint8_t* const bdst = sB + cw * 128;
    const int bsw = swk(cw);

    // wave tile: rows 64 wm + 32 i (i < 2), weight columns cb[j] (j < JW)
    const int wm = wave & 3, wn = wave >> 2;
    int cb[JW];
#pragma unroll
    for (int j = 0; j < JW; ++j)
        cb[j] = DOWN ? (BN / 2) * wn + 32 * j
                     : (j < JW / 2 ? (BN / 4) * wn + 32 * j : BN / 2 + (BN / 4) * wn + 32 * (j - JW / 2));
    f32x16_t acc[2][JW];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < JW; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
    // the code-unpacking constants: masks uniform (SGPRs: one scalar operand a v_and_or_b32), magic words in VGPRs
    QConst qc;
    qc.nib[0] = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    qc.nib[1] = __builtin_amdgcn_readfirstlane(0x00F000F0u);
    qc.two[0] = __builtin_amdgcn_readfirstlane(0x00300030u);
    qc.two[1] = __builtin_amdgcn_readfirstlane(0x03000300u);
    qc.byte = __builtin_amdgcn_readfirstlane(0x00FF00FFu);
    qc.mag[0] = vreg<0x64006400u>();
    qc.mag[1] = vreg<0x4C004C00u>();

    uint4 areg[4];   // A rows of the next step
    auto load_a = [&](int s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) areg[i] = ldg16(abase + aoff[i] + (size_t)s * 128);
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *(uint4*)(sA + buf * kTallSlab + i * 8192 + tid * 16) = areg[i];
    };
    // raw weights.  Q4_K: the step's 16 qs bytes (slot step & 1) and the block header (hnext, moved to hcur when the
    // block's first step is dequantized).  Q6_K: a half block's words (slot half & 1), loaded at odd steps for the
    // half three steps on; with TPC = 4 only the ql run of the thread's kp (in l0).
    uint4 qraw[2], hcur, hnext;
    Q6Raw r6[2];
    auto load_b = [&](int s, auto slot_c, auto p_c) {   // Q4_K: step s (its position p in the block)
        constexpr int SL = decltype(slot_c)::value, P = decltype(p_c)::value;
        const uint8_t* blk = brow + 144 * (s >> 2);
        qraw[SL] = ldg16(blk + 16 + 32 * P + 16 * hb);
        if (P == 0) hnext = ldg16(blk);
    };
    auto load_q6 = [&](int hh, Q6Raw& r) {   // half hh of the row
        const uint8_t* blk = brow + 210 * (hh >> 1);
        const int n = hh & 1;
        if constexpr (TPC == 2) {
            q6k_load(blk, n, hb, r);
        } else {
            r.l0 = ldg16(blk + 64 * n + 32 * kp + 16 * hb);
            r.hq = ldg16(blk + 128 + 32 * n + 16 * hb);
            r.sc = ldg8(blk + 192 + 8 * n);
            r.d = ldg_u16(blk + 208);
        }
    };
    // fragment f of step s (position p in its block; Q4_K: the block's header hdr) into B buffer buf
    auto dequant = [&](int f, int buf, auto slot_c, auto p_c, const uint4& hdr) {
        constexpr int SL = decltype(slot_c)::value, P = decltype(p_c)::value;
        const int kk = TPC == 2 ? f : 2 * kp + f;
        f16x8_t v;
        if constexpr (T == kQ4_K) {
            if constexpr (TPC == 2) {
                v = q4k_frag(qraw[SL], f, q4k_step(hdr, P), qc);
            } else {   // sub-block 2 p + kp: low nibbles (kp 0) or high (kp 1) of words (0, 1) / (2, 3)
                const float d = h2f((uint16_t)(hdr.x & 0xFFFFu)), dmin = h2f((uint16_t)(hdr.x >> 16));
                int sv, mv;
                q4k_sm(hdr.y, hdr.z, hdr.w, 2 * P + kp, sv, mv);
                const h2_t d1 = h2b(d * (float)sv);
                const h2_t sc = kp ? d1 * (h2_t){4.0f16, 4.0f16} : d1;
                const h2_t c = kp ? d1 * (h2_t){-64.0f16, -64.0f16} : d1 * (h2_t){-1024.0f16, -1024.0f16};
                const h2_t mn = -h2b(dmin * (float)mv);
                const uint32_t m = kp ? qc.nib[1] : qc.nib[0], o = kp ? qc.mag[1] : qc.mag[0];
                const uint4& D = qraw[SL];
                const uint32_t w0 = (f & 1) ? D.z : D.x, w1 = (f & 1) ? D.w : D.y;
                const uint32_t u[4] = {and_or(w0, m, o), and_or(w0 >> 8, m, o), and_or(w1, m, o),
                                       and_or(w1 >> 8, m, o)};
                uint32_t r[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] = u32(__builtin_elementwise_fma(h2(u[i]), sc, c) + mn);
                v = __builtin_bit_cast(f16x8_t, make_uint4(r[0], r[1], r[2], r[3]));
            }
        } else {
            const int t = P & 1;
            if constexpr (TPC == 2) {
                v = q6k_frag(r6[SL], t, f, q6k_scale(r6[SL], t, f, hb), qc);
            } else {   // ql words of the kp run (in l0), qh bits 2 (2 t + kp) of each byte
                const Q6Raw& r = r6[SL];
                const uint32_t l0 = (f & 1) ? r.l0.z : r.l0.x, l1 = (f & 1) ? r.l0.w : r.l0.y;
                const uint32_t q0 = (f & 1) ? r.hq.z : r.hq.x, q1 = (f & 1) ? r.hq.w : r.hq.y;
                const int sl = kp ? 2 : 4, sr = kp ? 6 : 4;
                const uint32_t ml = qc.nib[t], mh = qc.two[t], o = qc.mag[t];
                const uint32_t u[4] = {and_or(l0, ml, and_or(q0 << sl, mh, o)),
                                       and_or(l0 >> 8, ml, and_or(q0 >> sr, mh, o)),
                                       and_or(l1, ml, and_or(q1 << sl, mh, o)),
                                       and_or(l1 >> 8, ml, and_or(q1 >> sr, mh, o))};
                const int si = 2 * kp + hb;   // scale 4 t + si of the half
                const uint32_t sw = t ? r.sc.y : r.sc.x;
                const h2_t s1 = h2b(h2f((uint16_t)r.d) * (float)(int8_t)((sw >> (8 * si)) & 0xFFu));
                const h2_t sc = t ? s1 * (h2_t){4.0f16, 4.0f16} : s1;
                const h2_t off = t ? (h2_t){-24.0f16, -24.0f16} : (h2_t){-1056.0f16, -1056.0f16};
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) w[i] = u32((h2(u[i]) + off) * sc);
                v = __builtin_bit_cast(f16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
            }
        }
        *(f16x8_t*)(bdst + buf * (BN * 128) + 16 * ((2 * kk + hb) ^ bsw)) = v;
    };
    // prologue: step 0 staged, the raw weights of step 1 loaded
    load_a(0);
    if constexpr (T == kQ4_K) {
        hcur = ldg16(brow);
        load_b(0, IntC<0>{}, IntC<0>{});
        load_b(1, IntC<1>{}, IntC<1>{});
    } else {
        load_q6(0, r6[0]);
        load_q6(1, r6[1]);
    }
    store_a(0);
#pragma unroll
    for (int f = 0; f < NF; ++f) dequant(f, 0, IntC<0>{}, IntC<0>{}, hcur);
    lds_sync();

    // iteration ks = ks0 + U: products of step ks (buffer U & 1), step ks + 1 staged into the other buffer (its
    // weights dequantized between the products, its A rows - loaded at the iteration's start - stored halfway).  The
    // last iteration (LAST) stages nothing; no other branch is taken in the loop, so the compiler's waits for the raw
    // words count exactly the loads issued after them.
    auto iter = [&](int ks0, auto u_c) {
        constexpr int U = decltype(u_c)::value;
        const int ks = ks0 + U;
        const bool more = U < 3 || ks0 + 4 < nk;   // a step ks + 1
        // step ks + 1 opens a block at U = 3: its header, loaded an iteration ago, is current from here on
        if (T == kQ4_K && U == 3) hcur = hnext;
        {   // A of step ks + 1, raw weights of step ks + 2 (the last steps reload the last one: no branch around them)
            load_a(min(ks + 1, nk - 1));
            const int s2 = min(ks + 2, nk - 1);
            if constexpr (T == kQ4_K) {
                load_b(s2, IntC<U & 1>{}, IntC<(U + 2) & 3>{});
            } else if constexpr (U & 1) {   // half (ks + 3) / 2 into slot ((ks + 3) / 2) & 1 (= U / 2)
                load_q6(min((ks + 3) >> 1, 2 * (K / 256) - 1), r6[U >> 1]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);   // the loads stay ahead of the step's products
        const uint8_t* A = sA + (U & 1) * kTallSlab;
        const uint8_t* B = sB + (U & 1) * (BN * 128);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int ch = 2 * kk + hf;
            f16x8_t fa[2], fb[JW];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                fa[i] = *(const f16x8_t*)(A + 16 * swz(64 * wm + 32 * i + (lane & 31), ch));
#pragma unroll
            for (int j = 0; j < JW; ++j) fb[j] = *(const f16x8_t*)(B + 16 * swz(cb[j] + (lane & 31), ch));
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < JW; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
            if (more && kk < NF) {
                if constexpr (T == kQ4_K) dequant(kk, (U + 1) & 1, IntC<(U + 1) & 1>{}, IntC<(U + 1) & 3>{}, hcur);
                else dequant(kk, (U + 1) & 1, IntC<((U + 1) >> 1) & 1>{}, IntC<(U + 1) & 1>{}, hcur);
            }
            if (more && kk == 1) store_a((U + 1) & 1);
        }
        lds_sync();
    };
    for (int ks0 = 0; ks0 < nk; ks0 += 4) {
        iter(ks0, IntC<0>{});
        iter(ks0, IntC<1>{});
        iter(ks0, IntC<2>{});
        iter(ks0, IntC<3>{});
    }

    // Epilogue.  Lane holds C[64 wm + 32 i + 8 (q / 4) + 4 hf + q % 4][cb[j] + lane % 32]; the values go through a
    // row-major staging tile in LDS (the A and B buffers are free), so that each global store is 16 contiguous bytes
    if constexpr (!DOWN) {
        // h column hc = (BN / 4) wn + 32 j + lane % 32 (j < JW / 2) = SwiGLU(gate acc[i][j], up acc[i][j + JW / 2]),
        // at its place in the step order of the h row
        constexpr int stride = BN + 16;   // BN / 2 f16 values a staged row
        bool sat = false;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < JW / 2; ++j) {
                const int hc = (BN / 4) * wn + 32 * j + (lane & 31);
                const int spos = (hc & ~63) + perm64(hc & 63);
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int row = 64 * wm + 32 * i + 8 * (q >> 2) + 4 * hf + (q & 3);
                    const float gv = acc[i][j][q], uv = acc[i][j + JW / 2][q];
                    const float e = __builtin_amdgcn_exp2f(-gv * 1.4426950408889634f);
                    float hv = gv * __builtin_amdgcn_rcpf(1.0f + e) * uv;
                    sat |= past_f16(hv);
                    hv = __builtin_fminf(__builtin_fmaxf(hv, -65504.0f), 65504.0f);
                    *(uint16_t*)(lds + row * stride + 2 * spos) = f2h(hv);
                }
            }
        if (sat && a.err) atomicOr(a.err, kSatBit);
        lds_sync();
        constexpr int cpr = BN / 16;   // 16-byte chunks a row
#pragma unroll
        for (int u = 0; u < 256 * cpr / 512; ++u) {
            const int idx = tid + 512 * u, row = idx / cpr, c = idx % cpr;
            *(uint4*)(a.h + (int64_t)(r0 + row) * F + n0 + 8 * c) = *(const uint4*)(lds + row * stride + 16 * c);
        }
    } else {
        auto epilogue = [&](auto esz_c) {
            constexpr int ESZ = decltype(esz_c)::value;
            constexpr int stride = BN * ESZ + 16, rpp = BN * ESZ <= 256 ? 256 : BN * ESZ <= 512 ? 128 : 64;
            constexpr int cpr = BN * ESZ / 16;   // 16-byte chunks a staged row
            bool sat = false;
#pragma unroll
            for (int rb = 0; rb < 256; rb += rpp) {
                lds_sync();   // every wave is done with the buffers (or with the last pass's staging)
                if (64 * wm >= rb && 64 * wm < rb + rpp) {
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < JW; ++j) {
                            const int col = cb[j] + (lane & 31);
#pragma unroll
                            for (int q = 0; q < 16; ++q) {
                                const int row = 64 * wm + 32 * i + 8 * (q >> 2) + 4 * hf + (q & 3) - rb;
                                const float v = acc[i][j][q];
                                if constexpr (ESZ == 4) {
                                    *(float*)(lds + row * stride + 4 * col) = v;
                                } else {
                                    sat |= past_f16(v);
                                    *(uint16_t*)(lds + row * stride + 2 * col) =
                                        f2h(__builtin_fminf(__builtin_fmaxf(v, -65504.0f), 65504.0f));
                                }
                            }
                        }
                }
                lds_sync();
#pragma unroll
                for (int u = 0; u < rpp * cpr / 512; ++u) {
                    const int idx = tid + 512 * u, r = idx / cpr, c = idx - r * cpr;
                    const uint4 v = *(const uint4*)(lds + r * stride + 16 * c);
                    const int64_t o = (int64_t)s_entry[rb + r] * a.ld_parts + n0 + c * (16 / ESZ);
                    if constexpr (ESZ == 4) *(uint4*)(a.parts + o) = v;
                    else *(uint4*)(a.parts_h + o) = v;
                }
            }
            if (sat && a.err) atomicOr(a.err, kSatBit);
        };
        if (a.parts_h) epilogue(IntC<2>{});
        else epilogue(IntC<4>{});
    }
}

// weight rows a tall tile: Q4_K gate/up 256 (128 h columns); 128 for down (output columns) and for Q6_K gate/up,
// whose raw words take the registers a 256-row tile's accumulators need
__host__ __device__ constexpr int tall_bn(bool down, int t) { return down || t == kQ6_K ? 128 : 256; }

template <bool DOWN>
static hipError_t launch_tall(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s) {
    const int t = DOWN ? L.d_type : L.gu_type;
    const int BN = tall_bn(DOWN, t);
    const int n_tiles = DOWN ? (int)(L.n_embd / BN) : (int)(L.n_ff / (BN / 2));
    const int mt_cap = (int)(a.rows / 256);
    if (mt_cap == 0) return hipSuccess;
    const unsigned grid = (unsigned)(8 * ((mt_cap + 7) / 8) * n_tiles);
    const size_t lds = (size_t)tall_lds(BN) + (DOWN ? 256 * 4 : 0);
    void (*k)(ExpertLayout, PrefillArgs, const int32_t*, int) =
        t == kQ4_K ? tall_mfma_kernel<DOWN, kQ4_K, tall_bn(DOWN, kQ4_K)> : tall_mfma_kernel<DOWN, kQ6_K, 128>;
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3(grid), dim3(512), lds, s, L, a, tall_list(a.mtile, a.rows, a.cap_groups), n_tiles);
    return hipGetLastError();
}

bool tall_usable(const ExpertLayout& L) {
    auto q = [](int t) { return t == kQ4_K || t == kQ6_K; };
    return q(L.gu_type) && q(L.d_type) && !mixed_gu(L) && L.n_ff % 256 == 0 && L.n_embd % 256 == 0;
}

// rest: the rows past the tall tiles (at most two m-tiles a group).  Those, and groups of under 128 rows on average
// (config 5's prompt: ~32 rows an expert, 2,394 -> 2,359 us), take the m-tile-per-XCD order: a group's weights are
// fetched once either way, and the m-tile's activations once instead of into every XCD
template <bool DOWN, bool MMQ = false>
static hipError_t launch_gemm(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s, bool rest = false) {
    // (a mixed layer's gate/up: the generic path, which dequantizes each row by its own type)
    const int t = DOWN ? L.d_type : mixed_gu(L) ? -1 : L.gu_type;
    const int n_tiles = DOWN ? (int)(L.n_embd / (128 * lane_rows(DOWN, t))) : (int)(L.n_ff / (kBN / 2));
    const bool q8_fast = (DOWN ? L.n_ff : L.n_embd) % 128 == 0;   // Q8_0's own path takes its K steps in pairs
    const int bm = 32 * row_tiles(DOWN, q8_fast ? t : (t == kQ8_0 ? 0 : t));
    // tiles: at most ceil(rows / bm) + one partial tile a group (the standalone product counts every row of xq)
    const int64_t rows = MMQ ? a.n_tok : a.rows;
    const int mt_bound = (int)((rows + bm - 1) / bm + a.cap_groups);
    const int by_n = n_tiles % 8 == 0 && !rest && !(rows < 128 * a.cap_groups);
    const unsigned grid = (unsigned)(by_n ? mt_bound * n_tiles : 8 * ((mt_bound + 7) / 8) * n_tiles);
    const size_t lds = (size_t)entry_offset(bm) + (DOWN ? (size_t)bm * 4 : 0);
    void (*k)(ExpertLayout, PrefillArgs, const int32_t*, int, int, int) =
        t == kQ4_K   ? grouped_mfma_kernel<DOWN, kQ4_K, row_tiles(DOWN, kQ4_K), MMQ>
        : t == kQ6_K ? grouped_mfma_kernel<DOWN, kQ6_K, row_tiles(DOWN, kQ6_K), MMQ>
        : t == kQ8_0 && q8_fast ? grouped_mfma_kernel<DOWN, kQ8_0, row_tiles(DOWN, kQ8_0), MMQ>
                     : grouped_mfma_kernel<DOWN, 0, row_tiles(DOWN, 0), MMQ>;
    hipLaunchKernelGGL(k, dim3(grid), dim3(256), lds, s, L, a, a.mtile, mt_bound, n_tiles, by_n);
    return hipGetLastError();
}

hipError_t launch_mmq_product(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s) {
    return launch_gemm<true, true>(L, a, s);
}

hipError_t launch_prefill_experts(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s) {
    const int64_t nc = a.n_tok * L.n_embd / 8;
    if (!a.xb_ready)
        hipLaunchKernelGGL(to_f16_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, s, a.x, a.xb, nc, a.err);
    if (!a.mtile_ready)
        hipLaunchKernelGGL(tile_map_kernel, dim3(1), dim3(1024), 0, s, a.bounds, a.n_groups, a.mtile, a.rows,
                           (int)a.cap_groups);
    hipError_t e = launch_gemm<false>(L, a, s);
    if (e != hipSuccess) return e;
    return launch_gemm<true>(L, a, s);
}

hipError_t launch_prefill_experts_split(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s, hipStream_t side,
                                        hipEvent_t fork, hipEvent_t join) {
    if (!a.mtile_ready) return hipErrorInvalidValue;   // (the route writes the split maps and the tall list)
    const int64_t nc = a.n_tok * L.n_embd / 8;
    if (!a.xb_ready)
        hipLaunchKernelGGL(to_f16_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, s, a.x, a.xb, nc, a.err);
    hipError_t e;
    const bool two = side != s;   // (side == s: the two chains one after the other)
    if (two && ((e = hipEventRecord(fork, s)) != hipSuccess || (e = hipStreamWaitEvent(side, fork, 0)) != hipSuccess))
        return e;
    // the tall tiles on s, first (a tall work-group takes a whole compute unit: issued first, they are placed before
    // the other chain's work-groups fill the units), the remainder rows on the side stream
    if ((e = launch_tall<false>(L, a, s)) != hipSuccess || (e = launch_tall<true>(L, a, s)) != hipSuccess) return e;
    if ((e = launch_gemm<false>(L, a, side, true)) != hipSuccess ||
        (e = launch_gemm<true>(L, a, side, true)) != hipSuccess)
        return e;
    if (!two) return hipSuccess;
    if ((e = hipEventRecord(join, side)) != hipSuccess) return e;
    return hipStreamWaitEvent(s, join, 0);
}

}  // namespace xs
