// xestrata-win_amd/csrc/experts_prefill.hip - grouped expert products for prompt and verify batches: a bf16 MFMA
// grouped GEMM whose expert weight tiles are dequantized from the raw GGUF blocks into LDS (the MI355X replacement
// of the reference's int8 iq_mmq_grouped, src/kernels/xe/iq_mmq.cpp:483-943, and of its FP16 fallbacks
// xmx_gemm_grouped / Gemm::f16_groups, src/prefill/gemm.cpp:371-388).
//
// Rows are the routed rows in expert order (the permutation of src/prefill/plain_prompt.cpp:576-637).  Two launches:
//   gate/up: h[row, j] = SwiGLU(x[src[row]] . gate_j, x[src[row]] . up_j) in bf16, a tile = 128 rows x 64 h columns
//            (their 64 gate and 64 up weight rows, so the SwiGLU is formed in registers);
//   down:    parts[entry[row], c] = h[row] . down_c in fp32, a tile = 128 rows x 128 output columns, written straight
//            into routing order for the combine.
// Tiles: 128 rows x 256 weight rows, 256 threads, 4 waves of 64 x 128 (2 x 4 v_mfma_f32_32x32x16_bf16 tiles: the
// 32 x 32 MFMA sustains ~80% of the bf16 peak where 16 x 16 x 32 needs twice the independent accumulators), K steps of
// 64 with both operands in LDS as rows of 8 chunks of 16 bytes, chunk c of row r at slot c ^ (r & 7) (the fragment
// reads of 8 neighbouring rows hit 8 different bank groups).  Each step's activation rows (gathered through src for
// gate/up) and raw weight bytes are loaded into registers two steps ahead, so their latency runs under two steps of
// MFMAs; at its turn a step's activations are stored to LDS and its weights dequantized to bf16 there (Q4_K and Q6_K
// unpacked 16 bytes at a time, other formats 32 values at a time).  A work-group's m-tile comes from a flat index over every group's ceil(rows / 128) tiles (a
// prefix computed on the device).  Work-group b runs on XCD b % 8; an XCD takes every eighth m-tile and runs its
// n-tiles one after the other, so the m-tile's activations and its expert's weights are fetched into that XCD's L2
// once and reused across the n-tiles.
#include "xs_device.h"
#include "xs_dequant.h"
#include "xs_kernels.h"
#include "xs_units.h"

namespace xs {

typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 256, kBK = 64;

__global__ __launch_bounds__(256) void to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = f2bf(x[i]);
}

// mtile[g] = sum over groups before g of ceil(rows / kBM); mtile[n_groups] = the total
__global__ __launch_bounds__(1024) void tile_map_kernel(const int32_t* __restrict__ bounds,
                                                        const int32_t* __restrict__ n_groups, int32_t* __restrict__ mtile,
                                                        int cap_groups) {
    __shared__ int s_wave[16];
    __shared__ int s_carry;
    const int ng = min(*n_groups, cap_groups);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (int g0 = 0; g0 <= ng; g0 += 1024) {
        const int g = g0 + tid;
        const int t = g < ng ? (bounds[g + 1] - bounds[g] + kBM - 1) / kBM : 0;
        int inc = t;
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(inc, o, 64);
            if (lane >= o) inc += y;
        }
        if (lane == 63) s_wave[wave] = inc;
        __syncthreads();
        int before = s_carry;
        for (int w = 0; w < wave; ++w) before += s_wave[w];
        if (g <= ng) mtile[g] = before + inc - t;
        __syncthreads();
        if (tid == 1023) s_carry = before + inc;
        __syncthreads();
    }
}

// A load through a global-address-space pointer.  Blob addresses come from memory (the group table), so the compiler
// cannot prove them global and would emit FLAT loads, which also count on lgkmcnt: every wait for an LDS operand of
// the MFMAs would then wait for the weight prefetch in flight.
template <typename V>
__device__ __forceinline__ V ldg(const void* p) {
    return *(const __attribute__((address_space(1))) V*)p;
}
typedef unsigned int gu32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg16(const void* p) {
    const gu32x4_t v = *(const __attribute__((address_space(1))) gu32x4_t*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ int swz(int r, int c) { return r * 8 + (c ^ (r & 7)); }   // in 16-byte units


// the raw bytes of one thread's share of a weight step (row br = the thread, the step's 64 values); see stage_b.
// Q6_K blocks (210 bytes) sit at 2-byte alignment: their words are loaded aligned and realigned when staged, so the
// loads stay in flight until then.
struct BRegs {
    uint4 a, b, c;     // Q4_K: a = block header, b, c = the 32 qs bytes
    uint32_t q6[26];   // Q6_K: 17 aligned words over the step's 64 ql bytes, 9 over its 32 qh bytes
    uint32_t s, t;     // Q6_K: the 4 int8 scales; d | the byte misalignment << 16
};

template <int T>
__device__ __forceinline__ void load_b(const uint8_t* brow, int k0, BRegs& r) {
    if (T == kQ4_K) {
        const uint8_t* blk = brow + 144 * (k0 >> 8);
        const int p = (k0 & 255) >> 6;
        r.a = ldg16(blk);
        r.b = ldg16(blk + 16 + 32 * p);
        r.c = ldg16(blk + 32 + 32 * p);
    } else if (T == kQ6_K) {
        const uint8_t* blk = brow + 210 * (k0 >> 8);
        const int t = (k0 & 255) >> 6, n = t >> 1, sel = t & 1;
        const uintptr_t u = (uintptr_t)blk;
        const __attribute__((address_space(1))) uint32_t* q =
            (const __attribute__((address_space(1))) uint32_t*)(u & ~(uintptr_t)3);
        // dword-aligned 16-byte loads (fewer address passes than one load a word)
        typedef unsigned int u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
        const __attribute__((address_space(1))) u32x4_a4* q4 = (const __attribute__((address_space(1))) u32x4_a4*)q;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4_a4 v = *(const __attribute__((address_space(1))) u32x4_a4*)(q + 16 * n + 4 * i);
            r.q6[4 * i] = v.x; r.q6[4 * i + 1] = v.y; r.q6[4 * i + 2] = v.z; r.q6[4 * i + 3] = v.w;
        }
        r.q6[16] = q[16 * n + 16];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const u32x4_a4 v = *(const __attribute__((address_space(1))) u32x4_a4*)(q + 32 + 8 * n + 4 * i);
            r.q6[17 + 4 * i] = v.x; r.q6[18 + 4 * i] = v.y; r.q6[19 + 4 * i] = v.z; r.q6[20 + 4 * i] = v.w;
        }
        r.q6[25] = q[32 + 8 * n + 8];
        (void)q4;
        const uint8_t* sc = blk + 192 + 8 * n + 4 * sel;
        r.s = (uint32_t)ldg<uint16_t>(sc) | ((uint32_t)ldg<uint16_t>(sc + 2) << 16);
        r.t = (uint32_t)ldg<uint16_t>(blk + 208) | ((uint32_t)(u & 3) << 16);
    }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// two floats to packed bf16, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pk2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ float byte_f(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFFu); }   // v_cvt_f32_ubyteN
// scale * byte + offset for the 4 bytes of w, packed as two bf16 pairs
__device__ __forceinline__ uint2 deq4(uint32_t w, float sc, float off) {
    return make_uint2(pk2(__builtin_fmaf(sc, byte_f(w, 0), off), __builtin_fmaf(sc, byte_f(w, 1), off)),
                      pk2(__builtin_fmaf(sc, byte_f(w, 2), off), __builtin_fmaf(sc, byte_f(w, 3), off)));
}
// 16 codes (4 registers of 4 bytes) -> 2 chunks of 8 bf16 at chunk c of row br
__device__ __forceinline__ void put16(uint4* sb, int br, int c, const uint32_t (&q)[4], float sc, float off) {
    const uint2 v0 = deq4(q[0], sc, off), v1 = deq4(q[1], sc, off), v2 = deq4(q[2], sc, off), v3 = deq4(q[3], sc, off);
    sb[swz(br, c)] = make_uint4(v0.x, v0.y, v1.x, v1.y);
    sb[swz(br, c + 1)] = make_uint4(v2.x, v2.y, v3.x, v3.y);
}

// dequantize the thread's 64 values of the step (its weight row, chunks 0..7) to bf16 in the B stage.  Q4_K is
// d·sc·q − dmin·m and Q6_K d·sc·(q − 32), each one fma of the code (4 codes a register: nibble masks, byte converts),
// then packed bf16 converts; other formats go through dequant32.
template <int T>
__device__ __forceinline__ void stage_b(const BRegs& r, const uint8_t* brow, int type, int k0, int br, uint4* sb) {
    if (T == kQ4_K) {
        const int p = (k0 & 255) >> 6;
        const float d = h2f((uint16_t)(r.a.x & 0xFFFFu)), dmin = h2f((uint16_t)(r.a.x >> 16));
        int sc0, m0, sc1, m1;
        q4k_sm(r.a.y, r.a.z, r.a.w, 2 * p, sc0, m0);
        q4k_sm(r.a.y, r.a.z, r.a.w, 2 * p + 1, sc1, m1);
        const float d0 = d * (float)sc0, n0 = -(dmin * (float)m0), d1 = d * (float)sc1, n1 = -(dmin * (float)m1);
        const uint32_t w[8] = {r.b.x, r.b.y, r.b.z, r.b.w, r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
        for (int g = 0; g < 2; ++g) {   // values 16 g .. (low nibbles) and 32 + 16 g .. (high nibbles)
            const uint32_t lo[4] = {w[4 * g] & 0x0F0F0F0Fu, w[4 * g + 1] & 0x0F0F0F0Fu, w[4 * g + 2] & 0x0F0F0F0Fu,
                                    w[4 * g + 3] & 0x0F0F0F0Fu};
            const uint32_t hi[4] = {(w[4 * g] >> 4) & 0x0F0F0F0Fu, (w[4 * g + 1] >> 4) & 0x0F0F0F0Fu,
                                    (w[4 * g + 2] >> 4) & 0x0F0F0F0Fu, (w[4 * g + 3] >> 4) & 0x0F0F0F0Fu};
            put16(sb, br, 2 * g, lo, d0, n0);
            put16(sb, br, 4 + 2 * g, hi, d1, n1);
        }
    } else if (T == kQ6_K) {
        const int sel = ((k0 & 255) >> 6) & 1, ns = 4 * sel;
        const float d = h2f((uint16_t)(r.t & 0xFFFFu));
        const uint32_t sh = r.t >> 16;
        uint32_t ql[16], qh[8];
#pragma unroll
        for (int i = 0; i < 16; ++i) ql[i] = __builtin_amdgcn_alignbyte(r.q6[i + 1], r.q6[i], sh);
#pragma unroll
        for (int i = 0; i < 8; ++i) qh[i] = __builtin_amdgcn_alignbyte(r.q6[18 + i], r.q6[17 + i], sh);
#pragma unroll
        for (int g = 0; g < 4; ++g) {   // values 16 g ..: ql bytes 32 (g / 2) + 16 (g % 2) .., qh bits ns + 2 (g / 2)
            const float sc = d * (float)(int8_t)((r.s >> (8 * g)) & 0xFFu);
            const int hs = ns + 2 * (g >> 1);
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                q[i] = ((ql[4 * g + i] >> ns) & 0x0F0F0F0Fu) | (((qh[4 * (g & 1) + i] >> hs) & 0x03030303u) << 4);
            put16(sb, br, 2 * g, q, sc, -32.0f * sc);
        }
    } else {
        const int qk = block_values(type), bs = block_bytes(type);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float v[32];
            const int kv = k0 + 32 * half;
            dequant32(type, brow + (int64_t)(kv / qk) * bs, (kv % qk) / 32, v);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                sb[swz(br, 4 * half + c)] = make_uint4(pk2(v[8 * c], v[8 * c + 1]), pk2(v[8 * c + 2], v[8 * c + 3]),
                                                       pk2(v[8 * c + 4], v[8 * c + 5]), pk2(v[8 * c + 6], v[8 * c + 7]));
        }
    }
}

constexpr int kRing = 3;   // activation stages in LDS: a step's rows go out two steps before its MFMAs

// one K step of a consumer wave: 4 k-chunks of 16 over its 2 x 4 tiles of 32 x 32 (lane l holds A[row l % 32][k 8 (l / 32)
// ..] and B[k 8 (l / 32) ..][col l % 32]); the next chunk's fragments are read while this chunk's MFMAs run (one
// consumer wave a SIMD: nothing else hides the LDS latency)
struct Frags {
    bf16x8_t a0, a1, b0, b1, b2, b3;
};
__device__ __forceinline__ Frags read_frags(const uint4* sA, const uint4* sB, int rw, const int (&cb)[4], int lane,
                                            int kk) {
    const int ch = 2 * kk + (lane >> 5), r = lane & 31;
    Frags f;
    f.a0 = __builtin_bit_cast(bf16x8_t, sA[swz(rw + r, ch)]);
    f.a1 = __builtin_bit_cast(bf16x8_t, sA[swz(rw + 32 + r, ch)]);
    f.b0 = __builtin_bit_cast(bf16x8_t, sB[swz(cb[0] + r, ch)]);
    f.b1 = __builtin_bit_cast(bf16x8_t, sB[swz(cb[1] + r, ch)]);
    f.b2 = __builtin_bit_cast(bf16x8_t, sB[swz(cb[2] + r, ch)]);
    f.b3 = __builtin_bit_cast(bf16x8_t, sB[swz(cb[3] + r, ch)]);
    return f;
}
__device__ __forceinline__ void mfma8(const Frags& f, f32x16_t (&acc)[2][4]) {
    acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0, f.b0, acc[0][0], 0, 0, 0);
    acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1, f.b0, acc[1][0], 0, 0, 0);
    acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0, f.b1, acc[0][1], 0, 0, 0);
    acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1, f.b1, acc[1][1], 0, 0, 0);
    acc[0][2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0, f.b2, acc[0][2], 0, 0, 0);
    acc[1][2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1, f.b2, acc[1][2], 0, 0, 0);
    acc[0][3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0, f.b3, acc[0][3], 0, 0, 0);
    acc[1][3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1, f.b3, acc[1][3], 0, 0, 0);
}
__device__ __forceinline__ void mfma_step(const uint4* sA, const uint4* sB, int rw, const int (&cb)[4], int lane,
                                          f32x16_t (&acc)[2][4]) {
    Frags f0 = read_frags(sA, sB, rw, cb, lane, 0);
    Frags f1 = read_frags(sA, sB, rw, cb, lane, 1);
    mfma8(f0, acc);
    f0 = read_frags(sA, sB, rw, cb, lane, 2);
    mfma8(f1, acc);
    f1 = read_frags(sA, sB, rw, cb, lane, 3);
    mfma8(f0, acc);
    mfma8(f1, acc);
}

// a producer's step: its weight row's raw bytes prefetched three steps ahead (register sets r0, r1, r2 in turn)
template <int T>
struct Producer {
    const uint8_t* brow;
    int wtype, row, nk;
    BRegs r0, r1, r2;
    __device__ __forceinline__ void load(int ks, BRegs& r) {
        if (ks < nk) load_b<T>(brow, ks * kBK, r);
    }
    // dequantize step ks from r into the B stage, then reuse r for step ks + 3
    __device__ __forceinline__ void turn(int ks, BRegs& r, uint4* sb) {
        if (ks < nk) {
            stage_b<T>(r, brow, wtype, ks * kBK, row, sb);
            load(ks + 3, r);
        }
    }
};

// Work-group = 8 waves.  Waves 0-3 (consumers) hold the accumulators: they bring the activation rows into a ring of LDS
// stages by DMA, two steps ahead, and run the MFMAs.  Waves 4-7 (producers) hold no accumulators, so each keeps three
// steps of its weight row's raw bytes in flight in registers and dequantizes two steps ahead into a ring of three bf16
// stages (a producer's slow step is absorbed).  One barrier a step hands the stages over.
template <bool DOWN, int T>
__global__ __launch_bounds__(512, 1) void grouped_mfma_kernel(ExpertLayout L, PrefillArgs a,
                                                              const int32_t* __restrict__ mtile, int mt_bound,
                                                              int n_tiles) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the tile of this work-group: XCD x = blockIdx % 8 takes m-tiles x, x + 8, ..., each with its n-tiles one after
    // the other (the m-tile's activation rows and its expert's weight slabs stay in that XCD's L2 across them)
    const int c8 = (int)(blockIdx.x >> 3);
    const int mt = (c8 / n_tiles) * 8 + (int)(blockIdx.x & 7), nt = c8 % n_tiles;
    if (mt >= mt_bound) return;
    const int ng = *a.n_groups;
    if (ng <= 0 || mt >= mtile[ng]) return;
    int lo = 0, hi = ng - 1;   // the group whose tiles hold mt
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (mtile[mid] <= mt) lo = mid;
        else hi = mid - 1;
    }
    const int g = lo;
    const int r0 = a.bounds[g] + (mt - mtile[g]) * kBM;
    const int nrows = min(kBM, a.bounds[g + 1] - r0);
    const int H = (int)L.n_embd, F = (int)L.n_ff;
    const int K = DOWN ? F : H;
    const int nk = K / kBK;
    const int n0 = nt * (DOWN ? kBN : kBN / 2);
    uint4* ring = (uint4*)lds;                          // kRing x 128 rows x 8 chunks
    uint4* sB = (uint4*)(lds + kRing * kBM * 128);      // 3 x 256 rows x 8 chunks
    auto stage_a = [&](int ks) { return ring + (ks % kRing) * (kBM * 8); };
    auto stage_b_buf = [&](int ks) { return sB + (ks % 3) * (kBN * 8); };

    if (wave >= 4) {   // ---- producers: thread p = weight row p of the tile
        const int p = tid - 256;
        const int wrow = DOWN ? n0 + p : (p < kBN / 2 ? n0 + p : F + n0 + (p - kBN / 2));
        Producer<T> pr;
        pr.brow = (const uint8_t*)a.wptr[g] + (DOWN ? L.down_off : 0) + (int64_t)wrow * (DOWN ? L.d_row : L.gu_row);
        pr.wtype = DOWN ? L.d_type : L.gu_type;
        pr.row = p;
        pr.nk = nk;
        pr.load(0, pr.r0);
        pr.load(1, pr.r1);
        pr.load(2, pr.r2);
        pr.turn(0, pr.r0, stage_b_buf(0));
        pr.turn(1, pr.r1, stage_b_buf(1));
        __syncthreads();   // barrier 0: steps 0 and 1 staged
        // between barriers j and j + 1 (j = 0 .. nk - 2) the producers stage step j + 2 while the consumers run step
        // j; step s uses register set s % 3
        for (int st = 2; st <= nk; st += 3) {
            pr.turn(st, pr.r2, stage_b_buf(st));
            __syncthreads();
            if (st + 1 > nk) break;
            pr.turn(st + 1, pr.r0, stage_b_buf(st + 1));
            __syncthreads();
            if (st + 2 > nk) break;
            pr.turn(st + 2, pr.r1, stage_b_buf(st + 2));
            __syncthreads();
        }
        return;
    }

    // ---- consumers: A rows by DMA (instruction i of wave w fills slots [64 (4w + i), +64): row 8 (4w + i) + lane / 8,
    // slot lane % 8 = chunk (lane % 8) ^ (row & 7); rows past the tile's end read its first row, unused)
    const uint16_t* arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * (4 * wave + i) + (lane >> 3);
        const int rr = r < nrows ? r : 0;
        const int chunk = (lane & 7) ^ (r & 7);
        arow[i] = (DOWN ? a.h + (int64_t)(r0 + rr) * F : a.xb + (int64_t)a.src[r0 + rr] * H) + 8 * chunk;
    }
    auto dma_a = [&](int ks) {
        uint4* dst = stage_a(ks);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(arow[i] + ks * kBK,
                                             (__attribute__((address_space(3))) void*)(dst + 64 * (4 * wave + i)), 16,
                                             0, 0);
    };
    const int rw = 64 * (wave >> 1), wn = wave & 1;
    int cb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) cb[j] = DOWN ? 128 * wn + 32 * j : (j < 2 ? 64 * wn + 32 * j : 128 + 64 * wn + 32 * (j - 2));
    f32x16_t acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

    dma_a(0);
    if (nk > 1) {
        dma_a(1);
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");   // step 0's rows are in; step 1's fly
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();   // barrier 0
    for (int ks = 0; ks < nk; ++ks) {   // barrier ks + 1 follows the MFMAs of step ks (none after the last)
        const bool more = ks + 2 < nk;
        if (more) dma_a(ks + 2);
        mfma_step(stage_a(ks), stage_b_buf(ks), rw, cb, lane, acc);
        if (ks + 1 < nk) {   // step ks + 1's rows have landed before the barrier hands them over
            if (more) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
    }
    // lane holds C[rw + 32 i + 8 (q / 4) + 4 (lane / 32) + q % 4][cb[j] + lane % 32]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int row = rw + 32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
            if (row >= nrows) continue;
            if (DOWN) {
                float* dst = a.parts + (int64_t)a.entry[r0 + row] * H + n0;
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[cb[j] + (lane & 31)] = acc[i][j][q];
            } else {
                uint16_t* dst = a.h + (int64_t)(r0 + row) * F + n0;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float gv = acc[i][j][q], uv = acc[i][j + 2][q];
                    // SwiGLU on the hardware exp2 and reciprocal (the bf16 path's tolerance, not canon's bits)
                    const float e = __builtin_amdgcn_exp2f(-gv * 1.4426950408889634f);
                    const float hv = gv * __builtin_amdgcn_rcpf(1.0f + e) * uv;
                    dst[cb[j] + (lane & 31)] = f2bf(hv);
                }
            }
        }
}

template <bool DOWN>
static hipError_t launch_gemm(const ExpertLayout& L, const PrefillArgs& a, int mt_bound, hipStream_t s) {
    const int n_tiles = DOWN ? (int)(L.n_embd / kBN) : (int)(L.n_ff / (kBN / 2));
    const unsigned grid = (unsigned)(8 * ((mt_bound + 7) / 8) * n_tiles);
    const int t = DOWN ? L.d_type : L.gu_type;
    const size_t lds = (size_t)(kRing * kBM + 3 * kBN) * 128;
    void (*k)(ExpertLayout, PrefillArgs, const int32_t*, int, int) =
        t == kQ4_K ? grouped_mfma_kernel<DOWN, kQ4_K> : t == kQ6_K ? grouped_mfma_kernel<DOWN, kQ6_K>
                                                                    : grouped_mfma_kernel<DOWN, 0>;
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3(grid), dim3(512), lds, s, L, a, (const int32_t*)a.mtile, mt_bound, n_tiles);
    return hipGetLastError();
}

hipError_t launch_prefill_experts(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s) {
    const int64_t nx = a.n_tok * L.n_embd;
    hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, s, a.x, a.xb, nx);
    hipLaunchKernelGGL(tile_map_kernel, dim3(1), dim3(1024), 0, s, a.bounds, a.n_groups, a.mtile, (int)a.cap_groups);
    const int mt_bound = (int)((a.rows + kBM - 1) / kBM + a.cap_groups);
    hipError_t e = launch_gemm<false>(L, a, mt_bound, s);
    if (e != hipSuccess) return e;
    return launch_gemm<true>(L, a, mt_bound, s);
}

}  // namespace xs
