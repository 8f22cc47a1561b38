// xestrata-win_amd/csrc/xs_units.h - the canonical row arithmetic of the grouped expert products, shared by the
// modular decode kernels (experts_decode.hip) and the fused decode layer (decode_fused.hip).
//
// A row is a run of units: a whole 256-value block when the activation has one scale for each 256 values (gate/up:
// quantize_q8_1_rows), else a 32-value group (down, and Q8_0).  A unit's products are exact integers (v_dot4_i32_i8
// of the codes against the q8_1 int8 values, the sub-block scales applied in integers); its scale enters once, acc =
// fma(d * d8, S, acc) (Q4_K's min term a second fma) - the reference's integer-first canonical rows (seg_dot_canon,
// src/kernels/xe/iq_kernels.cpp:832-884) applied to every format.  L = min(8, the largest power of two dividing the
// unit count) lanes share a row, lane c taking units c, c + L, ..., then a xor butterfly over the L lanes.  The CPU
// oracle (oracle/xs_oracle.c, xso_vec_dot) takes the same steps, so rows agree bit for bit.
#pragma once

#include "xs_device.h"

namespace xs {

static __constant__ uint32_t kIq4Tab[4] = {0xBFAD9881u, 0xF6EADDCFu, 0x26190D01u, 0x71594535u};   // kvalues_iq4nl bytes

struct Act {            // one entry's activation in LDS
    const int8_t* q;    // n int8 values
    const float* d8;    // n / 32 scales (the q8_1 blocks' fp16 d, as float)
    const int* us16;    // n / 16 sums of 16 int8 values
};

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

// NW words at a 2-byte aligned byte offset `off` of a 16-byte aligned LDS buffer: aligned 32-bit reads, realigned
// with v_alignbyte (the offset, not the address, gives the alignment: LDS pointers are not cast to integers)
template <int NW>
__device__ __forceinline__ void lds_words_a2(const uint8_t* base, int off, uint32_t (&w)[NW]) {
    const uint32_t* q = (const uint32_t*)(base + (off & ~3));
    const uint32_t sh = (uint32_t)(off & 3);
    uint32_t d[NW + 1];
#pragma unroll
    for (int i = 0; i <= NW; ++i) d[i] = q[i];
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}

__device__ __forceinline__ int us32(const Act& a, int g) { return a.us16[2 * g] + a.us16[2 * g + 1]; }

// PAD: bytes between the int8 values of consecutive 256-value blocks of the activation (0: packed).  Lanes of a row
// read the same piece of 8 neighbouring blocks at once; 256 bytes apart those reads all hit the same LDS banks, 272
// apart they spread over all of them.
template <int T, bool S256, int PAD = 0>
struct Unit;
// the padding the modular kernels give their staged gate/up rows, and a staged row's int8 bytes with a padding
constexpr int kActPad = 16;
__host__ __device__ inline int act_rowq(int n, int pad) { return n + ((n + 255) >> 8) * pad; }

// ---- Q4_K
template <bool S256, int PAD>
struct Unit<kQ4_K, S256, PAD> {
    static constexpr int kUnit = S256 ? 256 : 32;
    template <int NE>
    __device__ static __forceinline__ void apply(const uint8_t* base, int roff, int u, const Act (&a)[NE], int n,
                                                 float (&acc)[NE]) {
        const int b = S256 ? u : u >> 3;
        const uint8_t* blk = base + roff + 144 * b;
        const uint4 hdr = *(const uint4*)blk;
        const float d = h2f((uint16_t)(hdr.x & 0xFFFFu)), dmin = h2f((uint16_t)(hdr.x >> 16));
        if (S256) {
            int sc[8], m[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) q4k_sm(hdr.y, hdr.z, hdr.w, s, sc[s], m[s]);
            int s1[NE], s2[NE];
#pragma unroll
            for (int e = 0; e < NE; ++e) s1[e] = s2[e] = 0;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint4 w0 = *(const uint4*)(blk + 16 + 32 * p), w1 = *(const uint4*)(blk + 32 + 32 * p);
                const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int e = 0; e < NE; ++e) {
                    if (e >= n) break;
                    const int8_t* q = a[e].q + (256 + PAD) * b + 64 * p;
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
                    s1[e] += sc[2 * p] * il + sc[2 * p + 1] * ih;
                    s2[e] += m[2 * p] * us32(a[e], 8 * b + 2 * p) + m[2 * p + 1] * us32(a[e], 8 * b + 2 * p + 1);
                }
            }
#pragma unroll
            for (int e = 0; e < NE; ++e) {
                if (e >= n) break;
                const float d8 = a[e].d8[8 * b];
                acc[e] = __builtin_fmaf(d * d8, (float)s1[e], acc[e]);
                acc[e] = __builtin_fmaf(-(dmin * d8), (float)s2[e], acc[e]);
            }
        } else {
            const int g = u & 7;
            int sc, m;
            q4k_sm(hdr.y, hdr.z, hdr.w, g, sc, m);
            const uint4 w0 = *(const uint4*)(blk + 16 + 32 * (g >> 1)), w1 = *(const uint4*)(blk + 32 + 32 * (g >> 1));
            const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            const int sh = 4 * (g & 1);
#pragma unroll
            for (int e = 0; e < NE; ++e) {
                if (e >= n) break;
                const int8_t* q = a[e].q + 32 * u + PAD * (u >> 3);
                const uint4 l0 = *(const uint4*)q, l1 = *(const uint4*)(q + 16);
                const uint32_t al[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
                int is = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) is = sdot4((int)((w[i] >> sh) & 0x0F0F0F0Fu), (int)al[i], is);
                const float d8 = a[e].d8[u];
                acc[e] = __builtin_fmaf(d * d8, (float)(sc * is), acc[e]);
                acc[e] = __builtin_fmaf(-(dmin * d8), (float)(m * us32(a[e], u)), acc[e]);
            }
        }
    }
};

// ---- Q6_K: 32-value group gg of a block: half n = gg / 4, s = gg % 4; codes (ql >> 4(s >> 1)) & 15 | ((qh >> 2s) & 3) << 4
// from ql[64n + 32(s & 1) + l] and qh[32n + l]; scales sc[2gg] (values 0..15), sc[2gg + 1] (16..31)
template <bool S256, int PAD>
struct Unit<kQ6_K, S256, PAD> {
    static constexpr int kUnit = S256 ? 256 : 32;
    template <int NE>
    __device__ static __forceinline__ void group(const uint8_t* base, int boff, int gg, int v0, const Act (&a)[NE],
                                                 int n, int (&S)[NE]) {
        const uint8_t* blk = base + boff;
        const int hn = gg >> 2, s = gg & 3;
        uint32_t ql[8], qh[8];
        lds_words_a2<8>(base, boff + 64 * hn + 32 * (s & 1), ql);
        lds_words_a2<8>(base, boff + 128 + 32 * hn, qh);
        const int nsh = 4 * (s >> 1), hsh = 2 * s;
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = ((ql[i] >> nsh) & 0x0F0F0F0Fu) | (((qh[i] >> hsh) & 0x03030303u) << 4);
        const int sc0 = (int)(int8_t)blk[192 + 2 * gg], sc1 = (int)(int8_t)blk[193 + 2 * gg];
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            if (e >= n) break;
            const int8_t* x = a[e].q + v0 + PAD * (v0 >> 8);
            const uint4 l0 = *(const uint4*)x, l1 = *(const uint4*)(x + 16);
            int i0 = 0, i1 = 0;
            i0 = sdot4((int)q[0], (int)l0.x, i0);
            i0 = sdot4((int)q[1], (int)l0.y, i0);
            i0 = sdot4((int)q[2], (int)l0.z, i0);
            i0 = sdot4((int)q[3], (int)l0.w, i0);
            i1 = sdot4((int)q[4], (int)l1.x, i1);
            i1 = sdot4((int)q[5], (int)l1.y, i1);
            i1 = sdot4((int)q[6], (int)l1.z, i1);
            i1 = sdot4((int)q[7], (int)l1.w, i1);
            i0 -= 32 * a[e].us16[v0 >> 4];          // codes are q + 32
            i1 -= 32 * a[e].us16[(v0 >> 4) + 1];
            S[e] += sc0 * i0 + sc1 * i1;
        }
    }
    template <int NE>
    __device__ static __forceinline__ void apply(const uint8_t* base, int roff, int u, const Act (&a)[NE], int n,
                                                 float (&acc)[NE]) {
        const int b = S256 ? u : u >> 3;
        const int boff = roff + 210 * b;
        const float d = h2f(*(const uint16_t*)(base + boff + 208));
        int S[NE];
#pragma unroll
        for (int e = 0; e < NE; ++e) S[e] = 0;
        if (S256) {
#pragma unroll 1
            for (int gg = 0; gg < 8; ++gg) group<NE>(base, boff, gg, 256 * b + 32 * gg, a, n, S);
        } else {
            group<NE>(base, boff, u & 7, 32 * u, a, n, S);
        }
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            if (e >= n) break;
            acc[e] = __builtin_fmaf(d * a[e].d8[S256 ? 8 * b : u], (float)S[e], acc[e]);
        }
    }
};

// ---- Q8_0: unit = block u (34 bytes)
template <bool S256, int PAD>
struct Unit<kQ8_0, S256, PAD> {
    static constexpr int kUnit = 32;
    template <int NE>
    __device__ static __forceinline__ void apply(const uint8_t* base, int roff, int u, const Act (&a)[NE], int n,
                                                 float (&acc)[NE]) {
        const int boff = roff + 34 * u;
        const float d = h2f(*(const uint16_t*)(base + boff));
        uint32_t w[8];
        lds_words_a2<8>(base, boff + 2, w);
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            if (e >= n) break;
            const int8_t* x = a[e].q + 32 * u + PAD * (u >> 3);
            const uint4 l0 = *(const uint4*)x, l1 = *(const uint4*)(x + 16);
            const uint32_t al[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
            int is = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) is = sdot4((int)w[i], (int)al[i], is);
            acc[e] = __builtin_fmaf(d * a[e].d8[u], (float)is, acc[e]);
        }
    }
};

// ---- IQ4_XS: sub-block s: 16 qs bytes, low nibbles values 0..15, high 16..31, codebook kvalues_iq4nl, scale ls - 32
template <bool S256, int PAD>
struct Unit<kIQ4_XS, S256, PAD> {
    static constexpr int kUnit = S256 ? 256 : 32;
    template <int NE>
    __device__ static __forceinline__ void sub(const uint8_t* blk, uint2 hdr, int s, int v0, const Act (&a)[NE], int n,
                                               int (&S)[NE]) {
        const uint2 q0 = *(const uint2*)(blk + 8 + 16 * s), q1 = *(const uint2*)(blk + 16 + 16 * s);
        const uint32_t qw[4] = {q0.x, q0.y, q1.x, q1.y};
        const uint32_t t0 = kIq4Tab[0], t1 = kIq4Tab[1], t2 = kIq4Tab[2], t3 = kIq4Tab[3];
        int lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[i] = table16_lookup(qw[i] & 0x0F0F0F0Fu, t0, t1, t2, t3);
            hi[i] = table16_lookup((qw[i] >> 4) & 0x0F0F0F0Fu, t0, t1, t2, t3);
        }
        const uint32_t scales_h = hdr.x >> 16;
        const uint32_t sl = (hdr.y >> (8 * (s >> 1))) & 0xFFu;
        const int ls = (int)(((sl >> (4 * (s & 1))) & 0x0Fu) | (((scales_h >> (2 * s)) & 3u) << 4)) - 32;
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            if (e >= n) break;
            const int8_t* x = a[e].q + v0 + PAD * (v0 >> 8);
            const uint4 l0 = *(const uint4*)x, l1 = *(const uint4*)(x + 16);
            int is = 0;
            is = sdot4(lo[0], (int)l0.x, is);
            is = sdot4(lo[1], (int)l0.y, is);
            is = sdot4(lo[2], (int)l0.z, is);
            is = sdot4(lo[3], (int)l0.w, is);
            is = sdot4(hi[0], (int)l1.x, is);
            is = sdot4(hi[1], (int)l1.y, is);
            is = sdot4(hi[2], (int)l1.z, is);
            is = sdot4(hi[3], (int)l1.w, is);
            S[e] += ls * is;
        }
    }
    template <int NE>
    __device__ static __forceinline__ void apply(const uint8_t* base, int roff, int u, const Act (&a)[NE], int n,
                                                 float (&acc)[NE]) {
        const int b = S256 ? u : u >> 3;
        const uint8_t* blk = base + roff + 136 * b;
        const uint2 hdr = *(const uint2*)blk;
        const float d = h2f((uint16_t)(hdr.x & 0xFFFFu));
        int S[NE];
#pragma unroll
        for (int e = 0; e < NE; ++e) S[e] = 0;
        if (S256) {
#pragma unroll 1
            for (int s = 0; s < 8; ++s) sub<NE>(blk, hdr, s, 256 * b + 32 * s, a, n, S);
        } else {
            sub<NE>(blk, hdr, u & 7, 32 * u, a, n, S);
        }
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            if (e >= n) break;
            acc[e] = __builtin_fmaf(d * a[e].d8[S256 ? 8 * b : u], (float)S[e], acc[e]);
        }
    }
};

// L = min(8, the largest power of two dividing the unit count): the canonical lane count
__host__ __device__ constexpr int canon_lanes(int units) {
    int l = 8;
    while (l > 1 && units % l) l >>= 1;
    return l;
}

}  // namespace xs
