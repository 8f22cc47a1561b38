/*
 * oracle/xs_oracle.c - CPU restatement of XeStrata's MoE-layer hot path.  TEST INFRASTRUCTURE ONLY (see
 * xs_oracle.h): the checker of the HIP library, never linked into it.
 *
 * Built with -ffp-contract=off: every product and sum below rounds on its own, as the reference library does
 * (CMakeLists.txt:396 `-fno-fast-math -ffp-contract=off`); fused multiply-adds are written out with fmaf where the
 * reference writes them (include/strata/kernels/canon_math.hpp).
 *
 * Parity pins (tests/test_oracle.py): dequantizers bit-for-bit against the reference's own dequant.hpp (compiled into
 * oracle/_ref here, and committed golden vectors); canonical math bit-for-bit against canon_math.hpp likewise; the
 * router against a stable-sort restatement on the reference test's seeded cases; the row dots against exact double
 * sums of dequantized operands; plan and permutation against brute-force group-bys.
 */
#include "xs_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ scalars */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* include/strata/artifact/dequant.hpp:36-56 (fp16_to_fp32: subnormals and infinities handled) */
float xso_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, f;
    if (e == 0) {
        if (m == 0) {
            f = sign << 31;
        } else {
            /* subnormal half: value m * 2^-24, exact in float */
            float v = (float)m * 5.9604644775390625e-08f;
            f = f2u(v) | (sign << 31);
        }
    } else if (e == 31) {
        f = (sign << 31) | 0x7F800000u | (m << 13);
    } else {
        f = (sign << 31) | ((e - 15 + 127) << 23) | (m << 13);
    }
    return u2f(f);
}

/* float -> fp16, round to nearest even (sycl::half(float), the q8_1 block's ds; iq_kernels.cpp q8_1_finite.hpp) */
uint16_t xso_fp32_to_fp16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);            /* rounds past 65504 */
    if (ax < 0x38800000u) {                                               /* below the smallest normal half */
        if (ax < 0x33000000u) return (uint16_t)sign;                      /* below half the smallest subnormal */
        const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        const int shift = 126 - (int)e;                                   /* value = m * 2^(e-150); unit 2^-24 */
        const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
        uint32_t r = q + ((rem > halfway || (rem == halfway && (q & 1u))) ? 1u : 0u);
        return (uint16_t)(sign | r);
    }
    const uint32_t e = (ax >> 23) - 127 + 15, m = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

static float h2f(const uint8_t* p) { return xso_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8))); }
static int32_t rd_i32(const uint8_t* p) { int32_t v; memcpy(&v, p, 4); return v; }

int xso_block_values(int type) { return type == XSO_Q8_0 ? 32 : (type == XSO_Q4_K || type == XSO_Q6_K || type == XSO_IQ4_XS) ? 256 : 0; }
static int block_bytes(int type) {
    switch (type) {
        case XSO_Q8_0: return 34;
        case XSO_Q4_K: return 144;
        case XSO_Q6_K: return 210;
        case XSO_IQ4_XS: return 136;
        default: return 0;
    }
}
int64_t xso_row_bytes(int type, int64_t n) {
    const int qk = xso_block_values(type);
    return qk ? (n / qk) * block_bytes(type) : 0;
}

/* ------------------------------------------------------------------------------------------------ dequant */

static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* include/strata/artifact/dequant.hpp:84-89 */
static void dq_q8_0(const uint8_t* b, float* y) {
    const float d = h2f(b);
    for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
}

/* the 6-bit scale and min of sub-block j (dequant.hpp:181-190) */
static void q4k_scale_min(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* dequant.hpp:192-209: value = (d * sc) * q - (dmin * m), each product rounded */
static void dq_q4_K(const uint8_t* b, float* y) {
    const float d = h2f(b), dmin = h2f(b + 2);
    const uint8_t* scales = b + 4;
    const uint8_t* q = b + 16;
    for (int p = 0; p < 4; ++p) {
        int sc, m;
        q4k_scale_min(2 * p, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        q4k_scale_min(2 * p + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) y[64 * p + l] = d1 * (float)(q[32 * p + l] & 0x0F) - m1;
        for (int l = 0; l < 32; ++l) y[64 * p + 32 + l] = d2 * (float)(q[32 * p + l] >> 4) - m2;
    }
}

/* dequant.hpp:152-175: two halves of 128; value = (d * sc) * (q - 32) */
static void dq_q6_K(const uint8_t* b, float* y) {
    const float d = h2f(b + 208);
    for (int n = 0; n < 2; ++n) {
        const uint8_t* ql = b + 64 * n;
        const uint8_t* qh = b + 128 + 32 * n;
        const int8_t* sc = (const int8_t*)(b + 192 + 8 * n);
        float* o = y + 128 * n;
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            o[l] = d * (float)sc[is] * (float)q1;
            o[l + 32] = d * (float)sc[is + 2] * (float)q2;
            o[l + 64] = d * (float)sc[is + 4] * (float)q3;
            o[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

/* dequant.hpp:283-299: 8 groups of 32, scale ls - 32 from scales_l / scales_h */
static void dq_iq4_xs(const uint8_t* b, float* y) {
    const float d = h2f(b);
    const unsigned scales_h = (unsigned)(b[2] | (b[3] << 8));
    const uint8_t* scales_l = b + 4;
    const uint8_t* qs = b + 8;
    for (int ib = 0; ib < 8; ++ib) {
        const int ls = ((scales_l[ib / 2] >> (4 * (ib % 2))) & 0x0F) | (((scales_h >> (2 * ib)) & 3) << 4);
        const float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; ++j) {
            y[32 * ib + j] = dl * (float)kIq4nl[qs[16 * ib + j] & 0x0F];
            y[32 * ib + j + 16] = dl * (float)kIq4nl[qs[16 * ib + j] >> 4];
        }
    }
}

void xso_dequant_row(int type, const uint8_t* src, int64_t n, float* dst) {
    const int qk = xso_block_values(type), bs = block_bytes(type);
    if (!qk) return;
    for (int64_t i = 0; i < n / qk; ++i) {
        const uint8_t* b = src + i * bs;
        float* y = dst + i * qk;
        switch (type) {
            case XSO_Q8_0: dq_q8_0(b, y); break;
            case XSO_Q4_K: dq_q4_K(b, y); break;
            case XSO_Q6_K: dq_q6_K(b, y); break;
            default: dq_iq4_xs(b, y); break;
        }
    }
}

/* ------------------------------------------------------------------------------------------------ canon */

/* canon_math.hpp:55-63: seed 0x7EF311C3 - bits(v), three Newton steps e = fma(-v, r, 1), r = fma(r, e, r) */
float xso_canon_rcp(float v) {
    float r = u2f(0x7EF311C3u - f2u(v));
    for (int i = 0; i < 3; ++i) {
        const float e = fmaf(-v, r, 1.0f);
        r = fmaf(r, e, r);
    }
    return r;
}

/* canon_math.hpp:67-82: clamp to [-80, 80], k = round(x / ln2) by the 1.5 * 2^23 trick, two-part ln2, degree 6 */
float xso_canon_exp(float x) {
    x = x < -80.0f ? -80.0f : x > 80.0f ? 80.0f : x;
    const float t = x * 1.44269504f;
    const float kf = (t + 12582912.0f) - 12582912.0f;
    float r = fmaf(-kf, 0.693145752f, x);
    r = fmaf(-kf, 1.42860677e-06f, r);
    float p = 1.0f / 720.0f;
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return u2f(f2u(p) + (uint32_t)((int32_t)kf << 23));
}

/* canon_math.hpp:85-89: g * rcp(1 + exp(-g)) * u, left to right */
float xso_canon_silu_mul(float g, float u) {
    const float den = 1.0f + xso_canon_exp(-g);
    const float a = g * xso_canon_rcp(den);
    return a * u;
}
void xso_canon_silu_mul_n(const float* g, const float* u, int64_t n, float* h) {
    for (int64_t i = 0; i < n; ++i) h[i] = xso_canon_silu_mul(g[i], u[i]);
}
void xso_canon_exp_n(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = xso_canon_exp(x[i]);
}
void xso_canon_rcp_n(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = xso_canon_rcp(x[i]);
}

/* canon_math.hpp:94-108 */
static float q8_scale(float amax) {
    const float d = amax * (1.0f / 127.0f);
    return d > 65504.0f ? 65504.0f : d;
}
static float q8_inv(float d) { return d >= 1e-30f ? xso_canon_rcp(d) : 0.0f; }
static int8_t q8_value(float x, float id) {
    const float t = x * id;
    const float r = t + (t < 0.0f ? -0.5f : 0.5f);
    const float c = r > 127.0f ? 127.0f : r < -127.0f ? -127.0f : r;
    return (int8_t)(int32_t)c;
}
/* src/kernels/xe/q8_1_finite.hpp:24 */
static float q8_1_finite(float v) { return fabsf(v) > 65504.0f ? copysignf(65504.0f, v) : v; }

static void put_ds(uint8_t* blk, float d, float s) {
    const uint16_t hd = xso_fp32_to_fp16(d), hs = xso_fp32_to_fp16(q8_1_finite(s));
    blk[0] = (uint8_t)hd; blk[1] = (uint8_t)(hd >> 8);
    blk[2] = (uint8_t)hs; blk[3] = (uint8_t)(hs >> 8);
}

/* the 32-lane xor butterfly sum of iq_kernels.cpp:823-826 (offsets 16, 8, 4, 2, 1), the value lane 0 ends with */
static float butterfly32(const float* v) {
    float a[32];
    memcpy(a, v, sizeof a);
    for (int o = 16; o > 0; o >>= 1) {
        float b[32];
        for (int i = 0; i < 32; ++i) b[i] = a[i] + a[i ^ o];
        memcpy(a, b, sizeof a);
    }
    return a[0];
}

/* per-32 canonical q8_1 (iq_kernels.cpp:1209-1223; also the SwiGLU pass's quantizer, :2118-2133) */
void xso_quantize_q8_1_per32(const float* x, int64_t n, uint8_t* y) {
    for (int64_t ib = 0; ib < n / 32; ++ib) {
        const float* v = x + 32 * ib;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
        const float sum = butterfly32(v);
        const float d = q8_scale(amax), id = q8_inv(d);
        uint8_t* blk = y + 36 * ib;
        for (int i = 0; i < 32; ++i) blk[4 + i] = (uint8_t)q8_value(v[i], id);
        put_ds(blk, d, sum);
    }
}

/* iq_kernels.cpp:1850-1879: rows of whole 256s take one scale for each 256 values (each of its 8 blocks stores it);
 * a block's sum is its 4 work-items' serial sums of 8, combined by xor 1 then xor 2.  Other widths: per-32. */
void xso_quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, uint8_t* y) {
    const int64_t n = n_rows * n_cols;
    if (n_cols % 256 != 0) { xso_quantize_q8_1_per32(x, n, y); return; }
    for (int64_t g = 0; g < n / 256; ++g) {
        const float* v = x + 256 * g;
        float amax = 0.0f;
        for (int i = 0; i < 256; ++i) amax = fmaxf(amax, fabsf(v[i]));
        const float d = q8_scale(amax), id = q8_inv(d);
        for (int b = 0; b < 8; ++b) {
            float s[4];
            for (int l = 0; l < 4; ++l) {
                float a = 0.0f;
                for (int q = 0; q < 8; ++q) a += v[32 * b + 8 * l + q];
                s[l] = a;
            }
            const float s01 = s[0] + s[1], s23 = s[2] + s[3];
            const float sum = s01 + s23;
            uint8_t* blk = y + 36 * (8 * g + b);
            for (int i = 0; i < 32; ++i) blk[4 + i] = (uint8_t)q8_value(v[32 * b + i], id);
            put_ds(blk, d, sum);
        }
    }
}

/* ------------------------------------------------------------------------------------------------ row dots */

static int dp4a(int32_t a, int32_t b, int c) {
    for (int i = 0; i < 4; ++i) c += (int)(int8_t)(a >> (8 * i)) * (int)(int8_t)(b >> (8 * i));
    return c;
}
static float q8d(const uint8_t* blk) { return h2f(blk); }                 /* low half of ds */
static int32_t q8u(const uint8_t* blk, int i) { return rd_i32(blk + 4 + 4 * i); }

/* Q4_K against q8_1 (iq_kernels.cpp:580-606 with vec_dot_q4_K_q8_1_impl_vmmq :435-447): call iqs = 0, 2, .., 30 of
 * block b covers 8 low nibbles (sub-block 2j) and 8 high (2j+1), j = iqs / 8; the min multiplies the sum of the
 * QUANTIZED activations */
static float dot_q4_K_call(const uint8_t* blk, const uint8_t* xb, int iqs) {
    const int off = 2 * (iqs / 8);
    const uint8_t* q4 = blk + 16 + 16 * off + 4 * ((iqs / 2) % 4);
    const int32_t v0 = rd_i32(q4), v1 = rd_i32(q4 + 16);
    float sumf_d = 0.0f, sumf_m = 0.0f;
    for (int i = 0; i < 2; ++i) {
        int sc, m;
        q4k_scale_min(off + i, blk + 4, &sc, &m);
        const uint8_t* b8 = xb + 36 * (off + i);
        const float d8 = q8d(b8);
        const int32_t u0 = q8u(b8, (iqs / 2) % 4), u1 = q8u(b8, (iqs / 2) % 4 + 4);
        const int32_t v0i = (v0 >> (4 * i)) & 0x0F0F0F0F, v1i = (v1 >> (4 * i)) & 0x0F0F0F0F;
        const int dot1 = dp4a(v1i, u1, dp4a(v0i, u0, 0));
        const int dot2 = dp4a(0x01010101, u1, dp4a(0x01010101, u0, 0));
        sumf_d += d8 * (float)(dot1 * sc);
        sumf_m += d8 * (float)(dot2 * m);
    }
    return h2f(blk) * sumf_d - h2f(blk + 2) * sumf_m;
}

/* Q6_K against q8_1 (iq_kernels.cpp:695-721): call iqs = 0..31 */
static float dot_q6_K_call(const uint8_t* blk, const uint8_t* xb, int iqs) {
    const int bq8 = 4 * (iqs / 16) + (iqs % 16) / 8;
    const int sco = 8 * (iqs / 16) + (iqs % 16) / 4;
    const int vh_shift = 2 * ((iqs % 16) / 8);
    const int32_t vl = rd_i32(blk + 4 * iqs);
    const int32_t vh = (int32_t)((uint32_t)rd_i32(blk + 128 + 4 * (8 * (iqs / 16) + iqs % 8)) >> vh_shift);
    float sumf = 0.0f;
    for (int i = 0; i < 2; ++i) {
        const uint8_t* b8 = xb + 36 * (bq8 + 2 * i);
        const int sc = (int8_t)blk[192 + sco + 4 * i];
        const uint32_t vil = ((uint32_t)vl >> (4 * i)) & 0x0F0F0F0Fu;
        const uint32_t vih = (((uint32_t)vh >> (4 * i)) << 4) & 0x30303030u;
        const uint32_t w = vil | vih;
        int32_t vi = 0;
        for (int b = 0; b < 4; ++b) vi |= (int32_t)((uint32_t)(uint8_t)((int)((w >> (8 * b)) & 0xFF) - 32) << (8 * b));
        sumf += q8d(b8) * (float)(dp4a(vi, q8u(b8, iqs % 8), 0) * sc);
    }
    return h2f(blk + 208) * sumf;
}

/* Q8_0 against q8_1 (iq_kernels.cpp:677-691): call iqs = 0, 2, 4, 6 */
static float dot_q8_0_call(const uint8_t* blk, const uint8_t* xb, int iqs) {
    int sumi = 0;
    for (int i = 0; i < 2; ++i) sumi = dp4a(rd_i32(blk + 2 + 4 * (iqs + i)), q8u(xb, iqs + i), sumi);
    return h2f(blk) * q8d(xb) * (float)sumi;
}

/* IQ4_XS against q8_1 (iq_kernels.cpp:398-428): the parts of sub-block sb: c = d * d8, t = sumi * (ls - 32) */
static void iq4xs_parts(const uint8_t* blk, const uint8_t* xb, int sb, float* c, int* t) {
    const unsigned scales_h = (unsigned)(blk[2] | (blk[3] << 8));
    const int ls = (((blk[4 + sb / 2] >> (4 * (sb % 2))) & 0x0F) | (((scales_h >> (2 * sb)) & 3) << 4)) - 32;
    const uint8_t* qs = blk + 8 + 16 * sb;
    const uint8_t* b8 = xb + 36 * sb;
    int sumi = 0;
    for (int j = 0; j < 16; ++j) {
        sumi += kIq4nl[qs[j] & 0x0F] * (int)(int8_t)b8[4 + j];
        sumi += kIq4nl[qs[j] >> 4] * (int)(int8_t)b8[4 + 16 + j];
    }
    *t = sumi * ls;
    *c = h2f(blk) * q8d(b8);
}

/* one row with the reference's per-call float expressions, calls in order (a cross-check of the canonical order below:
 * the same exact products, summed in another order); IQ4_XS against a 256-scale activation adds its block's 8 integer
 * sums first and takes one fma (seg_dot_canon, iq_kernels.cpp:832-884) */
float xso_vec_dot_calls(int type, const uint8_t* row, const uint8_t* xq, int64_t n, int s256) {
    const int qk = xso_block_values(type), bs = block_bytes(type);
    float s = 0.0f;
    for (int64_t kb = 0; kb < n / qk; ++kb) {
        const uint8_t* blk = row + kb * bs;
        const uint8_t* xb = xq + 36 * (kb * (qk / 32));
        switch (type) {
            case XSO_Q4_K:
                for (int iqs = 0; iqs < 32; iqs += 2) s += dot_q4_K_call(blk, xb, iqs);
                break;
            case XSO_Q6_K:
                for (int iqs = 0; iqs < 32; ++iqs) s += dot_q6_K_call(blk, xb, iqs);
                break;
            case XSO_Q8_0:
                for (int iqs = 0; iqs < 8; iqs += 2) s += dot_q8_0_call(blk, xb, iqs);
                break;
            default: {
                if (s256) {
                    float c = 0.0f;
                    int t = 0;
                    for (int sb = 0; sb < 8; ++sb) {
                        float cs;
                        int ts;
                        iq4xs_parts(blk, xb, sb, &cs, &ts);
                        c = cs;
                        t += ts;
                    }
                    s = fmaf(c, (float)t, s);
                } else {
                    for (int sb = 0; sb < 8; ++sb) {
                        float c;
                        int t;
                        iq4xs_parts(blk, xb, sb, &c, &t);
                        s += c * (float)t;
                    }
                }
            }
        }
    }
    return s;
}

/* ---- the canonical row order (the order of the HIP kernels, so device and host agree bit for bit)
 *
 * The reference fixes one float order for the i-quant rows it keeps bitwise between its devices (seg_dot_canon,
 * src/kernels/xe/iq_kernels.cpp:832-884; include/strata/kernels/canon_math.hpp): the exact integer sums of the calls
 * that share one activation scale first, then one written-out fma a group, lane-strided, then a butterfly.  The
 * canonical order here extends that to every format:
 *   unit   = the values that share one weight scale set and one activation scale: a whole 256-value block when the
 *            activation has one scale for each 256 (the gate/up rows: quantize_q8_1_rows), else 32 values (the down
 *            rows, and Q8_0 blocks);
 *   term   = its exact integer sums S (codes times int8 activations, scales applied in integers), then
 *            acc = fma(d * d8, (float) S, acc)  [Q4_K also acc = fma(-(dmin * d8), (float) Smin, acc)];
 *   row    = L = min(8, largest power of two dividing the unit count) lanes; lane c adds units c, c + L, ... in order;
 *            then a butterfly: acc[c] += acc[c ^ o] for o = L/2 .. 1; the row is lane 0's value. */
static int act(const uint8_t* xq, int64_t i) { return (int)(int8_t)xq[36 * (i / 32) + 4 + i % 32]; }
static float actd(const uint8_t* xq, int64_t g) { return h2f(xq + 36 * g); }

static int q4k_code(const uint8_t* blk, int v) { return (blk[16 + 32 * (v / 64) + v % 32] >> (4 * ((v / 32) % 2))) & 15; }
static int q6k_code(const uint8_t* blk, int v) {
    const int n = v / 128, s = (v % 128) / 32, l = v % 32;
    return (((blk[64 * n + 32 * (s & 1) + l] >> (4 * (s >> 1))) & 15) | (((blk[128 + 32 * n + l] >> (2 * s)) & 3) << 4)) - 32;
}
static int iq4xs_ls(const uint8_t* blk, int sb) {
    const unsigned scales_h = (unsigned)(blk[2] | (blk[3] << 8));
    return (((blk[4 + sb / 2] >> (4 * (sb % 2))) & 0x0F) | (((scales_h >> (2 * sb)) & 3) << 4)) - 32;
}
static int iq4xs_code(const uint8_t* blk, int v) {
    const uint8_t q = blk[8 + 16 * (v / 32) + v % 16];
    return kIq4nl[(v % 32) < 16 ? (q & 0x0F) : (q >> 4)];
}

/* unit u of a row against xq (q8_1 of the row's n values); s256: one activation scale a 256 */
static float canon_unit(int type, const uint8_t* row, int64_t u, const uint8_t* xq, int s256, float acc) {
    if (type == XSO_Q8_0) {
        const uint8_t* blk = row + 34 * u;
        int s = 0;
        for (int i = 0; i < 32; ++i) s += (int)(int8_t)blk[2 + i] * act(xq, 32 * u + i);
        return fmaf(h2f(blk) * actd(xq, u), (float)s, acc);
    }
    const int bs = block_bytes(type);
    const int64_t b = s256 ? u : u / 8;                    /* the block */
    const int g0 = s256 ? 0 : (int)(u % 8), g1 = s256 ? 8 : g0 + 1;   /* its 32-value groups in this unit */
    const uint8_t* blk = row + b * bs;
    const int64_t v0 = 256 * b;
    const float d8 = actd(xq, 8 * b + g0);
    if (type == XSO_Q4_K) {
        int s1 = 0, s2 = 0;
        for (int g = g0; g < g1; ++g) {
            int sc, m, is = 0, us = 0;
            q4k_scale_min(g, blk + 4, &sc, &m);
            for (int l = 0; l < 32; ++l) {
                const int a = act(xq, v0 + 32 * g + l);
                is += q4k_code(blk, 32 * g + l) * a;
                us += a;
            }
            s1 += sc * is;
            s2 += m * us;
        }
        acc = fmaf(h2f(blk) * d8, (float)s1, acc);
        return fmaf(-(h2f(blk + 2) * d8), (float)s2, acc);
    }
    if (type == XSO_Q6_K) {
        int s = 0;
        for (int j = 2 * g0; j < 2 * g1; ++j) {             /* 16-value sub-blocks */
            int is = 0;
            for (int l = 0; l < 16; ++l) is += q6k_code(blk, 16 * j + l) * act(xq, v0 + 16 * j + l);
            s += (int)(int8_t)blk[192 + j] * is;
        }
        return fmaf(h2f(blk + 208) * d8, (float)s, acc);
    }
    /* IQ4_XS */
    int s = 0;
    for (int g = g0; g < g1; ++g) {
        int is = 0;
        for (int l = 0; l < 32; ++l) is += iq4xs_code(blk, 32 * g + l) * act(xq, v0 + 32 * g + l);
        s += iq4xs_ls(blk, g) * is;
    }
    return fmaf(h2f(blk) * d8, (float)s, acc);
}

int xso_canon_lanes(int64_t units) {
    int l = 8;
    while (l > 1 && units % l) l >>= 1;
    return l;
}

float xso_vec_dot(int type, const uint8_t* row, const uint8_t* xq, int64_t n, int s256) {
    const int su = (type != XSO_Q8_0) && s256;
    const int64_t units = su ? n / 256 : n / 32;
    const int L = xso_canon_lanes(units);
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < L; ++c)
        for (int64_t u = c; u < units; u += L) acc[c] = canon_unit(type, row, u, xq, su, acc[c]);
    for (int o = L / 2; o > 0; o >>= 1) {
        float b[8];
        for (int c = 0; c < L; ++c) b[c] = acc[c] + acc[c ^ o];
        memcpy(acc, b, sizeof b);
    }
    return acc[0];
}

/* ------------------------------------------------------------------------------------------------ experts */

/* iq_kernels.cpp:2002-2036 (native_expert_layout: gate rows, then up rows of up_type's row bytes, then down rows) */
int xso_native_layout_mixed(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, int up_type, xso_layout* L) {
    const int qg = xso_block_values(gu_type), qd = xso_block_values(d_type), qu = xso_block_values(up_type);
    if (!qg || !qd || !qu || n_embd <= 0 || n_ff <= 0 || n_embd % qg || n_embd % qu || n_ff % qd || n_embd % 256)
        return 0;
    L->gu_type = gu_type;
    L->d_type = d_type;
    L->up_type = up_type;
    L->n_embd = n_embd;
    L->n_ff = n_ff;
    L->gu_row = xso_row_bytes(gu_type, n_embd);
    L->up_row = xso_row_bytes(up_type, n_embd);
    L->d_row = xso_row_bytes(d_type, n_ff);
    L->up_off = n_ff * L->gu_row;
    L->down_off = L->up_off + n_ff * L->up_row;
    L->bytes = L->down_off + n_embd * L->d_row;
    return 1;
}
int xso_native_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, xso_layout* L) {
    return xso_native_layout_mixed(gu_type, d_type, n_embd, n_ff, gu_type, L);
}

/* iq_kernels.cpp:2042-2178 (launch_native_gu :997-1031, SwiGLU + q8_1 :2118-2133, launch_native_down :1033-1063) */
void xso_native_expert_grouped(const xso_layout* L, const uint8_t* const* blobs, const int32_t* start, int n_groups,
                               const int32_t* ent_dst, const int32_t* ent_tok, const uint8_t* x_q8_1, float* out,
                               float* gate_out, float* up_out, uint8_t* hq_out, int n_threads) {
    const int64_t H = L->n_embd, F = L->n_ff, xb = H / 32 * 36;
    const int n_ent = start[n_groups] - start[0];
    (void)n_threads;
    float* gate = (float*)malloc(sizeof(float) * (size_t)(F > 0 ? F : 1) * (size_t)(n_ent > 0 ? n_ent : 1));
    float* up = (float*)malloc(sizeof(float) * (size_t)(F > 0 ? F : 1) * (size_t)(n_ent > 0 ? n_ent : 1));
    uint8_t* hq = (uint8_t*)malloc((size_t)(F / 32 * 36) * (size_t)(n_ent > 0 ? n_ent : 1));
    for (int g = 0; g < n_groups; ++g) {
        const uint8_t* blob = blobs[g];
        for (int e = start[g]; e < start[g + 1]; ++e) {
            const int le = e - start[0];
            const uint8_t* x = x_q8_1 + (int64_t)ent_tok[e] * xb;
#ifdef _OPENMP
#pragma omp parallel for num_threads(n_threads > 0 ? n_threads : 1) schedule(static)
#endif
            for (int64_t r = 0; r < F; ++r) {
                gate[(int64_t)le * F + r] = xso_vec_dot(L->gu_type, blob + r * L->gu_row, x, H, 1);
                up[(int64_t)le * F + r] = xso_vec_dot((int)L->up_type, blob + L->up_off + r * L->up_row, x, H, 1);
            }
            float* h = (float*)malloc(sizeof(float) * (size_t)F);
            for (int64_t r = 0; r < F; ++r) h[r] = xso_canon_silu_mul(gate[(int64_t)le * F + r], up[(int64_t)le * F + r]);
            xso_quantize_q8_1_per32(h, F, hq + (int64_t)le * (F / 32 * 36));
            free(h);
            float* o = out + (int64_t)ent_dst[e] * H;
            const uint8_t* hrow = hq + (int64_t)le * (F / 32 * 36);
#ifdef _OPENMP
#pragma omp parallel for num_threads(n_threads > 0 ? n_threads : 1) schedule(static)
#endif
            for (int64_t r = 0; r < H; ++r) o[r] = xso_vec_dot(L->d_type, blob + L->down_off + r * L->d_row, hrow, F, 0);
        }
    }
    if (gate_out) memcpy(gate_out, gate, sizeof(float) * (size_t)F * (size_t)n_ent);
    if (up_out) memcpy(up_out, up, sizeof(float) * (size_t)F * (size_t)n_ent);
    if (hq_out) memcpy(hq_out, hq, (size_t)(F / 32 * 36) * (size_t)n_ent);
    free(gate);
    free(up);
    free(hq);
}

/* ------------------------------------------------------------------------------------------------ router */

/* src/kernels/xe/router.cpp:59-145: softmax over every expert (float max; exp in double of l - mx; the sum serial
 * and ascending in double; inv = (float)(1 / sum); p = (float)(ex * inv)), k passes of an argmax that takes the
 * larger p and on a tie the lower index (NaN never wins), then w = (float)(w / max(sum of the k in rank order,
 * 2^-14)) in double.  A row whose ranks run out (NaN) leaves the remaining ranks as they were. */
void xso_router_top10(const float* logits, int n_tokens, int n_expert, int k, int32_t* ids, float* weights) {
    double* ex = (double*)malloc(sizeof(double) * (size_t)n_expert);
    float* p = (float*)malloc(sizeof(float) * (size_t)n_expert);
    unsigned char* taken = (unsigned char*)malloc((size_t)n_expert);
    for (int t = 0; t < n_tokens; ++t) {
        const float* l = logits + (int64_t)t * n_expert;
        float mx = -INFINITY;
        for (int x = 0; x < n_expert; ++x) mx = fmaxf(mx, l[x]);
        for (int x = 0; x < n_expert; ++x) ex[x] = exp((double)l[x] - (double)mx);
        double sum = 0.0;
        for (int x = 0; x < n_expert; ++x) sum += ex[x];
        const float inv = (float)(1.0 / sum);
        for (int x = 0; x < n_expert; ++x) { p[x] = (float)(ex[x] * (double)inv); taken[x] = 0; }
        int nsel = 0;
        for (int i = 0; i < k; ++i) {
            float bv = -INFINITY;
            int bi = n_expert;
            for (int x = 0; x < n_expert; ++x) {
                if (taken[x]) continue;
                if (p[x] > bv) { bv = p[x]; bi = x; }
            }
            if (bi >= n_expert) break;
            ids[(int64_t)t * k + i] = bi;
            weights[(int64_t)t * k + i] = bv;
            taken[bi] = 1;
            nsel = i + 1;
        }
        (void)nsel;
        double s = 0.0;
        for (int i = 0; i < k; ++i) s += (double)weights[(int64_t)t * k + i];
        const double sc = fmax(s, 6.103515625e-05);
        for (int i = 0; i < k; ++i) weights[(int64_t)t * k + i] = (float)((double)weights[(int64_t)t * k + i] / sc);
    }
    free(ex);
    free(p);
    free(taken);
}

/* DeepSeek-V3 routing from its published description (no reference implementation exists in XeStrata): s =
 * sigmoid(l) = rcp(1 + exp(-l)) with the canonical exp and reciprocal (canon_math.hpp's, so host and device agree
 * bit for bit); selection scores s + bias; a group's score is the sum of its two largest
 * selection scores; the topk_group best groups (ties: lower group index); the k best selection scores inside them
 * (ties: lower expert index), in descending order; weights are the unbiased s of the chosen, divided by their sum
 * (accumulated in rank order in float) and times routed_scale. */
void xso_router_grouped_sigmoid(const float* logits, const float* bias, int n_tokens, int n_expert, int n_group,
                                int topk_group, int k, float routed_scale, int32_t* ids, float* weights) {
    const int per = n_expert / n_group;
    float* s = (float*)malloc(sizeof(float) * (size_t)n_expert);
    float* c = (float*)malloc(sizeof(float) * (size_t)n_expert);
    float* gs = (float*)malloc(sizeof(float) * (size_t)n_group);
    unsigned char* gsel = (unsigned char*)malloc((size_t)n_group);
    unsigned char* taken = (unsigned char*)malloc((size_t)n_expert);
    for (int t = 0; t < n_tokens; ++t) {
        const float* l = logits + (int64_t)t * n_expert;
        for (int e = 0; e < n_expert; ++e) {
            s[e] = xso_canon_rcp(1.0f + xso_canon_exp(-l[e]));
            c[e] = s[e] + (bias ? bias[e] : 0.0f);
            taken[e] = 0;
        }
        for (int g = 0; g < n_group; ++g) {
            float b1 = -INFINITY, b2 = -INFINITY;
            for (int j = 0; j < per; ++j) {
                const float v = c[g * per + j];
                if (v > b1) { b2 = b1; b1 = v; }
                else if (v > b2) b2 = v;
            }
            gs[g] = b1 + b2;
            gsel[g] = 0;
        }
        for (int i = 0; i < topk_group; ++i) {
            float bv = -INFINITY;
            int bg = -1;
            for (int g = 0; g < n_group; ++g)
                if (!gsel[g] && (bg < 0 || gs[g] > bv)) { bv = gs[g]; bg = g; }
            gsel[bg] = 1;
        }
        float sum = 0.0f;
        for (int i = 0; i < k; ++i) {
            float bv = -INFINITY;
            int be = -1;
            for (int e = 0; e < n_expert; ++e)
                if (gsel[e / per] && !taken[e] && (be < 0 || c[e] > bv)) { bv = c[e]; be = e; }
            taken[be] = 1;
            ids[(int64_t)t * k + i] = be;
            weights[(int64_t)t * k + i] = s[be];
            sum += s[be];
        }
        for (int i = 0; i < k; ++i) weights[(int64_t)t * k + i] = weights[(int64_t)t * k + i] / sum * routed_scale;
    }
    free(s);
    free(c);
    free(gs);
    free(gsel);
    free(taken);
}

/* ------------------------------------------------------------------------------------------------ plans */

/* resident_plan's contract (verify_kernels.cpp:819-890; host replay resident_plan_parity.cpp:60-96): groups are the
 * distinct experts in order of first occurrence, a group's entries ascending; dst = entry index, tok = entry / k */
int xso_decode_plan(const int32_t* ids, int n, int k, int32_t* counts, int32_t* start, int32_t* dst, int32_t* tok,
                    int32_t* group_expert) {
    int groups = 0;
    for (int i = 0; i < n; ++i) {
        int seen = 0;
        for (int g = 0; g < groups; ++g) seen |= group_expert[g] == ids[i];
        if (!seen) group_expert[groups++] = ids[i];
    }
    int pos = 0;
    for (int g = 0; g < groups; ++g) {
        start[g] = pos;
        for (int i = 0; i < n; ++i)
            if (ids[i] == group_expert[g]) { dst[pos] = i; tok[pos] = i / k; ++pos; }
    }
    start[groups] = n;
    counts[0] = groups;
    counts[1] = n;
    counts[2] = 0;
    return groups;
}

/* src/prefill/plain_prompt.cpp:576-637 with every expert on the GPU: count[e]; experts ascending; start = exclusive
 * prefix; a stable fill over entries i: row = fill[e]++, src[row] = i / k, slot[i] = row, entry[row] = i; bounds =
 * the starts of the experts with rows, then the total */
int xso_prefill_route(const int32_t* ids, int64_t n_entries, int k, int n_expert, int32_t* src, int32_t* slot,
                      int32_t* entry, int32_t* bounds, int32_t* experts, int32_t* counts) {
    int32_t* cnt = (int32_t*)calloc((size_t)n_expert, sizeof(int32_t));
    int32_t* st = (int32_t*)calloc((size_t)n_expert, sizeof(int32_t));
    for (int64_t i = 0; i < n_entries; ++i) ++cnt[ids[i]];
    int32_t at = 0;
    int groups = 0;
    for (int e = 0; e < n_expert; ++e) {
        if (counts) counts[e] = cnt[e];
        if (cnt[e] > 0) {
            st[e] = at;
            bounds[groups] = at;
            experts[groups++] = e;
            at += cnt[e];
        }
    }
    bounds[groups] = at;
    for (int64_t i = 0; i < n_entries; ++i) {
        const int32_t e = ids[i], row = st[e]++;
        src[row] = (int32_t)(i / k);
        slot[i] = row;
        entry[row] = (int32_t)i;
    }
    free(cnt);
    free(st);
    return groups;
}

/* ------------------------------------------------------------------------------------------------ combine */

/* src/kernels/xe/native_moe.cpp:36-58: fl(p0 w0), then + fl(pj wj) in rank order, then + shared (times the gate's
 * sigmoid 1 / (1 + exp(-g)), its product rounded, when gated) */
void xso_combine(const float* parts, const float* weights, const float* shared, const float* shared_gate, float* out,
                 int64_t n_embd, int k, int n_tok) {
    for (int t = 0; t < n_tok; ++t) {
        const float* p = parts + (int64_t)t * k * n_embd;
        const float* w = weights + (int64_t)t * k;
        for (int64_t c = 0; c < n_embd; ++c) {
            float sum = p[c] * w[0];
            for (int e = 1; e < k; ++e) {
                const float prod = p[(int64_t)e * n_embd + c] * w[e];
                sum = sum + prod;
            }
            if (shared) {
                float sv = shared[(int64_t)t * n_embd + c];
                if (shared_gate) {
                    const float gt = 1.0f / (1.0f + expf(-shared_gate[t]));
                    sv = sv * gt;
                }
                sum += sv;
            }
            out[(int64_t)t * n_embd + c] = sum;
        }
    }
}

/* A shared expert over n_tok tokens: one group holding every token (the engine's shared-expert decode,
 * src/core/plain_model.cpp:959-973, on the same canonical rows as the routed experts). */
void xso_shared_expert(const xso_layout* SL, const uint8_t* blob, const float* x, int n_tok, float* shared,
                       int n_threads) {
    const int64_t H = SL->n_embd;
    uint8_t* xq = (uint8_t*)malloc((size_t)(H / 32 * 36) * (size_t)n_tok);
    int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)n_tok);
    int32_t start[2] = {0, n_tok};
    const uint8_t* blobs[1] = {blob};
    for (int t = 0; t < n_tok; ++t) idx[t] = t;
    xso_quantize_q8_1_rows(x, n_tok, H, xq);
    xso_native_expert_grouped(SL, blobs, start, 1, idx, idx, xq, shared, NULL, NULL, NULL, n_threads);
    free(xq); free(idx);
}

/* The decode layer with a shared expert: the routed layer's combine then + the shared row once (times
 * 1 / (1 + exp(-gate_logit[t])) when given), then the residual (plain_model.cpp:951-988). */
void xso_moe_layer_decode_shared(const xso_layout* L, const uint8_t* const* blobs_by_expert, int n_expert, int k,
                                 const float* x, const float* logits, const float* residual, int n_tok,
                                 const xso_layout* SL, const uint8_t* shared_blob, const float* gate_logit, float* out,
                                 int n_threads) {
    const int64_t H = L->n_embd, n = (int64_t)n_tok * k;
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    float* w = (float*)malloc(sizeof(float) * (size_t)n);
    int32_t counts[4], *start = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n + 1));
    int32_t* dst = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    int32_t* gexp = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    uint8_t* xq = (uint8_t*)malloc((size_t)(H / 32 * 36) * (size_t)n_tok);
    float* parts = (float*)malloc(sizeof(float) * (size_t)(n * H));
    float* shared = (float*)malloc(sizeof(float) * (size_t)((int64_t)n_tok * H));
    const uint8_t** gblob = (const uint8_t**)malloc(sizeof(void*) * (size_t)n);
    xso_router_top10(logits, n_tok, n_expert, k, ids, w);
    const int groups = xso_decode_plan(ids, (int)n, k, counts, start, dst, tok, gexp);
    for (int g = 0; g < groups; ++g) gblob[g] = blobs_by_expert[gexp[g]];
    xso_quantize_q8_1_rows(x, n_tok, H, xq);
    xso_native_expert_grouped(L, gblob, start, groups, dst, tok, xq, parts, NULL, NULL, NULL, n_threads);
    xso_shared_expert(SL, shared_blob, x, n_tok, shared, n_threads);
    xso_combine(parts, w, shared, gate_logit, out, H, k, n_tok);
    for (int64_t i = 0; i < (int64_t)n_tok * H; ++i) out[i] = residual[i] + out[i];
    free(ids); free(w); free(start); free(dst); free(tok); free(gexp); free(xq); free(parts); free(shared); free(gblob);
}

/* ------------------------------------------------------------------------------------------------ float reference */

/* src/kernels/native_expert_parity.cpp:104-130 */
void xso_expert_float(const xso_layout* L, const uint8_t* const* blobs, const float* x, const int32_t* tok, int n,
                      float* out, int n_threads) {
    const int64_t H = L->n_embd, F = L->n_ff;
    (void)n_threads;
    for (int j = 0; j < n; ++j) {
        const uint8_t* blob = blobs[j];
        const float* xr = x + (int64_t)tok[j] * H;
        float* h = (float*)malloc(sizeof(float) * (size_t)F);
#ifdef _OPENMP
#pragma omp parallel for num_threads(n_threads > 0 ? n_threads : 1) schedule(static)
#endif
        for (int64_t r = 0; r < F; ++r) {
            float* wg = (float*)malloc(sizeof(float) * (size_t)H);
            float* wu = (float*)malloc(sizeof(float) * (size_t)H);
            xso_dequant_row(L->gu_type, blob + r * L->gu_row, H, wg);
            xso_dequant_row((int)L->up_type, blob + L->up_off + r * L->up_row, H, wu);
            double g = 0.0, u = 0.0;
            for (int64_t i = 0; i < H; ++i) { g += (double)wg[i] * xr[i]; u += (double)wu[i] * xr[i]; }
            h[r] = (float)(g / (1.0 + exp(-g)) * u);
            free(wg);
            free(wu);
        }
#ifdef _OPENMP
#pragma omp parallel for num_threads(n_threads > 0 ? n_threads : 1) schedule(static)
#endif
        for (int64_t r = 0; r < H; ++r) {
            float* wd = (float*)malloc(sizeof(float) * (size_t)F);
            xso_dequant_row(L->d_type, blob + L->down_off + r * L->d_row, F, wd);
            double o = 0.0;
            for (int64_t i = 0; i < F; ++i) o += (double)wd[i] * h[i];
            out[(int64_t)j * H + r] = (float)o;
            free(wd);
        }
        free(h);
    }
}

/* ------------------------------------------------------------------------------------------------ the layer */

void xso_moe_layer_decode(const xso_layout* L, const uint8_t* const* blobs_by_expert, int n_expert, int k,
                          const float* x, const float* logits, const float* residual, int n_tok, float* out,
                          int n_threads) {
    const int64_t H = L->n_embd, n = (int64_t)n_tok * k;
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    float* w = (float*)malloc(sizeof(float) * (size_t)n);
    int32_t counts[4], *start = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n + 1));
    int32_t* dst = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    int32_t* gexp = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    uint8_t* xq = (uint8_t*)malloc((size_t)(H / 32 * 36) * (size_t)n_tok);
    float* parts = (float*)malloc(sizeof(float) * (size_t)(n * H));
    const uint8_t** gblob = (const uint8_t**)malloc(sizeof(void*) * (size_t)n);
    (void)n_expert;
    xso_router_top10(logits, n_tok, n_expert, k, ids, w);
    const int groups = xso_decode_plan(ids, (int)n, k, counts, start, dst, tok, gexp);
    for (int g = 0; g < groups; ++g) gblob[g] = blobs_by_expert[gexp[g]];
    xso_quantize_q8_1_rows(x, n_tok, H, xq);
    xso_native_expert_grouped(L, gblob, start, groups, dst, tok, xq, parts, NULL, NULL, NULL, n_threads);
    xso_combine(parts, w, NULL, NULL, out, H, k, n_tok);
    for (int64_t i = 0; i < (int64_t)n_tok * H; ++i) out[i] = residual[i] + out[i];
    free(ids); free(w); free(start); free(dst); free(tok); free(gexp); free(xq); free(parts); free(gblob);
}

/* ------------------------------------------------------------------------------------------------ router projections */

static float bf(uint16_t b) { return u2f((uint32_t)b << 16); }

/* the 32-lane xor butterfly of warp_sum (src/kernels/xe/bf16_gemv.cpp:43-46): v[l] += v[l ^ off], off 16 .. 1, all
 * lanes at once; lane 0's value */
static float butterfly32_sum(float* v) {
    for (int off = 16; off > 0; off >>= 1) {
        float n[32];
        for (int l = 0; l < 32; ++l) n[l] = v[l] + v[l ^ off];
        memcpy(v, n, sizeof n);
    }
    return v[0];
}

/* mmvf_block_size (bf16_gemv.cpp:213-225) */
int xso_mmvf_block(int64_t n_in) {
    int best = 32;
    int64_t best_it = (n_in + 63) / 64;
    for (int c = 64; c <= 256; c += 32) {
        const int64_t it = (n_in + 2 * c - 1) / (2 * c);
        if (it < best_it) { best_it = it; best = c; }
    }
    return best;
}

/* launch_mmvf (bf16_gemv.cpp:91-147): w_bf16 non-NULL selects the BF16 weights, else w_f32 */
void xso_mmvf(const float* x, int64_t ldx, const float* w_f32, const uint16_t* w_bf16, float* y, int64_t ldy,
              int64_t n_in, int64_t n_out, int n_tok) {
    const int B = xso_mmvf_block(n_in);
    const int64_t pairs = n_in / 2;
    float* acc = (float*)malloc(sizeof(float) * (size_t)B);
    for (int64_t o = 0; o < n_out; ++o)
        for (int k = 0; k < n_tok; ++k) {
            for (int t = 0; t < B; ++t) {
                float a = 0.0f;
                for (int64_t p = t; p < pairs; p += B) {
                    const float w0 = w_bf16 ? bf(w_bf16[o * n_in + 2 * p]) : w_f32[o * n_in + 2 * p];
                    const float w1 = w_bf16 ? bf(w_bf16[o * n_in + 2 * p + 1]) : w_f32[o * n_in + 2 * p + 1];
                    a = fmaf(w0, x[k * ldx + 2 * p], a);
                    a = fmaf(w1, x[k * ldx + 2 * p + 1], a);
                }
                acc[t] = a;
            }
            float part[32] = {0};
            for (int g = 0; g < B / 32; ++g) {
                float v[32];
                memcpy(v, acc + 32 * g, sizeof v);
                part[g] = butterfly32_sum(v);
            }
            y[k * ldy + o] = B > 32 ? butterfly32_sum(part) : part[0];
        }
    free(acc);
}

/* f32_gemm_rows (bf16_gemv.cpp:475-502): acc = fma(x[t][k], w[o][k], acc), k up to the next multiple of 16 (zeros) */
void xso_gemm_rows(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in, int64_t n_out,
                   int64_t n_tok) {
    const int64_t k_end = (n_in + 15) / 16 * 16;
    for (int64_t t = 0; t < n_tok; ++t)
        for (int64_t o = 0; o < n_out; ++o) {
            float a = 0.0f;
            for (int64_t k = 0; k < k_end; ++k)
                a = k < n_in ? fmaf(x[t * ldx + k], w[o * n_in + k], a) : fmaf(0.0f, 0.0f, a);
            y[t * ldy + o] = a;
        }
}

/* bf16 x . bf16 rows: form 0 launch_warp (bf16_gemv.cpp:62-77), 1 launch_naive (50-60), 2 the split tree at tpr
 * threads (318-339).  Products of bf16 values are exact in f32, so fmaf and the reference's `acc += a * b` agree. */
void xso_bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out, int form, int tpr) {
    const int lanes = form == 0 ? 32 : form == 1 ? 1 : tpr;
    float* acc = (float*)malloc(sizeof(float) * (size_t)lanes);
    for (int64_t o = 0; o < n_out; ++o) {
        for (int l = 0; l < lanes; ++l) {
            float a = 0.0f;
            for (int64_t i = l; i < n_in; i += lanes) a = fmaf(bf(x[i]), bf(w[o * n_in + i]), a);
            acc[l] = a;
        }
        if (form == 0) y[o] = butterfly32_sum(acc);
        else if (form == 1) y[o] = acc[0];
        else {
            for (int off = lanes >> 1; off > 0; off >>= 1)
                for (int l = 0; l < off; ++l) acc[l] = acc[l] + acc[l + off];
            y[o] = acc[0];
        }
    }
    free(acc);
}
