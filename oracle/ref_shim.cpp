// oracle/ref_shim.cpp - C entry points over the reference's own header-only host arithmetic, compiled (by
// oracle/Makefile, into oracle/_ref/) from include/strata/artifact/dequant.hpp and
// include/strata/kernels/canon_math.hpp where they lie in the reference tree.  TEST INFRASTRUCTURE: it validates
// oracle/xs_oracle.c's restatement and writes tests/golden's vectors; it is never part of the product.
#include "strata/artifact/dequant.hpp"
#include "strata/kernels/canon_math.hpp"

#include <cstdint>

extern "C" {

float xsref_fp16_to_fp32(uint16_t h) { return strata::fp16_to_fp32(h); }

// type ids are ggml's: Q8_0 8, Q4_K 12, Q6_K 14, IQ4_XS 23
int xsref_dequant(int type, const uint8_t* src, int64_t n_blocks, float* dst) {
    for (int64_t i = 0; i < n_blocks; ++i) {
        switch (type) {
            case 8: strata::dequantize_q8_0(src + 34 * i, dst + 32 * i); break;
            case 12: strata::dequantize_q4_K(src + 144 * i, dst + 256 * i); break;
            case 14: strata::dequantize_q6_K(src + 210 * i, dst + 256 * i); break;
            case 23: strata::dequantize_iq4_xs(src + 136 * i, dst + 256 * i); break;
            default: return -1;
        }
    }
    return 0;
}

void xsref_canon_exp(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = strata::kernels::canon::exp(x[i]);
}
void xsref_canon_rcp(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = strata::kernels::canon::rcp(x[i]);
}
void xsref_canon_silu_mul(const float* g, const float* u, int64_t n, float* h) {
    for (int64_t i = 0; i < n; ++i) h[i] = strata::kernels::canon::silu_mul(g[i], u[i]);
}
void xsref_canon_q8(const float* x, int64_t n, float* d, float* id, int8_t* q) {
    // n values as one block: the scale of their largest magnitude, its inverse, and each value's int8
    float amax = 0.0f;
    for (int64_t i = 0; i < n; ++i) amax = amax > (x[i] < 0 ? -x[i] : x[i]) ? amax : (x[i] < 0 ? -x[i] : x[i]);
    *d = strata::kernels::canon::q8_scale(amax);
    *id = strata::kernels::canon::q8_inv(*d);
    for (int64_t i = 0; i < n; ++i) q[i] = strata::kernels::canon::q8_value(x[i], *id);
}

}  // extern "C"
