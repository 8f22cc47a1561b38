// xestrata-win_amd/csrc/xs_dequant.h - 32 values of a GGUF block to fp32, the reference's host dequantizers' values
// bit for bit (reference include/strata/artifact/dequant.hpp:84-89 Q8_0, 152-175 Q6_K, 181-209 Q4_K, 283-299
// IQ4_XS): each product and difference rounds on its own (no fused multiply-add), as there.
#pragma once

#include "xs_device.h"

namespace xs {

__device__ __forceinline__ float rd_h(const uint8_t* p) { return h2f((uint16_t)(p[0] | (p[1] << 8))); }

__device__ __forceinline__ int8_t iq4nl_value(int i) {
    const int8_t t[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    return t[i];
}

// values [32 g, 32 g + 32) of the block at b (g < block_values(type) / 32)
__device__ __forceinline__ void dequant32(int type, const uint8_t* b, int g, float* y) {
    switch (type) {
        case kQ8_0: {
            const float d = rd_h(b);
            for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
            break;
        }
        case kQ4_K: {
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
            const uint8_t* qs = b + 16 + 32 * (g / 2);
            const int sh = 4 * (g % 2);
            for (int l = 0; l < 32; ++l) y[l] = d1 * (float)((qs[l] >> sh) & 0x0F) - m1;
            break;
        }
        case kQ6_K: {
            const float d = rd_h(b + 208);
            const int n = g / 4, s = g % 4;   // half n, 32-value group s of it
            const uint8_t* ql = b + 64 * n + 32 * (s & 1);
            const uint8_t* qh = b + 128 + 32 * n;
            const int8_t* sc = (const int8_t*)(b + 192 + 8 * n);
            const int nsh = 4 * (s >> 1), hsh = 2 * s;
            for (int l = 0; l < 32; ++l) {
                const int q = (int)(((ql[l] >> nsh) & 0x0F) | (((qh[l] >> hsh) & 3) << 4)) - 32;
                y[l] = d * (float)sc[2 * s + l / 16] * (float)q;
            }
            break;
        }
        default: {
            const float d = rd_h(b);
            const unsigned scales_h = (unsigned)(b[2] | (b[3] << 8));
            const int ls = ((b[4 + g / 2] >> (4 * (g % 2))) & 0x0F) | (((scales_h >> (2 * g)) & 3) << 4);
            const float dl = d * (float)(ls - 32);
            const uint8_t* qs = b + 8 + 16 * g;
            for (int j = 0; j < 16; ++j) {
                y[j] = dl * (float)iq4nl_value(qs[j] & 0x0F);
                y[j + 16] = dl * (float)iq4nl_value(qs[j] >> 4);
            }
        }
    }
}

}  // namespace xs
