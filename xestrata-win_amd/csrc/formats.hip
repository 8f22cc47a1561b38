// xestrata-win_amd/csrc/formats.hip - the GGUF expert formats on the device: this library's quantizer (float rows ->
// Q8_0 / Q4_K / Q6_K / IQ4_XS blocks) and the dequantizer whose values must equal the reference's host dequantizers
// bit for bit (reference include/strata/artifact/dequant.hpp:84-89, 152-175, 181-209, 283-299).
//
// The quantizer is this library's own (the reference ships none for these types: its tests call ggml's
// ggml_quantize_chunk).  It only has to produce valid blocks close to the input: every consumer reads a block
// through the dequantizer's meaning, which is the pinned contract.
#include "xs_device.h"
#include "xs_kernels.h"
#include "xs_dequant.h"

namespace xs {


__device__ __forceinline__ float round_half_away(float v) { return v < 0.0f ? -floorf(-v + 0.5f) : floorf(v + 0.5f); }

// ---------------------------------------------------------------- quantizer: one thread per block

__device__ void quant_q8_0(const float* x, uint8_t* b) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    const float d = amax / 127.0f, id = amax > 0.0f ? 127.0f / amax : 0.0f;
    const uint16_t hd = f2h(d);
    b[0] = (uint8_t)hd;
    b[1] = (uint8_t)(hd >> 8);
    for (int i = 0; i < 32; ++i) {
        float q = round_half_away(x[i] * id);
        q = q > 127.0f ? 127.0f : q < -127.0f ? -127.0f : q;
        b[2 + i] = (uint8_t)(int8_t)(int)q;
    }
}

// Q4_K: value = (d * sc) * q - dmin * m with q in 0..15, sc and m 6-bit.  Per 32-value sub-block the range
// [min(0, lo), hi] is split in 15 steps; the 8 steps and 8 offsets are then quantized against d and dmin.
__device__ void quant_q4_K(const float* x, uint8_t* b) {
    float scale[8], off[8], smax = 0.0f, omax = 0.0f;
    for (int s = 0; s < 8; ++s) {
        float lo = 0.0f, hi = 0.0f;
        for (int i = 0; i < 32; ++i) { lo = fminf(lo, x[32 * s + i]); hi = fmaxf(hi, x[32 * s + i]); }
        scale[s] = (hi - lo) / 15.0f;
        off[s] = -lo;
        smax = fmaxf(smax, scale[s]);
        omax = fmaxf(omax, off[s]);
    }
    const float d = smax / 63.0f, dmin = omax / 63.0f;
    const uint16_t hd = f2h(d), hm = f2h(dmin);
    const float dq = h2f(hd), dmq = h2f(hm);
    int sc[8], m[8];
    for (int s = 0; s < 8; ++s) {
        const float a = dq > 0.0f ? round_half_away(scale[s] / dq) : 0.0f;
        const float c = dmq > 0.0f ? round_half_away(off[s] / dmq) : 0.0f;
        sc[s] = (int)fminf(fmaxf(a, 0.0f), 63.0f);
        m[s] = (int)fminf(fmaxf(c, 0.0f), 63.0f);
    }
    b[0] = (uint8_t)hd; b[1] = (uint8_t)(hd >> 8);
    b[2] = (uint8_t)hm; b[3] = (uint8_t)(hm >> 8);
    uint8_t* q = b + 4;
    for (int j = 0; j < 4; ++j) {
        q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    uint8_t* qs = b + 16;
    for (int p = 0; p < 4; ++p) {
        int qq[2][32];
        for (int h = 0; h < 2; ++h) {
            const int s = 2 * p + h;
            const float ds = dq * (float)sc[s], dm = dmq * (float)m[s];
            for (int i = 0; i < 32; ++i) {
                float v = ds > 0.0f ? round_half_away((x[32 * s + i] + dm) / ds) : 0.0f;
                qq[h][i] = (int)fminf(fmaxf(v, 0.0f), 15.0f);
            }
        }
        for (int i = 0; i < 32; ++i) qs[32 * p + i] = (uint8_t)(qq[0][i] | (qq[1][i] << 4));
    }
}

// Q6_K: value = (d * sc) * (q - 32), sc int8 per 16 values, q 6-bit
__device__ void quant_q6_K(const float* x, uint8_t* b) {
    float scale[16], smax = 0.0f;
    for (int s = 0; s < 16; ++s) {
        float a = 0.0f;
        for (int i = 0; i < 16; ++i) a = fmaxf(a, fabsf(x[16 * s + i]));
        scale[s] = a / 31.0f;
        smax = fmaxf(smax, scale[s]);
    }
    const float d = smax / 127.0f;
    const uint16_t hd = f2h(d);
    const float dq = h2f(hd);
    int8_t* scales = (int8_t*)(b + 192);
    int q[256];
    for (int s = 0; s < 16; ++s) {
        const float a = dq > 0.0f ? round_half_away(scale[s] / dq) : 0.0f;
        const int sc = (int)fminf(fmaxf(a, 0.0f), 127.0f);
        scales[s] = (int8_t)sc;
        const float ds = dq * (float)sc;
        for (int i = 0; i < 16; ++i) {
            float v = ds > 0.0f ? round_half_away(x[16 * s + i] / ds) : 0.0f;
            v = fminf(fmaxf(v, -32.0f), 31.0f);
            q[16 * s + i] = (int)v + 32;
        }
    }
    uint8_t* ql = b;
    uint8_t* qh = b + 128;
    for (int n = 0; n < 2; ++n)
        for (int l = 0; l < 32; ++l) {
            const int q1 = q[128 * n + l], q2 = q[128 * n + l + 32], q3 = q[128 * n + l + 64], q4 = q[128 * n + l + 96];
            ql[64 * n + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
            ql[64 * n + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
            qh[32 * n + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    b[208] = (uint8_t)hd;
    b[209] = (uint8_t)(hd >> 8);
}

// IQ4_XS: value = (d * (ls - 32)) * kvalues[q], ls 6-bit per 32 values, q an index into the IQ4_NL codebook
__device__ void quant_iq4_xs(const float* x, uint8_t* b) {
    float scale[8], smax = 0.0f;
    for (int s = 0; s < 8; ++s) {
        float a = 0.0f;
        for (int i = 0; i < 32; ++i) a = fmaxf(a, fabsf(x[32 * s + i]));
        scale[s] = a / 127.0f;
        smax = fmaxf(smax, scale[s]);
    }
    const float d = smax / 31.0f;
    const uint16_t hd = f2h(d);
    const float dq = h2f(hd);
    b[0] = (uint8_t)hd;
    b[1] = (uint8_t)(hd >> 8);
    uint32_t scales_h = 0;
    uint8_t* scales_l = b + 4;
    scales_l[0] = scales_l[1] = scales_l[2] = scales_l[3] = 0;
    uint8_t* qs = b + 8;
    for (int s = 0; s < 8; ++s) {
        const float a = dq > 0.0f ? round_half_away(scale[s] / dq) : 0.0f;
        const int ls = (int)fminf(fmaxf(a, 0.0f), 31.0f) + 32;
        scales_l[s / 2] |= (uint8_t)((ls & 15) << (4 * (s % 2)));
        scales_h |= (uint32_t)(ls >> 4) << (2 * s);
        const float dl = dq * (float)(ls - 32);
        int idx[32];
        for (int i = 0; i < 32; ++i) {
            const float t = dl > 0.0f ? x[32 * s + i] / dl : 0.0f;
            int best = 0;
            float be = fabsf(t - (float)iq4nl_value(0));
            for (int c = 1; c < 16; ++c) {
                const float e = fabsf(t - (float)iq4nl_value(c));
                if (e < be) { be = e; best = c; }
            }
            idx[i] = best;
        }
        for (int j = 0; j < 16; ++j) qs[16 * s + j] = (uint8_t)(idx[j] | (idx[j + 16] << 4));
    }
    b[2] = (uint8_t)scales_h;
    b[3] = (uint8_t)(scales_h >> 8);
}

__global__ void quantize_rows_kernel(int type, const float* __restrict__ x, int64_t n_blocks, uint8_t* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    const int qk = block_values(type), bs = block_bytes(type);
    const float* xb = x + i * qk;
    uint8_t* yb = y + i * bs;
    switch (type) {
        case kQ8_0: quant_q8_0(xb, yb); break;
        case kQ4_K: quant_q4_K(xb, yb); break;
        case kQ6_K: quant_q6_K(xb, yb); break;
        default: quant_iq4_xs(xb, yb); break;
    }
}

// ---------------------------------------------------------------- dequantizer: one thread per 32 values

template <typename Out>
__device__ __forceinline__ void put(Out* y, int i, float v);
template <>
__device__ __forceinline__ void put<float>(float* y, int i, float v) { y[i] = v; }
template <>
__device__ __forceinline__ void put<uint16_t>(uint16_t* y, int i, float v) { y[i] = f2bf(v); }
struct f16_out {   // an f16 output (the bits of a half), told apart from the bf16 one by type
    uint16_t bits;
};
template <>
__device__ __forceinline__ void put<f16_out>(f16_out* y, int i, float v) { y[i].bits = f2h(v); }

template <typename Out>
__global__ void dequant_kernel(int type, const uint8_t* __restrict__ src, int64_t n32, Out* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n32) return;
    const int per = block_values(type) / 32;
    const int64_t blk = i / per;
    float v[32];
    dequant32(type, src + blk * block_bytes(type), (int)(i % per), v);
    Out* y = dst + 32 * i;
#pragma unroll
    for (int j = 0; j < 32; ++j) put(y, j, v[j]);
}

hipError_t launch_quantize_rows(int type, const float* x, int64_t n, void* y, hipStream_t s) {
    const int64_t nb = n / block_values(type);
    if (nb <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)((nb + 63) / 64)), dim3(64), 0, s, type, x, nb, (uint8_t*)y);
    return hipGetLastError();
}

hipError_t launch_dequant(int type, const void* src, int64_t n, void* dst, int out, hipStream_t s) {
    const int64_t n32 = n / 32;
    if (n32 <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n32 + 255) / 256));
    if (out == kDequantBf16)
        hipLaunchKernelGGL(dequant_kernel<uint16_t>, grid, dim3(256), 0, s, type, (const uint8_t*)src, n32, (uint16_t*)dst);
    else if (out == kDequantF16)
        hipLaunchKernelGGL(dequant_kernel<f16_out>, grid, dim3(256), 0, s, type, (const uint8_t*)src, n32, (f16_out*)dst);
    else
        hipLaunchKernelGGL(dequant_kernel<float>, grid, dim3(256), 0, s, type, (const uint8_t*)src, n32, (float*)dst);
    return hipGetLastError();
}

}  // namespace xs
