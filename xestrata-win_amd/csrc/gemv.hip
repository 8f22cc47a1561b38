// xestrata-win_amd/csrc/gemv.hip - the router's projections (logits = W x, W n_out rows of n_in) in the summation
// orders of the reference's kernels, so that logits, and the ids routed from them, come out bit for bit:
//
//   mmvf (f32_gemv_fp32_mmvf(_multi), bf16_gemv_fp32_mmvf(_multi); src/kernels/xe/bf16_gemv.cpp:91-147, 213-225,
//     464-517): a work-group of B threads a row, B the candidate of 32, 64, ..., 256 with the fewest pair iterations
//     (the smallest on a tie).  Thread t walks pairs t, t + B, ... with two ordered FMAs a pair (weight 2p, then
//     2p + 1) into one accumulator a token; a xor butterfly (16, 8, 4, 2, 1) over each 32 threads; for B > 32 the
//     partials of the B / 32 groups (then zeros up to 32) summed by the same butterfly.  Up to 8 tokens a launch.
//   gemm_rows (f32_gemm_rows, bf16_gemv.cpp:475-502; the prompt path's router and shared gate): one FMA chain a
//     logit, k = 0, 1, ... n_in - 1, then FMAs with zeros up to the next multiple of 16.
//   warp (bf16_gemv for n_out >= 64 and bf16_gemv_split at 32 threads a row, bf16_gemv.cpp:62-77, 300-317): bf16
//     activations and weights, 32 lanes a row, lane l over l, l + 32, ..., then the 32-lane butterfly; every product
//     of two bf16 values is exact in f32, so a fused and an unfused multiply-add agree.
//   naive (bf16_gemv for n_out < 64, bf16_gemv.cpp:50-60): one chain a row over the whole row.
//   tree (bf16_gemv_split at another power of two, bf16_gemv.cpp:318-339): lane chains as warp's, then the shared
//     memory tree s[t] += s[t + off], off = tpr / 2 ... 1.
//
// MI355X layout: a 32-lane group is half a wave64 (a xor below 32 stays inside it), so the warp form takes two rows a
// wave and the mmvf form's 32-thread groups are wave halves.  The gemm_rows form tiles 64 tokens x 64 rows a
// work-group, K through LDS 32 at a time stored K-major so a thread's 4 tokens and 4 rows are one 16-byte LDS read
// each; its 16 chains stay in registers.
#include "xs_device.h"
#include "xs_kernels.h"

namespace xs {

__device__ __forceinline__ float bf2f(uint16_t b) { return u2f((uint32_t)b << 16); }

__device__ __forceinline__ float sum32(float v) {   // the 32-lane xor butterfly, inside each wave half
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 1, 64);
    return v;
}

int mmvf_block(int64_t n_in) {
    int best = 32;
    int64_t best_it = (n_in + 63) / 64;
    for (int c = 64; c <= 256; c += 32) {
        const int64_t it = (n_in + 2 * c - 1) / (2 * c);
        if (it < best_it) {
            best_it = it;
            best = c;
        }
    }
    return best;
}

template <typename W>
__device__ __forceinline__ void weight_pair(const W* row, int64_t p, float& w0, float& w1);
template <>
__device__ __forceinline__ void weight_pair<float>(const float* row, int64_t p, float& w0, float& w1) {
    const float2 v = *(const float2*)(row + 2 * p);
    w0 = v.x;
    w1 = v.y;
}
template <>
__device__ __forceinline__ void weight_pair<uint16_t>(const uint16_t* row, int64_t p, float& w0, float& w1) {
    const uint32_t v = *(const uint32_t*)(row + 2 * p);
    w0 = u2f(v << 16);
    w1 = u2f(v & 0xFFFF0000u);
}

template <typename W>
__global__ __launch_bounds__(256) void mmvf_kernel(const float* __restrict__ x, int64_t ldx, const W* __restrict__ w,
                                                   float* __restrict__ y, int64_t ldy, int64_t n_pairs, int n_tok) {
    __shared__ float partials[8 * 32];
    const int t = threadIdx.x, B = blockDim.x;
    const int64_t o = blockIdx.x;
    const W* row = w + o * 2 * n_pairs;
    if (B > 32) {
        if (t < 32)
            for (int k = 0; k < 8; ++k) partials[k * 32 + t] = 0.0f;
        __syncthreads();
    }
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = 0.0f;
    for (int64_t p = t; p < n_pairs; p += B) {
        float w0, w1;
        weight_pair<W>(row, p, w0, w1);
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k < n_tok) {
                const float2 xv = *(const float2*)(x + k * ldx + 2 * p);
                acc[k] = __builtin_fmaf(w0, xv.x, acc[k]);
                acc[k] = __builtin_fmaf(w1, xv.y, acc[k]);
            }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = sum32(acc[k]);
    if (B > 32) {
        if ((t & 31) == 0)
            for (int k = 0; k < n_tok; ++k) partials[k * 32 + t / 32] = acc[k];
        __syncthreads();
        if (t < 64) {   // lanes 32..63 run the same sums on the same values; only lane 0 stores
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] = sum32(partials[k * 32 + (t & 31)]);
        }
    }
    if (t == 0)
        for (int k = 0; k < n_tok; ++k) y[k * ldy + o] = acc[k];
}

template <typename W>
hipError_t launch_mmvf(const float* x, int64_t ldx, const W* w, float* y, int64_t ldy, int64_t n_in, int64_t n_out,
                       int n_tok, hipStream_t s) {
    hipLaunchKernelGGL(mmvf_kernel<W>, dim3((unsigned)n_out), dim3(mmvf_block(n_in)), 0, s, x, ldx, w, y, ldy,
                       n_in / 2, n_tok);
    return hipGetLastError();
}
template hipError_t launch_mmvf<float>(const float*, int64_t, const float*, float*, int64_t, int64_t, int64_t, int,
                                       hipStream_t);
template hipError_t launch_mmvf<uint16_t>(const float*, int64_t, const uint16_t*, float*, int64_t, int64_t, int64_t,
                                          int, hipStream_t);

// 64 tokens x 64 rows a work-group; thread (ti, tj) = (tid / 16, tid % 16) owns tokens 4 ti .. and rows 4 tj ..
constexpr int kGT = 64, kGK = 32;
__global__ __launch_bounds__(256) void gemm_rows_kernel(const float* __restrict__ x, int64_t ldx,
                                                        const float* __restrict__ w, float* __restrict__ y,
                                                        int64_t ldy, int64_t n_in, int64_t n_out, int64_t n_tok) {
    __shared__ float4 xs[kGK][kGT / 4];
    __shared__ float4 ws[kGK][kGT / 4];
    const int tid = threadIdx.x, ti = tid >> 4, tj = tid & 15;
    const int64_t t0 = (int64_t)blockIdx.y * kGT, o0 = (int64_t)blockIdx.x * kGT;
    const int64_t k_end = (n_in + 15) / 16 * 16;   // the reference's chain: zeros up to a multiple of 16
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    // loader: thread tid reads 8 consecutive k of token / row (tid / 4) at k offset 8 (tid % 4)
    const int lr = tid >> 2, lk = (tid & 3) * 8;
    for (int64_t k0 = 0; k0 < k_end; k0 += kGK) {
        float xv[8], wv[8];
        const int64_t tr = t0 + lr, wr = o0 + lr;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t k = k0 + lk + u;
            xv[u] = tr < n_tok && k < n_in ? x[tr * ldx + k] : 0.0f;
            wv[u] = wr < n_out && k < n_in ? w[wr * n_in + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            ((float*)&xs[lk + u][0])[lr] = xv[u];
            ((float*)&ws[lk + u][0])[lr] = wv[u];
        }
        __syncthreads();
        const int kn = (int)min((int64_t)kGK, k_end - k0);
        for (int kk = 0; kk < kn; ++kk) {
            const float4 a = xs[kk][ti], b = ws[kk][tj];
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t t = t0 + 4 * ti + i;
        if (t >= n_tok) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t o = o0 + 4 * tj + j;
            if (o < n_out) y[t * ldy + o] = acc[i][j];
        }
    }
}

hipError_t launch_gemm_rows(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in,
                            int64_t n_out, int64_t n_tok, hipStream_t s) {
    const dim3 grid((unsigned)((n_out + kGT - 1) / kGT), (unsigned)((n_tok + kGT - 1) / kGT));
    hipLaunchKernelGGL(gemm_rows_kernel, grid, dim3(256), 0, s, x, ldx, w, y, ldy, n_in, n_out, n_tok);
    return hipGetLastError();
}

// x bf16 (or f32 rounded to bf16 on the fly: the same bits as converting first) against bf16 rows, 32 lanes a row
template <bool XF32>
__global__ __launch_bounds__(256) void bf16_warp_kernel(const void* __restrict__ xv, const uint16_t* __restrict__ w,
                                                        float* __restrict__ y, int64_t n_in, int64_t n_out) {
    const int lane = threadIdx.x & 31;
    const int64_t o = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const bool live = o < n_out;
    const uint16_t* row = w + (live ? o : 0) * n_in;
    float acc = 0.0f;
    if (live)
        for (int64_t i = lane; i < n_in; i += 32) {
            const float xf = XF32 ? bf2f(f2bf(((const float*)xv)[i])) : bf2f(((const uint16_t*)xv)[i]);
            acc = __builtin_fmaf(xf, bf2f(row[i]), acc);
        }
    acc = sum32(acc);
    if (live && lane == 0) y[o] = acc;
}

__global__ __launch_bounds__(256) void bf16_naive_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w, float* __restrict__ y,
                                                         int64_t n_in, int64_t n_out) {
    const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= n_out) return;
    const uint16_t* row = w + o * n_in;
    float acc = 0.0f;
    for (int64_t i = 0; i < n_in; ++i) acc = __builtin_fmaf(bf2f(x[i]), bf2f(row[i]), acc);
    y[o] = acc;
}

__global__ __launch_bounds__(1024) void bf16_tree_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w, float* __restrict__ y,
                                                         int64_t n_in) {
    extern __shared__ float tree[];
    const int t = threadIdx.x, tpr = blockDim.x;
    const int64_t o = blockIdx.x;
    const uint16_t* row = w + o * n_in;
    float acc = 0.0f;
    for (int64_t i = t; i < n_in; i += tpr) acc = __builtin_fmaf(bf2f(x[i]), bf2f(row[i]), acc);
    tree[t] = acc;
    __syncthreads();
    for (int off = tpr >> 1; off > 0; off >>= 1) {
        if (t < off) tree[t] = tree[t] + tree[t + off];
        __syncthreads();
    }
    if (t == 0) y[o] = tree[0];
}

__global__ __launch_bounds__(256) void to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                      int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = f2bf(x[i]);
}

hipError_t launch_to_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_bf16_gemv(const void* x, bool x_f32, const uint16_t* w, float* y, int64_t n_in, int64_t n_out,
                            int form, int tpr, hipStream_t s) {
    if (form == kBf16Warp) {
        const dim3 grid((unsigned)((n_out + 7) / 8));
        if (x_f32)
            hipLaunchKernelGGL(bf16_warp_kernel<true>, grid, dim3(256), 0, s, x, w, y, n_in, n_out);
        else
            hipLaunchKernelGGL(bf16_warp_kernel<false>, grid, dim3(256), 0, s, x, w, y, n_in, n_out);
    } else if (form == kBf16Naive) {
        hipLaunchKernelGGL(bf16_naive_kernel, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s,
                           (const uint16_t*)x, w, y, n_in, n_out);
    } else {
        hipLaunchKernelGGL(bf16_tree_kernel, dim3((unsigned)n_out), dim3(tpr), (size_t)tpr * 4, s,
                           (const uint16_t*)x, w, y, n_in);
    }
    return hipGetLastError();
}

}  // namespace xs
