// xestrata-win_amd/csrc/experts_prefill.hip - grouped expert products for prompt and verify batches: a bf16 MFMA
// grouped GEMM whose expert weight tiles are dequantized from the raw GGUF blocks into LDS (the MI355X replacement
// of the reference's int8 iq_mmq_grouped, src/kernels/xe/iq_mmq.cpp:483-943, and of its FP16 fallbacks
// xmx_gemm_grouped / Gemm::f16_groups, src/prefill/gemm.cpp:371-388).
//
// Rows are the routed rows in expert order (the permutation of src/prefill/plain_prompt.cpp:576-637).  Two launches:
//   gate/up: h[row, j] = SwiGLU(x[src[row]] . gate_j, x[src[row]] . up_j) in bf16, a tile = 64 rows x 64 h columns
//            (its 64 gate and 64 up weight rows, so the SwiGLU is formed in registers);
//   down:    parts[entry[row], c] = h[row] . down_c in fp32, a tile = 64 rows x 128 output columns, written straight
//            into routing order for the combine.
// A work-group's m-tile comes from a flat tile index over every group's ceil(rows / 64) tiles (a prefix computed on
// the device), so Zipf-skewed groups cost their own tiles only.  4 waves a tile, each 32 rows x 64 weight rows as
// 2 x 4 v_mfma_f32_16x16x32_bf16 blocks; K steps of 64 values with both operands staged in LDS.
#include "xs_device.h"
#include "xs_dequant.h"
#include "xs_kernels.h"

namespace xs {

typedef short bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 64, kBN = 128, kBK = 64, kPad = 8, kLd = kBK + kPad;

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

template <bool DOWN>
__global__ __launch_bounds__(256) void grouped_mfma_kernel(ExpertLayout L, PrefillArgs a, const int32_t* __restrict__ mtile) {
    __shared__ __align__(16) uint16_t sA[kBM * kLd];
    __shared__ __align__(16) uint16_t sB[kBN * kLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ng = *a.n_groups;
    if (ng <= 0) return;
    const int mt = blockIdx.x;
    if (mt >= mtile[ng]) return;
    int lo = 0, hi = ng - 1;   // the group whose tiles hold mt
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (mtile[mid] <= mt) lo = mid;
        else hi = mid - 1;
    }
    const int g = lo;
    const int r0 = a.bounds[g] + (mt - mtile[g]) * kBM;
    const int nrows = min(kBM, a.bounds[g + 1] - r0);
    const uint8_t* blob = (const uint8_t*)a.wptr[g];
    const int H = (int)L.n_embd, F = (int)L.n_ff;
    const int K = DOWN ? F : H;
    const int wtype = DOWN ? L.d_type : L.gu_type;
    const int64_t wrb = DOWN ? L.d_row : L.gu_row;
    const int qk = block_values(wtype), bs = block_bytes(wtype);
    const int n0 = blockIdx.y * (DOWN ? kBN : kBN / 2);

    // this thread's A row (4 threads a row, 16 values each) and B row (2 threads a row, 32 values each)
    const int ar = tid >> 2, ac = (tid & 3) * 16;
    const uint16_t* arow = nullptr;
    if (ar < nrows) arow = DOWN ? a.h + (int64_t)(r0 + ar) * F : a.xb + (int64_t)a.src[r0 + ar] * H;
    const int br = tid >> 1, bh = tid & 1;
    int wrow;
    if (DOWN) wrow = n0 + br;
    else wrow = br < kBN / 2 ? n0 + br : F + n0 + (br - kBN / 2);
    const uint8_t* brow = blob + (DOWN ? L.down_off : 0) + (int64_t)wrow * wrb;

    // the wave's blocks: rows 32 (wave / 2) + 16 i, weight rows cb[j]
    const int rw = 32 * (wave >> 1);
    int cb[4];
    if (DOWN) {
        for (int j = 0; j < 4; ++j) cb[j] = 64 * (wave & 1) + 16 * j;
    } else {
        const int c0 = 32 * (wave & 1);
        cb[0] = c0; cb[1] = c0 + 16; cb[2] = 64 + c0; cb[3] = 64 + c0 + 16;
    }
    f32x4_t acc[2][4];
    for (int i = 0; i < 2; ++i)
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    for (int k0 = 0; k0 < K; k0 += kBK) {
        uint4 av0 = make_uint4(0, 0, 0, 0), av1 = make_uint4(0, 0, 0, 0);
        if (arow) {
            av0 = *(const uint4*)(arow + k0 + ac);
            av1 = *(const uint4*)(arow + k0 + ac + 8);
        }
        float v[32];
        const int kv = k0 + 32 * bh;
        dequant32(wtype, brow + (int64_t)(kv / qk) * bs, (kv % qk) / 32, v);
        uint32_t pk[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) pk[q] = (uint32_t)f2bf(v[2 * q]) | ((uint32_t)f2bf(v[2 * q + 1]) << 16);
        __syncthreads();   // the previous step's readers are done
        *(uint4*)(sA + ar * kLd + ac) = av0;
        *(uint4*)(sA + ar * kLd + ac + 8) = av1;
        uint4* bd = (uint4*)(sB + br * kLd + 32 * bh);
        bd[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        bd[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        bd[2] = make_uint4(pk[8], pk[9], pk[10], pk[11]);
        bd[3] = make_uint4(pk[12], pk[13], pk[14], pk[15]);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 32) {
            const int ko = kk + 8 * (lane >> 4);
            bf16x8_t fa[2], fb[4];
#pragma unroll
            for (int i = 0; i < 2; ++i) fa[i] = *(const bf16x8_t*)(sA + (rw + 16 * i + (lane & 15)) * kLd + ko);
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[j] = *(const bf16x8_t*)(sB + (cb[j] + (lane & 15)) * kLd + ko);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
    }
    // lane holds C[rw + 16 i + 4 (lane / 16) + r][cb[j] + lane % 16]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = rw + 16 * i + 4 * (lane >> 4) + r;
            if (row >= nrows) continue;
            if (DOWN) {
                float* dst = a.parts + (int64_t)a.entry[r0 + row] * H + n0;
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[cb[j] + (lane & 15)] = acc[i][j][r];
            } else {
                uint16_t* dst = a.h + (int64_t)(r0 + row) * F + n0;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float gv = acc[i][j][r], uv = acc[i][j + 2][r];
                    const float hv = gv / (1.0f + expf(-gv)) * uv;
                    dst[cb[j] + (lane & 15)] = f2bf(hv);
                }
            }
        }
}

hipError_t launch_prefill_experts(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s) {
    const int64_t nx = a.n_tok * L.n_embd;
    hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, s, a.x, a.xb, nx);
    hipLaunchKernelGGL(tile_map_kernel, dim3(1), dim3(1024), 0, s, a.bounds, a.n_groups, a.mtile, (int)a.cap_groups);
    const unsigned mt_bound = (unsigned)((a.rows + kBM - 1) / kBM + a.cap_groups);
    hipLaunchKernelGGL(grouped_mfma_kernel<false>, dim3(mt_bound, (unsigned)(L.n_ff / (kBN / 2))), dim3(256), 0, s, L, a,
                       (const int32_t*)a.mtile);
    hipLaunchKernelGGL(grouped_mfma_kernel<true>, dim3(mt_bound, (unsigned)(L.n_embd / kBN)), dim3(256), 0, s, L, a,
                       (const int32_t*)a.mtile);
    return hipGetLastError();
}

}  // namespace xs
