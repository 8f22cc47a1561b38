// xestrata-win_amd/csrc/xs_f16.h - the prompt path's f16 copy of the activations: the K order of a GEMM step, the
// saturating conversion and its status bit.  Shared by the GEMMs (experts_prefill.hip) and the permutation kernel
// (dispatch.hip), which builds the copy in its idle work-groups.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xs {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// slot order inside an octet and octet order inside a step (an involution)
__host__ __device__ constexpr int perm8(int i) { return (i == 1 || i == 5) ? i + 1 : (i == 2 || i == 6) ? i - 1 : i; }
__host__ __device__ constexpr int perm64(int p) { return 8 * perm8(p >> 3) + perm8(p & 7); }

__device__ __forceinline__ uint32_t sat_f16x2(float a, float b) {   // RNE, saturated to the f16 range (NaN kept)
    a = __builtin_fminf(__builtin_fmaxf(a, -65504.0f), 65504.0f);
    b = __builtin_fminf(__builtin_fmaxf(b, -65504.0f), 65504.0f);
    return __builtin_bit_cast(uint32_t, (h2_t){(_Float16)a, (_Float16)b});
}

// a value past the f16 range, saturated: status bit 8 (kSatBit) of the call's status word, when it has one
constexpr int kSatBit = 8;
__device__ __forceinline__ bool past_f16(float v) { return __builtin_fabsf(v) > 65504.0f; }   // (NaN: false)

// chunk i (8 values) of x [n, H] fp32 -> f16 in the step order
__device__ __forceinline__ void to_f16_chunk(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t i,
                                             int32_t* __restrict__ err) {
    const int c = (int)(i & 7);
    const float* s = x + (i & ~(int64_t)7) * 8 + 8 * perm8(c);
    const float4 v0 = *(const float4*)s, v1 = *(const float4*)(s + 4);
    if (err && (past_f16(v0.x) || past_f16(v0.y) || past_f16(v0.z) || past_f16(v0.w) || past_f16(v1.x) ||
                past_f16(v1.y) || past_f16(v1.z) || past_f16(v1.w)))
        atomicOr(err, kSatBit);
    *(uint4*)(y + 8 * i) = make_uint4(sat_f16x2(v0.x, v0.z), sat_f16x2(v0.y, v0.w), sat_f16x2(v1.x, v1.z),
                                      sat_f16x2(v1.y, v1.w));
}

}  // namespace xs
