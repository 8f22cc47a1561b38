// xestrata-win_amd/csrc/xs_device.h - device-side building blocks shared by the MoE kernels (gfx950, wave64).
//
// GGUF block layouts (ggml-common.h, the reference's third_party/main/ggml/ggml-common.h):
//   Q8_0 34 B/32, Q8_1 36 B/32, Q4_K 144 B/256, Q6_K 210 B/256, IQ4_XS 136 B/256.
// Every source file is compiled with -ffp-contract=off: products and sums round on their own unless a fused
// multiply-add is written out (__builtin_fmaf), which is what the reference's canonical arithmetic requires
// (include/strata/kernels/canon_math.hpp, CMakeLists.txt:396).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xs {

enum : int { kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kIQ4_XS = 23 };
constexpr int kWave = 64;

__host__ __device__ constexpr int block_values(int t) { return t == kQ8_0 ? 32 : 256; }
__host__ __device__ constexpr int block_bytes(int t) {
    return t == kQ8_0 ? 34 : t == kQ4_K ? 144 : t == kQ6_K ? 210 : t == kIQ4_XS ? 136 : 0;
}
__host__ __device__ constexpr int64_t row_bytes(int t, int64_t n) { return n / block_values(t) * block_bytes(t); }

// ---------------------------------------------------------------- scalar conversions

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// fp16 bits -> float (exact; the hardware conversion keeps subnormals)
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// float -> fp16 bits, round to nearest even
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
// float -> bf16 bits, round to nearest even (NaN kept quiet)
__device__ __forceinline__ uint16_t f2bf(float f) {
    const uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// ---------------------------------------------------------------- canonical arithmetic
// canon_math.hpp's SwiGLU and int8 scale: the same IEEE operations in the same order on every device, so the GPU and
// the CPU give the same bits (reference include/strata/kernels/canon_math.hpp:55-108).

__device__ __forceinline__ float canon_rcp(float v) {
    float r = u2f(0x7EF311C3u - f2u(v));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const float e = __builtin_fmaf(-v, r, 1.0f);
        r = __builtin_fmaf(r, e, r);
    }
    return r;
}
__device__ __forceinline__ float canon_exp(float x) {
    x = x < -80.0f ? -80.0f : x > 80.0f ? 80.0f : x;
    const float t = x * 1.44269504f;
    const float kf = (t + 12582912.0f) - 12582912.0f;
    float r = __builtin_fmaf(-kf, 0.693145752f, x);
    r = __builtin_fmaf(-kf, 1.42860677e-06f, r);
    float p = 1.0f / 720.0f;
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return u2f(f2u(p) + (uint32_t)((int32_t)kf << 23));
}
__device__ __forceinline__ float canon_silu_mul(float g, float u) {
    const float den = 1.0f + canon_exp(-g);
    const float a = g * canon_rcp(den);
    return a * u;
}
__device__ __forceinline__ float q8_scale(float amax) {
    const float d = amax * (1.0f / 127.0f);
    return d > 65504.0f ? 65504.0f : d;
}
__device__ __forceinline__ float q8_inv(float d) { return d >= 1e-30f ? canon_rcp(d) : 0.0f; }
__device__ __forceinline__ int q8_value(float x, float id) {
    const float t = x * id;
    const float r = t + (t < 0.0f ? -0.5f : 0.5f);
    const float c = r > 127.0f ? 127.0f : r < -127.0f ? -127.0f : r;
    return (int)(int8_t)(int32_t)c;
}
__device__ __forceinline__ float q8_1_finite(float v) { return fabsf(v) > 65504.0f ? copysignf(65504.0f, v) : v; }

// ---------------------------------------------------------------- integer dot and wave reductions

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// sum over groups of `W` neighbouring lanes (W a power of two up to 64); every lane of a group ends with the sum
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int W>
__device__ __forceinline__ int group_sum_i(int v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ---------------------------------------------------------------- DPP lane moves
// A __shfl_xor is an LDS-unit round trip (ds_bpermute, ~100 cycles, serialised along a reduction); a DPP operand moves
// lanes inside the VALU.  quad_perm [1,0,3,2] / [2,3,0,1] are the xor-1 / xor-2 exchanges; row_shl:4 gives lane i of a
// 16-lane row the value of lane i + 4 (lanes 12..15 keep their own); row_ror:4 / :8 rotate a row.  The 16-lane rows
// are joined with v_readlane (uniform results) or one ds_swizzle (xor 16 inside 32 lanes).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppShl4 = 0x104, kDppRor4 = 0x124, kDppRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = dpp_i<CTRL>((int)b), hi = dpp_i<CTRL>((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ float swz_xor16_f(float v) {   // lane i ^ 16 within each 32 lanes
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, l), hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

constexpr int kDppBcast15 = 0x142, kDppBcast31 = 0x143;   // lane 15 of each row to the next row; lane 31 to rows 2, 3

template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
    const int lo = __builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROWS, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp((int)(v >> 32), (int)(v >> 32), CTRL, ROWS, 0xF, false);
    return ((unsigned long long)(unsigned int)hi << 32) | (unsigned int)lo;
}
// the largest 32-bit unsigned value of the wave, uniform: rows by xor and rotation, then rows 0+1 into row 1, 2+3 into
// row 3 and row 1 into row 3 (row_bcast), read from lane 63.  0 is the identity of the max, so each move fuses into one
// v_max_u32_dpp (lanes of rows a move leaves out keep their value); no exec-mask or scalar round trips on the way.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t max_dpp_u32(uint32_t v) {
    return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, true));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max_dpp_u32<kDppXor1, 0xF>(v);
    v = max_dpp_u32<kDppXor2, 0xF>(v);
    v = max_dpp_u32<kDppRor4, 0xF>(v);
    v = max_dpp_u32<kDppRor8, 0xF>(v);
    v = max_dpp_u32<kDppBcast15, 0xA>(v);
    v = max_dpp_u32<kDppBcast31, 0xC>(v);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// max over each 16-lane row (every lane ends with its row's), over 32 lanes, over the wave (uniform); every lane of
// the wave active
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppRor4>(v));
    return fmaxf(v, dpp_f<kDppRor8>(v));
}
__device__ __forceinline__ float group_max32(float v) {
    v = row_max16(v);
    return fmaxf(v, swz_xor16_f(v));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max16(v);
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
// a sum over the wave in an unspecified order (uniform result)
__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_d<kDppXor1>(v);
    v += dpp_d<kDppXor2>(v);
    v += dpp_d<kDppRor4>(v);
    v += dpp_d<kDppRor8>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
// The butterfly sum of a row dot over groups of L neighbouring lanes (L = 1, 2, 4, 8; o = L/2 .. 1): lane 0 of each
// group ends with group_sum<L>'s value bit for bit (same operands in the same order); other lanes' values are
// unspecified.
template <int L>
__device__ __forceinline__ float lane0_sum(float v) {
    if (L >= 8) v += dpp_f<kDppShl4>(v);
    if (L >= 4) v += dpp_f<kDppXor2>(v);
    if (L >= 2) v += dpp_f<kDppXor1>(v);
    return v;
}

// bytes of a 16-entry signed table picked by the 4 nibbles of `idx` bytes (each byte < 16): v_perm over the table's
// halves, then a select on bit 3 of each index
__device__ __forceinline__ int table16_lookup(uint32_t idx, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t m = ((idx & 0x08080808u) >> 3) * 0xFFu;   // 0xFF in every byte whose index is >= 8
    return (int)((hi & m) | (lo & ~m));
}

// ---------------------------------------------------------------- 2-byte aligned reads
// Q8_0 and Q6_K blocks are 34 / 210 bytes: inside a row they sit at even addresses only.  Words are assembled from
// 16-bit reads, never from an unaligned 32-bit one.
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) {
    const uint16_t* q = (const uint16_t*)p;
    return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}

// ---------------------------------------------------------------- LDS DMA with waits of the kernel's own
// wait until at most n of the wave's vector memory operations are outstanding (n wave-uniform; past 63, 63)
__device__ __forceinline__ void vm_wait_le(int n) {
    switch (n < 63 ? n : 63) {
#define XS_SW(i) \
    case i: asm volatile("s_waitcnt vmcnt(" #i ")" ::: "memory"); break;
        XS_SW(0) XS_SW(1) XS_SW(2) XS_SW(3) XS_SW(4) XS_SW(5) XS_SW(6) XS_SW(7) XS_SW(8) XS_SW(9) XS_SW(10) XS_SW(11)
        XS_SW(12) XS_SW(13) XS_SW(14) XS_SW(15) XS_SW(16) XS_SW(17) XS_SW(18) XS_SW(19) XS_SW(20) XS_SW(21) XS_SW(22)
        XS_SW(23) XS_SW(24) XS_SW(25) XS_SW(26) XS_SW(27) XS_SW(28) XS_SW(29) XS_SW(30) XS_SW(31) XS_SW(32) XS_SW(33)
        XS_SW(34) XS_SW(35) XS_SW(36) XS_SW(37) XS_SW(38) XS_SW(39) XS_SW(40) XS_SW(41) XS_SW(42) XS_SW(43) XS_SW(44)
        XS_SW(45) XS_SW(46) XS_SW(47) XS_SW(48) XS_SW(49) XS_SW(50) XS_SW(51) XS_SW(52) XS_SW(53) XS_SW(54) XS_SW(55)
        XS_SW(56) XS_SW(57) XS_SW(58) XS_SW(59) XS_SW(60) XS_SW(61) XS_SW(62) XS_SW(63)
#undef XS_SW
        default: break;
    }
}

// One LDS DMA (global_load_lds_dwordx4: 16 bytes a lane to lds_off + 16 lane) issued from inline assembly: the
// compiler does not count it, so it places no conservative vmcnt(0) before the slots' LDS reads (it would for the
// builtin, whose LDS write may alias them); the kernel's own waits order the slots.  Waits the compiler places for
// other loads can only grow by the uncounted DMAs (returns are in order), never shrink.
__device__ __forceinline__ void dma16_nt(const void* src, uint32_t lds_off) {
    // an SALU write of M0 needs one wait state before an LDS DMA reads it (the compiler adds it for its own code, not
    // inside inline assembly)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(lds_off)
                 : "memory", "m0");
}
// the same without the nontemporal hint (data other work-groups read again soon)
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_off) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_off)
                 : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

}  // namespace xs
