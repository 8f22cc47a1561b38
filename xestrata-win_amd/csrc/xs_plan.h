// xestrata-win_amd/csrc/xs_plan.h - where the decode plan's arrays sit in its int32 words, for the host (abi.cpp) and
// the device writers (dispatch.hip, decode_layer.hip).
//
// The words are the engine's GpuPlanSink (reference include/strata/core/expert_source.hpp:219-243) in the packing its
// device writer lays them out in (src/kernels/xe/verify_kernels.cpp:860-866), since the engine reads them there:
//   counts[4] | start[cap + 1] | dst[cap] | tok[cap] | (one word to 8-byte alignment) | ptr u64[cap] | ptr2 u64[cap]
//   | start2[cap + 1] | one spare word
// counts[0] = the HBM groups, counts[1] = the entries, counts[2] = the PCIe groups (ptr2 / start2).
#pragma once

#include <stdint.h>

namespace xs {

struct PlanWords {
    long long cap;   // entries the plan has room for
    __host__ __device__ constexpr long long counts() const { return 0; }
    __host__ __device__ constexpr long long start() const { return 4; }
    __host__ __device__ constexpr long long dst() const { return start() + cap + 1; }
    __host__ __device__ constexpr long long tok() const { return dst() + cap; }
    __host__ __device__ constexpr long long ptr() const { return (tok() + cap + 1) & ~1ll; }   // u64: even word
    __host__ __device__ constexpr long long ptr2() const { return ptr() + 2 * cap; }
    __host__ __device__ constexpr long long start2() const { return ptr2() + 2 * cap; }
    __host__ __device__ constexpr long long words() const { return start2() + cap + 2; }
};

}  // namespace xs
