// xestrata-win_amd/csrc/noalloc.hip - the decode MoE layer for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): xs_moe_layer_decode with the library's own
// scratch, a fixed array in device memory, in place of the caller's workspace.
//
// The array is a file-scope __device__ variable: every GPU the library runs on holds its own copy, at its own address,
// from the module's load until the process ends, zero-filled by the loader (it has no initializer).  Host code never
// passes the array's name to a kernel (on the host that name is only a stand-in): the first call on a device, with the
// device current, looks its address up with hipGetSymbolAddress and keeps it per device.
//
// The decode workspace needs no clearing between calls: its call counters advance by one epoch a call and every
// hand-over word carries the epoch it was written in, so words of earlier calls never match (the scratch only has to
// start at zero, which the loader does).  The tagged words sit in regions sized for the largest layout
// (xs::kScratchMaxEmbd, kScratchMaxFF) ahead of everything else, so calls of any layout and token count can share the
// one array.  Calls that overlap on one GPU (two streams, two threads) race on it: a caller runs them one at a time.
#include "../../include/xs_moe.h"
#include "xs_error.h"
#include "xs_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>
#include <string>

namespace xs {
size_t layer_decode_fixed_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok);
int layer_decode_fixed(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                       const float* x, const float* logits, const float* residual, float* out, int n_tok,
                       void* scratch, size_t scratch_bytes, int32_t* status, void* stream);
}  // namespace xs

namespace {

constexpr size_t kScratchBytes = XS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_addr[kMaxDevices] = {};   // scratch's device address on each device, once looked up

// this device's address of `scratch` (looked up once per device, with the device current)
int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return xs::set_error(XS_EDEVICE, std::string("moe_layer_decode_noalloc: hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return xs::set_error(XS_EDEVICE, "moe_layer_decode_noalloc: device " + std::to_string(dev) + " past " +
                                             std::to_string(kMaxDevices));
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_addr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return xs::set_error(XS_EDEVICE, std::string("moe_layer_decode_noalloc: hipGetSymbolAddress(scratch): ") +
                                                 hipGetErrorString(e));
        g_addr[dev] = ptr;
    }
    *out = g_addr[dev];
    return XS_OK;
}

}  // namespace

extern "C" {

int xs_moe_layer_decode_noalloc(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert,
                                int k, const float* x, const float* logits, const float* residual, float* out,
                                int n_tok, int32_t* status, void* stream) {
    if (n_tok <= 0) return XS_OK;
    if (!L) return xs::set_error(XS_EINVAL, "moe_layer_decode_noalloc: no layout");
    if (L->n_embd > xs::kScratchMaxEmbd || L->n_ff > xs::kScratchMaxFF)
        return xs::set_error(XS_EINVAL, "moe_layer_decode_noalloc: hidden " + std::to_string(L->n_embd) + " x F " +
                                            std::to_string(L->n_ff) + " is past the fixed scratch's layouts (hidden <= " +
                                            std::to_string(xs::kScratchMaxEmbd) + ", F <= " +
                                            std::to_string(xs::kScratchMaxFF) + ")");
    const size_t need = xs::layer_decode_fixed_bytes(L, n_expert, k, n_tok);
    if (need == 0) return xs::set_error(XS_EINVAL, "moe_layer_decode_noalloc: empty geometry");
    if (need > kScratchBytes)
        return xs::set_error(XS_EINVAL, "moe_layer_decode_noalloc: " + std::to_string(n_tok) + " tokens x top-" +
                                            std::to_string(k) + " need " + std::to_string(need) +
                                            " bytes of scratch, past the fixed " + std::to_string(kScratchBytes));
    void* ptr = nullptr;
    if (int r = scratch_address(&ptr)) return r;
    return xs::layer_decode_fixed(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, ptr,
                                  kScratchBytes, status, stream);
}

// the fixed scratch's own status word (its first int32, where calls with status == NULL OR their bits): this device's
int32_t* xs_moe_layer_decode_noalloc_status(void) {
    void* ptr = nullptr;
    if (scratch_address(&ptr)) return nullptr;
    return (int32_t*)ptr;
}

}  // extern "C"
