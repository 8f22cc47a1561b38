// include/xs_strata_kernels.hpp - the reference engine's C++ MoE kernel surface (namespace strata::kernels) over the
// C ABI of xs_moe.h, header-only: the same names, argument meanings and exceptions as the reference's headers, so the
// engine's callers (src/core/moe_window.cpp:191-245, src/core/plain_model.cpp:955-988, src/core/verify.cpp:1160-1360,
// src/prefill/plain_prompt.cpp:558-797) build against it unchanged.  A failing call throws
// strata::core::DeviceError (a HIP error) or std::invalid_argument (geometry, alignment, overlap, a missing stream),
// as the reference's entry points do.
//
// DeviceError is the engine's own class (include/strata/core/device.hpp:66): in an engine build that header is on
// the include path and is included here.  A translation unit that declares the class itself before this header
// defines XS_STRATA_HAVE_DEVICE_ERROR; only a build with neither gets the stand-alone definition below.
#pragma once

#include "xs_moe.h"

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#if __has_include("strata/core/device.hpp")
#include "strata/core/device.hpp"
#elif !defined(XS_STRATA_HAVE_DEVICE_ERROR)
namespace strata::core {
class DeviceError : public std::runtime_error {   // stand-alone builds only: the engine's is device.hpp's
public:
    using std::runtime_error::runtime_error;
};
}  // namespace strata::core
#endif

namespace strata::kernels {

namespace detail {
inline void check(int code) {
    if (code == XS_OK) return;
    if (code == XS_EINVAL) throw std::invalid_argument(xs_last_error());
    throw core::DeviceError(xs_last_error());
}
}  // namespace detail

/// include/strata/kernels/iq_kernels.hpp:66-75
struct NativeExpertLayout {
    int gu_type = -1, d_type = -1;
    int up_type = -1;
    int64_t n_embd = 0, n_ff = 0;
    size_t gu_row = 0, d_row = 0;
    size_t up_row = 0;
    size_t up_off = 0, down_off = 0;
    size_t bytes = 0;
};

namespace detail {
inline xs_expert_layout_t to_c(const NativeExpertLayout& L) {
    xs_expert_layout_t c;
    c.gu_type = L.gu_type;
    c.d_type = L.d_type;
    c.up_type = L.up_type;
    c.n_embd = L.n_embd;
    c.n_ff = L.n_ff;
    c.gu_row = L.gu_row;
    c.d_row = L.d_row;
    c.up_row = L.up_row;
    c.up_off = L.up_off;
    c.down_off = L.down_off;
    c.bytes = L.bytes;
    return c;
}
}  // namespace detail

/// include/strata/kernels/iq_kernels.hpp:22
inline size_t iq_row_bytes(int ggml_type, int64_t n) noexcept { return xs_iq_row_bytes(ggml_type, n); }

/// include/strata/kernels/iq_kernels.hpp:79
inline bool native_expert_supported(int gu, int d, int64_t n_embd, int64_t n_ff, int up = -1) noexcept {
    return xs_native_expert_supported(gu, d, n_embd, n_ff, up) != 0;
}

/// include/strata/kernels/iq_kernels.hpp:81
inline NativeExpertLayout native_expert_layout(int gu, int d, int64_t n_embd, int64_t n_ff, int up = -1) {
    xs_expert_layout_t c;
    detail::check(xs_native_expert_layout(gu, d, n_embd, n_ff, up, &c));
    NativeExpertLayout L;
    L.gu_type = c.gu_type;
    L.d_type = c.d_type;
    L.up_type = c.up_type;
    L.n_embd = c.n_embd;
    L.n_ff = c.n_ff;
    L.gu_row = c.gu_row;
    L.d_row = c.d_row;
    L.up_row = c.up_row;
    L.up_off = c.up_off;
    L.down_off = c.down_off;
    L.bytes = c.bytes;
    return L;
}

/// include/strata/kernels/iq_kernels.hpp:83
inline size_t native_expert_scratch_bytes(int64_t cap_entries, int64_t n_ff) {
    return xs_native_expert_scratch_bytes(cap_entries, n_ff);
}

/// include/strata/kernels/iq_kernels.hpp:26
inline void quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, void* y, void* stream) {
    detail::check(xs_quantize_q8_1_rows(x, n_rows, n_cols, y, stream));
}

/// include/strata/kernels/iq_kernels.hpp:30
inline void iq_dequant_f32(int ggml_type, const void* src, int64_t n, float* dst, void* stream) {
    detail::check(xs_iq_dequant_f32(ggml_type, src, n, dst, stream));
}

/// include/strata/kernels/iq_kernels.hpp:32 (IEEE half bits)
inline void iq_dequant_f16(int ggml_type, const void* src, int64_t n, uint16_t* dst, void* stream) {
    detail::check(xs_iq_dequant_f16(ggml_type, src, n, dst, stream));
}

/// include/strata/kernels/iq_mmq.hpp:33 (the int8 activations' bytes)
inline size_t iq_mmq_act_bytes(int64_t rows, int64_t cols) { return xs_iq_mmq_act_bytes(rows, cols); }
/// include/strata/kernels/iq_mmq.hpp:35
inline bool iq_mmq_type_sums(int ggml_type) { return xs_iq_mmq_type_sums(ggml_type) != 0; }
/// include/strata/kernels/iq_mmq.hpp:38
inline bool iq_mmq_type_dup(int ggml_type) { return xs_iq_mmq_type_dup(ggml_type) != 0; }
/// include/strata/kernels/iq_mmq.hpp:39-41; the reference's sycl::queue& is the stream here, and the call is
/// asynchronous on it (the reference returns the event)
inline void iq_mmq_quantize(void* stream, const float* x, const int32_t* ids, void* xq, int64_t cols, int64_t ld,
                            int64_t rows, bool sums, bool dup = false) {
    detail::check(xs_iq_mmq_quantize(x, ids, xq, cols, ld, rows, sums, dup, stream));
}
/// include/strata/kernels/iq_mmq.hpp:46-47
inline void iq_mmq_quantize_scatter(void* stream, const float* x, const int32_t* slot, void* xq, int64_t cols,
                                    int64_t ld, int64_t tokens, int k_used, bool sums, bool dup = false) {
    detail::check(xs_iq_mmq_quantize_scatter(x, slot, xq, cols, ld, tokens, k_used, sums, dup, stream));
}

/// include/strata/kernels/iq_kernels.hpp:90-93
inline void native_expert_grouped(const NativeExpertLayout& L, const unsigned long long* grp_ptr,
                                  const int32_t* grp_start, const int32_t* n_groups, const int32_t* ent_dst,
                                  const int32_t* ent_tok, int64_t cap_groups, int64_t cap_entries, const void* x_q8_1,
                                  void* scratch, float* out, void* stream, int64_t grid_groups = 0) {
    const xs_expert_layout_t c = detail::to_c(L);
    detail::check(xs_native_expert_grouped(&c, grp_ptr, grp_start, n_groups, ent_dst, ent_tok, cap_groups, cap_entries,
                                           x_q8_1, scratch, out, stream, grid_groups));
}

/// include/strata/kernels/router_top10.hpp:20-21 (a null stream synchronises)
inline void router_top10(const float* logits, int n_tokens, int n_expert, int k, int* ids, float* weights,
                         void* stream) {
    detail::check(xs_router_top10(logits, n_tokens, n_expert, k, ids, weights, stream));
}

/// include/strata/kernels/verify_kernels.hpp:81-83 (the reference's native kernels require an explicit queue)
inline void resident_plan(const int32_t* ids, int n_entries, int k, const int32_t* res_layer, int n_expert,
                          const uint8_t* cache_base, const unsigned long long* slot_off, long long blob, int32_t* plan,
                          long long capx, uint32_t* skip, uint32_t ring, void* stream) {
    if (!stream) throw std::invalid_argument("resident_plan requires an explicit stream");
    if (!res_layer) throw std::invalid_argument("resident_plan requires the layer's residency table");
    detail::check(xs_resident_plan(ids, n_entries, k, res_layer, n_expert, cache_base, slot_off, blob, plan, capx, skip,
                                   ring, stream));
}

/// include/strata/kernels/native_moe.hpp:22-23
inline void native_moe_combine(const float* parts, const float* weights, const float* shared, float* output,
                               int64_t n_embd, int64_t k, void* stream) {
    if (!stream) throw std::invalid_argument("native MoE combine requires a stream, positive width and 1..15 experts");
    detail::check(xs_native_moe_combine(parts, weights, shared, output, n_embd, k, stream));
}

/// include/strata/kernels/native_moe.hpp:24-25
inline void native_moe_combine_multi(const float* parts, const float* weights, const float* shared, float* output,
                                     int64_t n_embd, int64_t k, int n_tok, void* stream,
                                     const float* shared_gate = nullptr) {
    if (!stream)
        throw std::invalid_argument("native MoE combine (multi) requires a stream, width, 1..15 experts, tokens");
    detail::check(xs_native_moe_combine_multi(parts, weights, shared, output, n_embd, k, n_tok, stream, shared_gate));
}

/// include/strata/kernels/native_moe.hpp:30-32
inline void native_moe_combine_multi_hits(const float* parts, const float* hits, const int32_t* dst,
                                          const int32_t* count, const float* weights, const float* shared,
                                          float* output, int64_t n_embd, int64_t k, int n_tok, void* stream,
                                          const float* shared_gate = nullptr) {
    if (!stream)
        throw std::invalid_argument("native MoE combine (hits) requires a stream, width, 1..15 experts, tokens, hits");
    detail::check(xs_native_moe_combine_multi_hits(parts, hits, dst, count, weights, shared, output, n_embd, k, n_tok,
                                                   stream, shared_gate));
}
/// include/strata/kernels/native_moe.hpp:29: this library always fuses the hit add
inline bool native_moe_fuse_hits() { return true; }

/// src/core/plain_model.cpp:987 (add_inplace)
inline void add_inplace(float* x, const float* y, int64_t n, void* stream) {
    detail::check(xs_add_inplace(x, y, n, stream));
}

/// The whole decode MoE layer (the engine's moe_route + moe_finish, src/core/plain_model.cpp:951-988) in one call,
/// every expert resident in `arena`.  Asynchronous: the persistent form's co-residency is a checked contract, so the
/// caller runs moe_layer_check(workspace, stream) at its next synchronisation point, which throws
/// core::DeviceError when a bounded wait expired (the layer's work-groups were not all resident) or a router row was
/// NaN; that call's output is then not to be used.
inline void moe_layer_decode(const NativeExpertLayout& L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                             const float* x, const float* logits, const float* residual, float* out, int n_tok,
                             void* workspace, size_t workspace_bytes, void* stream) {
    if (!stream) throw std::invalid_argument("moe_layer_decode requires an explicit stream");
    const xs_expert_layout_t c = detail::to_c(L);
    detail::check(xs_moe_layer_decode(&c, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, workspace,
                                      workspace_bytes, stream));
}
inline size_t moe_layer_decode_workspace_bytes(const NativeExpertLayout& L, int n_expert, int k, int n_tok) {
    const xs_expert_layout_t c = detail::to_c(L);
    return xs_moe_layer_decode_workspace_bytes(&c, n_expert, k, n_tok);
}
/// Synchronises `stream` and throws core::DeviceError when the decode workspace's status word is set (then cleared).
inline void moe_layer_check(void* workspace, void* stream) {
    detail::check(xs_moe_status_check(xs_moe_layer_decode_status(workspace), stream));
}
/// The prompt / verify layer (src/prefill/plain_prompt.cpp:558-797) in one call.
inline void moe_layer_prefill(const NativeExpertLayout& L, const uint8_t* arena, size_t blob_bytes, int n_expert,
                              int k, const float* x, const float* logits, const float* residual, float* out, int n_tok,
                              void* workspace, size_t workspace_bytes, void* stream) {
    if (!stream) throw std::invalid_argument("moe_layer_prefill requires an explicit stream");
    const xs_expert_layout_t c = detail::to_c(L);
    detail::check(xs_moe_layer_prefill(&c, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, workspace,
                                       workspace_bytes, stream));
}
inline size_t moe_layer_prefill_workspace_bytes(const NativeExpertLayout& L, int n_expert, int k, int n_tok) {
    const xs_expert_layout_t c = detail::to_c(L);
    return xs_moe_layer_prefill_workspace_bytes(&c, n_expert, k, n_tok);
}

/// include/strata/kernels/bf16_gemv.hpp:48-49 (one token).
inline void bf16_gemv_fp32_mmvf(const float* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out,
                                void* stream) {
    detail::check(xs_bf16_gemv_fp32_mmvf_multi(x, n_in, w, y, n_out, n_in, n_out, 1, stream));
}
/// include/strata/kernels/bf16_gemv.hpp:52 (one token).
inline void f32_gemv_fp32_mmvf(const float* x, const float* w, float* y, int64_t n_in, int64_t n_out, void* stream) {
    detail::check(xs_f32_gemv_fp32_mmvf_multi(x, n_in, w, y, n_out, n_in, n_out, 1, stream));
}
/// include/strata/kernels/bf16_gemv.hpp:55-56
inline void f32_gemv_fp32_mmvf_multi(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy,
                                     int64_t n_in, int64_t n_out, int n_tok, void* stream) {
    detail::check(xs_f32_gemv_fp32_mmvf_multi(x, ldx, w, y, ldy, n_in, n_out, n_tok, stream));
}
/// include/strata/kernels/bf16_gemv.hpp:64-65
inline void bf16_gemv_fp32_mmvf_multi(const float* x, int64_t ldx, const uint16_t* w, float* y, int64_t ldy,
                                      int64_t n_in, int64_t n_out, int n_tok, void* stream) {
    detail::check(xs_bf16_gemv_fp32_mmvf_multi(x, ldx, w, y, ldy, n_in, n_out, n_tok, stream));
}
/// include/strata/kernels/bf16_gemv.hpp:60-61
inline void f32_gemm_rows(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in,
                          int64_t n_out, int64_t n_tok, void* stream) {
    detail::check(xs_f32_gemm_rows(x, ldx, w, y, ldy, n_in, n_out, n_tok, stream));
}
/// include/strata/kernels/bf16_gemv.hpp:30
inline void bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out, void* stream) {
    detail::check(xs_bf16_gemv(x, w, y, n_in, n_out, stream));
}
/// include/strata/kernels/bf16_gemv.hpp:38-39
inline void bf16_gemv_split(const uint16_t* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out,
                            int threads_per_row, void* stream) {
    detail::check(xs_bf16_gemv_split(x, w, y, n_in, n_out, threads_per_row, stream));
}
/// include/strata/kernels/elementwise.hpp:71
inline void f32_to_bf16_bulk(const float* x, uint16_t* y, int64_t n, void* stream) {
    detail::check(xs_f32_to_bf16_bulk(x, y, n, stream));
}

/// include/strata/kernels/iq_mmq.hpp:53-58 (the stream in place of the queue).
inline void iq_mmq_grouped(void* stream, int ggml_type, const void* w, size_t expert_bytes, int64_t w_rows,
                           int64_t w_cols, int n, const void* xq, int64_t total_rows, const int32_t* bounds,
                           int64_t max_rows, const int32_t* ids, float* dst, int64_t ld_dst,
                           const uint8_t* const* wtab = nullptr, size_t woff = 0, int64_t rows = 0) {
    detail::check(xs_iq_mmq_grouped(ggml_type, w, expert_bytes, w_rows, w_cols, n, xq, total_rows, bounds, max_rows,
                                    ids, dst, ld_dst, wtab, woff, rows, stream));
}

}  // namespace strata::kernels

namespace strata::prefill::mmq {

/// include/strata/prefill/moe_mmq.hpp:57-72: one grouped product over n experts.
struct Product {
    const void* w = nullptr;
    int type = -1;
    int64_t w_rows = 0, w_cols = 0;
    size_t expert_bytes = 0;
    int n = 0;
    const void* xq = nullptr;
    const int32_t* bounds = nullptr;
    const int32_t* ids = nullptr;
    int64_t total_rows = 0, max_rows = 0;
    int64_t rows = 0;
    float* dst = nullptr;
    int64_t ld_dst = 0;
    const uint8_t* const* wtab = nullptr;
    size_t woff = 0;
};

/// include/strata/prefill/moe_mmq.hpp:74-84: the launch context.  It holds nothing: the product allocates nothing and
/// keeps no state (one launch), so one Context per prompt path, as the reference has it, costs nothing.
class Context {
public:
    void run(const Product& p, void* stream) {
        kernels::detail::check(xs_iq_mmq_grouped(p.type, p.w, p.expert_bytes, p.w_rows, p.w_cols, p.n, p.xq,
                                                 p.total_rows, p.bounds, p.max_rows, p.ids, p.dst, p.ld_dst, p.wtab,
                                                 p.woff, p.rows, stream));
    }
};

/// include/strata/prefill/moe_mmq.hpp:41-43
inline size_t q8_bytes(int64_t rows, int64_t cols) { return xs_iq_mmq_act_bytes(rows, cols); }
/// include/strata/prefill/moe_mmq.hpp:46-49
inline void quantize(const float* x, const int32_t* ids, void* xq, int ggml_type, int64_t cols, int64_t ld,
                     int64_t rows, void* stream) {
    kernels::detail::check(xs_iq_mmq_quantize(x, ids, xq, cols, ld, rows, xs_iq_mmq_type_sums(ggml_type),
                                              xs_iq_mmq_type_dup(ggml_type), stream));
}
/// include/strata/prefill/moe_mmq.hpp:50-55 (src, the gathered form's map, is not needed by the scatter)
inline void quantize_scatter(const float* x, const int32_t* slot, const int32_t* /*src*/, void* xq, int ggml_type,
                             int64_t cols, int64_t ld, int64_t tokens, int k_used, void* stream) {
    kernels::detail::check(xs_iq_mmq_quantize_scatter(x, slot, xq, cols, ld, tokens, k_used,
                                                      xs_iq_mmq_type_sums(ggml_type), xs_iq_mmq_type_dup(ggml_type),
                                                      stream));
}
/// include/strata/prefill/moe_mmq.hpp:106-108
inline void swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, bool interleaved, void* stream) {
    kernels::detail::check(xs_mmq_swiglu(gu, h, rows, n_ff, interleaved, stream));
}
/// include/strata/prefill/moe_mmq.hpp:110
inline void iota(int32_t* dst, int64_t n, void* stream) { kernels::detail::check(xs_mmq_iota(dst, n, stream)); }

}  // namespace strata::prefill::mmq
