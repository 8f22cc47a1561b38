// xestrata-win_amd/csrc/abi.cpp - the C ABI (include/xs_moe.h): argument checks with the reference's rules, the
// thread's error message, and the launches.  Nothing here allocates device memory.
#include "../../include/xs_moe.h"
#include "xs_kernels.h"
#include "xs_plan.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>
#include <vector>
#include <string>

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
int ok() { return XS_OK; }
int hip_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(XS_EDEVICE, "%s: %s", what, hipGetErrorString(e));
    return ok();
}
hipStream_t S(void* s) { return (hipStream_t)s; }
// a NULL stream: the default stream, then a wait (the reference's sync_if_needed)
int finish(void* stream, hipError_t launched, const char* what) {
    if (launched != hipSuccess) return hip_status(launched, what);
    if (!stream) return hip_status(hipStreamSynchronize(nullptr), what);
    return ok();
}
bool aligned(const void* p, size_t a) { return p && ((uintptr_t)p % a) == 0; }
bool overlap(const void* a, size_t an, const void* b, size_t bn) {
    const auto ap = (uintptr_t)a, bp = (uintptr_t)b;
    return a && b && ap < bp + bn && bp < ap + an;
}
size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// the bound of the persistent decode layers' waits (each normally a few microseconds): 50 ms of the device's wall
// clock, or the ticks xs_moe_set_wait_bound set; 0 when it asked every wait to expire at once (the kernels then take
// no hand-over word: a test of the expired-wait path forced from the host)
std::atomic<long long> g_wait_bound{0};
// the prompt layer's tall-tile split (xs_moe_set_prefill_tall): on unless switched off
std::atomic<int> g_tall{1};
int help_all() { return g_wait_bound.load(std::memory_order_relaxed) == -2 ? 1 : 0; }
long long spin_ticks() {
    const long long set = g_wait_bound.load(std::memory_order_relaxed);
    if (set > 0) return set;
    if (set == -1) return 0;
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess ||
        khz <= 0)
        khz = 100000;
    return (long long)khz * 50;
}

int type_qk(int t) { return t == 8 ? 32 : (t == 12 || t == 14 || t == 23) ? 256 : 0; }
int type_bytes(int t) { return t == 8 ? 34 : t == 12 ? 144 : t == 14 ? 210 : t == 23 ? 136 : 0; }

xs::ExpertLayout to_layout(const xs_expert_layout_t* L) {
    xs::ExpertLayout x;
    x.gu_type = L->gu_type;
    x.d_type = L->d_type;
    x.n_embd = L->n_embd;
    x.n_ff = L->n_ff;
    x.gu_row = (int64_t)L->gu_row;
    x.d_row = (int64_t)L->d_row;
    x.up_off = (int64_t)L->up_off;
    x.down_off = (int64_t)L->down_off;
    x.bytes = (int64_t)L->bytes;
    x.up_type = L->up_type >= 0 ? L->up_type : L->gu_type;
    x.up_row = L->up_row ? (int64_t)L->up_row : x.gu_row;
    return x;
}

int check_layout(const xs_expert_layout_t* L, const char* what) {
    if (!L) return fail(XS_EINVAL, "%s: no layout", what);
    if (!xs_native_expert_supported(L->gu_type, L->d_type, L->n_embd, L->n_ff, L->up_type))
        return fail(XS_EINVAL, "%s: gate/up type %d, down type %d at %lld x %lld is not supported", what, L->gu_type,
                    L->d_type, (long long)L->n_embd, (long long)L->n_ff);
    xs_expert_layout_t want;
    if (xs_native_expert_layout(L->gu_type, L->d_type, L->n_embd, L->n_ff, L->up_type, &want) != XS_OK) return XS_EINVAL;
    if (want.bytes != L->bytes || want.up_off != L->up_off || want.down_off != L->down_off || want.up_row != L->up_row)
        return fail(XS_EINVAL, "%s: the layout's offsets are not native_expert_layout's", what);
    return ok();
}

// the plan's words for capx entries (xs_plan.h)
size_t plan_words(long long capx) { return (size_t)xs::PlanWords{capx}.words(); }

}  // namespace

namespace xs {
int set_error(int code, const std::string& message) {
    g_err = message;
    return code;
}
}  // namespace xs

extern "C" {

const char* xs_last_error(void) { return g_err.c_str(); }
int xs_abi_version(void) { return 1; }

size_t xs_iq_row_bytes(int type, int64_t n) {
    const int qk = type_qk(type);
    return qk && n > 0 && n % qk == 0 ? (size_t)(n / qk) * (size_t)type_bytes(type) : 0;
}

// the gate/up and down types of the four formats; every row a whole number of blocks; n_embd a whole number of 256s
// (the q8_1 activation's 256-value scale; reference iq_kernels.cpp:2002-2019) and of 32s of units per lane set.  A
// mixed layer (up_type >= 0 and not the gate's): gate and up each a gate/up type of its own (iq_kernels.cpp:2003-2005)
int xs_native_expert_supported(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, int up_type) {
    if (up_type >= 0 && up_type != gu_type && (!type_qk(up_type) || n_embd % type_qk(up_type))) return 0;
    if (!type_qk(gu_type) || !type_qk(d_type)) return 0;
    if (n_embd <= 0 || n_ff <= 0 || n_embd % 256 || n_ff % 32) return 0;
    if (n_embd % type_qk(gu_type) || n_ff % type_qk(d_type)) return 0;
    if (n_embd > (1 << 20) || n_ff > (1 << 20)) return 0;
    return 1;
}

int xs_native_expert_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, int up_type,
                            xs_expert_layout_t* out) {
    if (!out) return fail(XS_EINVAL, "native_expert_layout: no output");
    if (!xs_native_expert_supported(gu_type, d_type, n_embd, n_ff, up_type))
        return fail(XS_EINVAL, "native_expert_layout: gate/up type %d, down type %d at %lld x %lld not supported",
                    gu_type, d_type, (long long)n_embd, (long long)n_ff);
    out->gu_type = gu_type;
    out->d_type = d_type;
    out->up_type = up_type >= 0 ? up_type : gu_type;
    out->n_embd = n_embd;
    out->n_ff = n_ff;
    out->gu_row = xs_iq_row_bytes(gu_type, n_embd);
    out->up_row = xs_iq_row_bytes(out->up_type, n_embd);
    out->d_row = xs_iq_row_bytes(d_type, n_ff);
    out->up_off = (size_t)n_ff * out->gu_row;
    out->down_off = out->up_off + (size_t)n_ff * out->up_row;
    out->bytes = out->down_off + (size_t)n_embd * out->d_row;
    return ok();
}

size_t xs_native_expert_scratch_bytes(int64_t cap, int64_t n_ff) {
    if (cap <= 0 || n_ff <= 0) return 0;
    const size_t f = (size_t)cap * (size_t)n_ff * sizeof(float);
    return 3 * up256(f) + up256((size_t)cap * (size_t)(n_ff / 32) * 36) + 256;
}

int32_t* xs_native_expert_status(void* scratch, int64_t cap, int64_t n_ff) {
    if (!scratch || cap <= 0 || n_ff <= 0) return nullptr;
    return (int32_t*)((uint8_t*)scratch + xs_native_expert_scratch_bytes(cap, n_ff) - 256);
}

int xs_quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, void* y, void* stream) {
    if (n_rows * n_cols <= 0) return ok();
    if (n_cols % 32) return fail(XS_EINVAL, "quantize_q8_1_rows: n_cols %lld is not a multiple of 32", (long long)n_cols);
    if (!aligned(x, 4) || !aligned(y, 4)) return fail(XS_EINVAL, "quantize_q8_1_rows: unaligned span");
    return finish(stream, xs::launch_quantize_q8_1_rows(x, n_rows, n_cols, y, S(stream)), "quantize_q8_1_rows");
}

size_t xs_iq_mmq_act_bytes(int64_t rows, int64_t cols) {
    return rows > 0 && cols > 0 ? (size_t)(rows * cols + 2 * rows * (cols / 32) * 4) : 0;
}
int xs_iq_mmq_type_sums(int type) { return type == 12 /* Q4_K */ || type == 13 /* Q5_K */; }
int xs_iq_mmq_type_dup(int type) { return type == 10 /* Q2_K */; }

int xs_iq_mmq_quantize(const float* x, const int32_t* ids, void* xq, int64_t cols, int64_t ld, int64_t rows, int sums,
                       int dup, void* stream) {
    if (rows <= 0) return ok();
    if (cols <= 0 || cols % 32 || ld < cols || ld % 4)
        return fail(XS_EINVAL, "iq_mmq_quantize: %lld columns (a multiple of 32), %lld floats a row", (long long)cols,
                    (long long)ld);
    if (!aligned(x, 16) || !aligned(xq, 4) || (ids && !aligned(ids, 4)))
        return fail(XS_EINVAL, "iq_mmq_quantize: a span is missing or misaligned");
    return finish(stream, xs::launch_mmq_quantize(x, ids, xq, cols, ld, rows, rows, 1, false, sums, dup, S(stream)),
                  "iq_mmq_quantize");
}

int xs_iq_mmq_quantize_scatter(const float* x, const int32_t* slot, void* xq, int64_t cols, int64_t ld,
                               int64_t tokens, int k_used, int sums, int dup, void* stream) {
    if (tokens <= 0) return ok();
    if (cols <= 0 || cols % 32 || ld < cols || ld % 4 || k_used < 1)
        return fail(XS_EINVAL, "iq_mmq_quantize_scatter: %lld columns (a multiple of 32), %lld floats a row, k %d",
                    (long long)cols, (long long)ld, k_used);
    if (!aligned(x, 16) || !aligned(xq, 4) || !aligned(slot, 4))
        return fail(XS_EINVAL, "iq_mmq_quantize_scatter: a span is missing or misaligned");
    return finish(stream,
                  xs::launch_mmq_quantize(x, slot, xq, cols, ld, tokens, tokens * k_used, k_used, true, sums, dup,
                                          S(stream)),
                  "iq_mmq_quantize_scatter");
}

int xs_mmq_swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, int interleaved, void* stream) {
    if (rows <= 0) return ok();
    if (n_ff <= 0 || !aligned(gu, 4) || !aligned(h, 4))
        return fail(XS_EINVAL, "mmq swiglu: %lld values a row, or a span is missing", (long long)n_ff);
    return finish(stream, xs::launch_mmq_swiglu(gu, h, rows, n_ff, interleaved != 0, S(stream)), "mmq swiglu");
}

int xs_mmq_iota(int32_t* dst, int64_t n, void* stream) {
    if (n <= 0) return ok();
    if (!aligned(dst, 4) || n > INT32_MAX) return fail(XS_EINVAL, "mmq iota: a span is missing or too long");
    return finish(stream, xs::launch_iota(dst, n, S(stream)), "mmq iota");
}

namespace {
int grouped_args(const xs_expert_layout_t* L, const unsigned long long* grp_ptr, const int32_t* grp_start,
                 const int32_t* n_groups, const int32_t* ent_dst, const int32_t* ent_tok, int64_t cap_groups,
                 int64_t cap_entries, const void* x_q8_1, void* scratch, float* out, int64_t grid_groups,
                 const char* what, xs::GroupedArgs* a) {
    if (int r = check_layout(L, what)) return r;
    if (cap_groups > 65535) return fail(XS_EINVAL, "%s: cap_groups %lld", what, (long long)cap_groups);
    if (!aligned(grp_ptr, 8) || !aligned(grp_start, 4) || !aligned(n_groups, 4) || (ent_dst && !aligned(ent_dst, 4)) ||
        (ent_tok && !aligned(ent_tok, 4)) || (x_q8_1 && !aligned(x_q8_1, 4)) || !aligned(scratch, 16) ||
        (out && !aligned(out, 4)))
        return fail(XS_EINVAL, "%s: a span is missing or misaligned", what);
    const size_t f = (size_t)cap_entries * (size_t)L->n_ff * sizeof(float), fa = up256(f);
    a->grp_ptr = grp_ptr;
    a->grp_start = grp_start;
    a->n_groups = n_groups;
    a->ent_dst = ent_dst;
    a->ent_tok = ent_tok;
    a->x_q8_1 = x_q8_1;
    a->gate = (float*)scratch;
    a->up = (float*)((uint8_t*)scratch + fa);
    a->hq = (uint8_t*)scratch + 3 * fa;
    a->hact = (uint8_t*)scratch + 2 * fa;
    a->cap_entries_hint = cap_entries;
    a->out = out;
    a->err = xs_native_expert_status(scratch, cap_entries, L->n_ff);
    a->cap_groups = cap_groups;
    a->grid_groups = grid_groups;
    a->max_entries = 0;
    return ok();
}

// max_entries: the most entries one group can hold (the call's token count), 0 when not known
int grouped_impl(const xs_expert_layout_t* L, const unsigned long long* grp_ptr, const int32_t* grp_start,
                 const int32_t* n_groups, const int32_t* ent_dst, const int32_t* ent_tok, int64_t cap_groups,
                 int64_t cap_entries, const void* x_q8_1, void* scratch, float* out, void* stream, int64_t grid_groups,
                 int max_entries) {
    if (cap_groups <= 0 || cap_entries <= 0) return ok();
    if (!ent_dst || !ent_tok || !x_q8_1 || !out) return fail(XS_EINVAL, "native_expert_grouped: a span is missing");
    xs::GroupedArgs a;
    if (int r = grouped_args(L, grp_ptr, grp_start, n_groups, ent_dst, ent_tok, cap_groups, cap_entries, x_q8_1,
                             scratch, out, grid_groups, "native_expert_grouped", &a))
        return r;
    a.max_entries = max_entries;
    const xs::ExpertLayout XL = to_layout(L);
    hipError_t e;
    if (xs::stream_usable(XL, max_entries, cap_groups, cap_entries)) {   // the weight-stream kernels (the same bits)
        e = xs::launch_stream_gu(XL, a, S(stream));
        if (e == hipSuccess) e = xs::launch_stream_down(XL, a, S(stream));
    } else {
        e = xs::launch_native_gu(XL, a, S(stream));
        if (e == hipSuccess) e = xs::launch_native_down(XL, a, S(stream));
    }
    return finish(stream, e, "native_expert_grouped");
}
}  // namespace

int xs_native_expert_grouped(const xs_expert_layout_t* L, const unsigned long long* grp_ptr,
                             const int32_t* grp_start, const int32_t* n_groups, const int32_t* ent_dst,
                             const int32_t* ent_tok, int64_t cap_groups, int64_t cap_entries, const void* x_q8_1,
                             void* scratch, float* out, void* stream, int64_t grid_groups) {
    return grouped_impl(L, grp_ptr, grp_start, n_groups, ent_dst, ent_tok, cap_groups, cap_entries, x_q8_1, scratch,
                        out, stream, grid_groups, 0);
}

int xs_native_expert_gate_up(const xs_expert_layout_t* L, const unsigned long long* grp_ptr, const int32_t* grp_start,
                             const int32_t* n_groups, const int32_t* ent_tok, int64_t cap_groups, int64_t cap_entries,
                             const void* x_q8_1, void* scratch, void* stream, int64_t grid_groups) {
    if (cap_groups <= 0 || cap_entries <= 0) return ok();
    if (!ent_tok || !x_q8_1) return fail(XS_EINVAL, "native_expert_gate_up: a span is missing");
    xs::GroupedArgs a;
    if (int r = grouped_args(L, grp_ptr, grp_start, n_groups, nullptr, ent_tok, cap_groups, cap_entries, x_q8_1,
                             scratch, nullptr, grid_groups, "native_expert_gate_up", &a))
        return r;
    return finish(stream, xs::launch_native_gu(to_layout(L), a, S(stream)), "native_expert_gate_up");
}

int xs_native_expert_down(const xs_expert_layout_t* L, const unsigned long long* grp_ptr, const int32_t* grp_start,
                          const int32_t* n_groups, const int32_t* ent_dst, int64_t cap_groups, int64_t cap_entries,
                          void* scratch, float* out, void* stream, int64_t grid_groups) {
    if (cap_groups <= 0 || cap_entries <= 0) return ok();
    if (!ent_dst || !out) return fail(XS_EINVAL, "native_expert_down: a span is missing");
    xs::GroupedArgs a;
    if (int r = grouped_args(L, grp_ptr, grp_start, n_groups, ent_dst, nullptr, cap_groups, cap_entries, nullptr,
                             scratch, out, grid_groups, "native_expert_down", &a))
        return r;
    return finish(stream, xs::launch_native_down(to_layout(L), a, S(stream)), "native_expert_down");
}

int xs_iq_dequant_f32(int type, const void* src, int64_t n, float* dst, void* stream) {
    if (n <= 0) return ok();
    if (!type_qk(type) || n % type_qk(type)) return fail(XS_EINVAL, "iq_dequant_f32: type %d, %lld values", type, (long long)n);
    if (!src || !aligned(dst, 4)) return fail(XS_EINVAL, "iq_dequant_f32: a span is missing or misaligned");
    return finish(stream, xs::launch_dequant(type, src, n, dst, xs::kDequantF32, S(stream)), "iq_dequant_f32");
}

int xs_iq_dequant_bf16(int type, const void* src, int64_t n, uint16_t* dst, void* stream) {
    if (n <= 0) return ok();
    if (!type_qk(type) || n % type_qk(type)) return fail(XS_EINVAL, "iq_dequant_bf16: type %d, %lld values", type, (long long)n);
    if (!src || !aligned(dst, 2)) return fail(XS_EINVAL, "iq_dequant_bf16: a span is missing or misaligned");
    return finish(stream, xs::launch_dequant(type, src, n, dst, xs::kDequantBf16, S(stream)), "iq_dequant_bf16");
}

int xs_iq_dequant_f16(int type, const void* src, int64_t n, uint16_t* dst, void* stream) {
    if (n <= 0) return ok();
    if (!type_qk(type) || n % type_qk(type)) return fail(XS_EINVAL, "iq_dequant_f16: type %d, %lld values", type, (long long)n);
    if (!src || !aligned(dst, 2)) return fail(XS_EINVAL, "iq_dequant_f16: a span is missing or misaligned");
    return finish(stream, xs::launch_dequant(type, src, n, dst, xs::kDequantF16, S(stream)), "iq_dequant_f16");
}

int xs_quantize_rows(int type, const float* x, int64_t n, void* y, void* stream) {
    if (n <= 0) return ok();
    if (!type_qk(type) || n % type_qk(type)) return fail(XS_EINVAL, "quantize_rows: type %d, %lld values", type, (long long)n);
    if (!aligned(x, 4) || !y) return fail(XS_EINVAL, "quantize_rows: a span is missing or misaligned");
    return finish(stream, xs::launch_quantize_rows(type, x, n, y, S(stream)), "quantize_rows");
}

int xs_router_top10(const float* logits, int n_tokens, int n_expert, int k, int32_t* ids, float* weights,
                    void* stream) {
    if (n_tokens <= 0 || n_expert <= 0 || k <= 0) return ok();
    if (k > 64) return fail(XS_EINVAL, "router_top10: k %d exceeds the kernel's 64", k);
    if (n_expert > 1024) return fail(XS_EINVAL, "router_top10: n_expert %d is past the kernel's 1024", n_expert);
    if (k > n_expert) return fail(XS_EINVAL, "router_top10: k %d > n_expert %d", k, n_expert);
    if (!aligned(logits, 4) || !aligned(ids, 4) || !aligned(weights, 4))
        return fail(XS_EINVAL, "router_top10: a span is missing or misaligned");
    return finish(stream, xs::launch_router_topk(logits, n_tokens, n_expert, k, ids, weights, S(stream)), "router_top10");
}

int xs_router_grouped_sigmoid(const float* logits, const float* bias, int n_tokens, int n_expert, int n_group,
                              int topk_group, int k, float routed_scale, int32_t* ids, float* weights, void* stream) {
    if (n_tokens <= 0) return ok();
    if (n_expert <= 0 || n_expert > 1024 || n_group <= 0 || n_group > 64 || n_expert % n_group || topk_group <= 0 ||
        topk_group > n_group || k <= 0 || k > 64 || k > (n_expert / n_group) * topk_group)
        return fail(XS_EINVAL, "router_grouped_sigmoid: geometry %d experts, %d groups, top %d groups, k %d", n_expert,
                    n_group, topk_group, k);
    if (!aligned(logits, 4) || !aligned(ids, 4) || !aligned(weights, 4) || (bias && !aligned(bias, 4)))
        return fail(XS_EINVAL, "router_grouped_sigmoid: a span is missing or misaligned");
    return finish(stream, xs::launch_router_grouped_sigmoid(logits, bias, n_tokens, n_expert, n_group, topk_group, k,
                                                            routed_scale, ids, weights, S(stream)),
                  "router_grouped_sigmoid");
}

int xs_router_logits_f32(const float* x, const float* w, float* logits, int n_tokens, int64_t n_embd, int n_expert,
                         void* stream) {
    if (n_tokens <= 0 || n_expert <= 0) return ok();
    if (n_tokens <= 8) return xs_f32_gemv_fp32_mmvf_multi(x, n_embd, w, logits, n_expert, n_embd, n_expert, n_tokens, stream);
    return xs_f32_gemm_rows(x, n_embd, w, logits, n_expert, n_embd, n_expert, n_tokens, stream);
}

namespace {
int mmvf_args(const float* x, int64_t ldx, const void* w, const float* y, int64_t ldy, int64_t n_in, int64_t n_out,
              int n_tok, const char* what) {
    if (n_tok < 1 || n_tok > 8 || n_in <= 0 || (n_in & 1) || n_in > INT32_MAX || n_out <= 0 || n_out > INT32_MAX ||
        (ldx & 1) || ldx < n_in || ldy < (n_tok > 1 ? n_out : 1))
        return fail(XS_EINVAL, "%s: 1..8 rows, even n_in/ldx, aligned pointers", what);
    if (!aligned(x, 8) || !aligned(w, 4) || !aligned(y, 4)) return fail(XS_EINVAL, "%s: null or misaligned pointer", what);
    return XS_OK;
}
}  // namespace

int xs_f32_gemv_fp32_mmvf_multi(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in,
                                int64_t n_out, int n_tok, void* stream) {
    if (int r = mmvf_args(x, ldx, w, y, ldy, n_in, n_out, n_tok, "f32_gemv_fp32_mmvf_multi")) return r;
    if (!aligned(w, 8)) return fail(XS_EINVAL, "f32_gemv_fp32_mmvf_multi: null or misaligned pointer");
    return finish(stream, xs::launch_mmvf<float>(x, ldx, w, y, ldy, n_in, n_out, n_tok, S(stream)),
                  "f32_gemv_fp32_mmvf_multi");
}

int xs_bf16_gemv_fp32_mmvf_multi(const float* x, int64_t ldx, const uint16_t* w, float* y, int64_t ldy, int64_t n_in,
                                 int64_t n_out, int n_tok, void* stream) {
    if (int r = mmvf_args(x, ldx, w, y, ldy, n_in, n_out, n_tok, "bf16_gemv_fp32_mmvf_multi")) return r;
    return finish(stream, xs::launch_mmvf<uint16_t>(x, ldx, w, y, ldy, n_in, n_out, n_tok, S(stream)),
                  "bf16_gemv_fp32_mmvf_multi");
}

int xs_f32_gemm_rows(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in, int64_t n_out,
                     int64_t n_tok, void* stream) {
    if (n_in <= 0 || n_out <= 0 || n_tok <= 0) return ok();
    if (!aligned(x, 4) || !aligned(w, 4) || !aligned(y, 4) || ldx < n_in || ldy < n_out || n_tok > 65535 * 64)
        return fail(XS_EINVAL, "f32_gemm_rows: null pointer or bad strides");
    return finish(stream, xs::launch_gemm_rows(x, ldx, w, y, ldy, n_in, n_out, n_tok, S(stream)), "f32_gemm_rows");
}

int xs_f32_to_bf16_bulk(const float* x, uint16_t* y, int64_t n, void* stream) {
    if (n <= 0) return ok();
    if (!aligned(x, 4) || !aligned(y, 2)) return fail(XS_EINVAL, "f32_to_bf16_bulk: null or misaligned pointer");
    return finish(stream, xs::launch_to_bf16(x, y, n, S(stream)), "f32_to_bf16_bulk");
}

int xs_bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out, void* stream) {
    if (n_in <= 0 || n_out <= 0) return ok();
    if (!aligned(x, 2) || !aligned(w, 2) || !aligned(y, 4)) return fail(XS_EINVAL, "bf16_gemv: null or misaligned pointer");
    return finish(stream,
                  xs::launch_bf16_gemv(x, false, w, y, n_in, n_out, n_out >= 64 ? xs::kBf16Warp : xs::kBf16Naive, 32,
                                       S(stream)),
                  "bf16_gemv");
}

int xs_bf16_gemv_split(const uint16_t* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out,
                       int threads_per_row, void* stream) {
    if (n_in <= 0 || n_out <= 0) return ok();
    if (!aligned(x, 2) || !aligned(w, 2) || !aligned(y, 4))
        return fail(XS_EINVAL, "bf16_gemv_split: null or misaligned pointer");
    if (threads_per_row == 32)
        return finish(stream, xs::launch_bf16_gemv(x, false, w, y, n_in, n_out, xs::kBf16Warp, 32, S(stream)),
                      "bf16_gemv_split(warp)");
    if (threads_per_row <= 0 || (threads_per_row & (threads_per_row - 1)) || threads_per_row > 1024)
        return fail(XS_EDEVICE, "bf16_gemv_split: threads_per_row %d must be a power of two (32 selects the "
                    "warp-per-row path)", threads_per_row);
    return finish(stream, xs::launch_bf16_gemv(x, false, w, y, n_in, n_out, xs::kBf16Tree, threads_per_row, S(stream)),
                  "bf16_gemv_split");
}

int xs_project_bf16(const float* x, uint16_t* x_bf16, const uint16_t* w, float* out, int64_t n_in, int64_t n_out,
                    int split, int native, void* stream) {
    if (n_in <= 0 || n_out <= 0) return ok();
    if (native) return xs_bf16_gemv_fp32_mmvf_multi(x, n_in, w, out, n_out, n_in, n_out, 1, stream);
    if (!x_bf16) {   // converted on the fly: the same bits as the two launches, with no bf16 copy of x
        if (!aligned(x, 4) || !aligned(w, 2) || !aligned(out, 4) || (!split && n_out < 64))
            return fail(XS_EINVAL, "project_bf16: a span is missing or misaligned (the on-the-fly form is the row-split "
                        "one)");
        return finish(stream, xs::launch_bf16_gemv(x, true, w, out, n_in, n_out, xs::kBf16Warp, 32, S(stream)),
                      "project_bf16");
    }
    if (int r = xs_f32_to_bf16_bulk(x, x_bf16, n_in, stream)) return r;
    return split ? xs_bf16_gemv_split(x_bf16, w, out, n_in, n_out, 32, stream)
                 : xs_bf16_gemv(x_bf16, w, out, n_in, n_out, stream);
}

void xs_plan_offsets(long long capx, long long* start, long long* dst, long long* tok, long long* ptr,
                     long long* start2) {
    const xs::PlanWords w{capx};
    if (start) *start = w.start();
    if (dst) *dst = w.dst();
    if (tok) *tok = w.tok();
    if (ptr) *ptr = w.ptr();
    if (start2) *start2 = w.start2();
}

int xs_resident_plan(const int32_t* ids, int n_entries, int k, const int32_t* res_layer, int n_expert,
                     const uint8_t* cache_base, const unsigned long long* slot_off, long long blob, int32_t* plan,
                     long long capx, uint32_t* skip, uint32_t ring, void* stream) {
    if (n_entries <= 0) return ok();
    if (n_entries > 1024) return fail(XS_EINVAL, "resident_plan: more entries (%d) than a work-group", n_entries);
    if (n_entries > capx || k <= 0 || n_expert <= 0 || n_expert > 16384)
        return fail(XS_EINVAL, "resident_plan: %d entries, capx %lld, k %d, %d experts", n_entries, capx, k, n_expert);
    if (!aligned(ids, 4) || !aligned(plan, 8) || !aligned(skip, 4) || (res_layer && !aligned(res_layer, 4)) ||
        (slot_off && !aligned(slot_off, 8)))
        return fail(XS_EINVAL, "resident_plan: a span is missing or misaligned");
    return finish(stream, xs::launch_resident_plan(ids, n_entries, k, res_layer, n_expert, cache_base, slot_off, blob,
                                                   plan, capx, skip, ring, S(stream)),
                  "resident_plan");
}

int xs_prefill_route(const int32_t* ids, int64_t n_entries, int k, int n_expert, int32_t* src, int32_t* slot,
                     int32_t* entry_of, int32_t* bounds, int32_t* experts, int32_t* n_groups,
                     const uint8_t* cache_base, long long blob, unsigned long long* grp_ptr, void* stream) {
    if (n_entries <= 0) return ok();
    if (k <= 0 || n_expert <= 0 || n_expert > 1024 || n_entries > (1ll << 30))
        return fail(XS_EINVAL, "prefill_route: %lld entries, k %d, %d experts", (long long)n_entries, k, n_expert);
    if (!aligned(ids, 4) || !aligned(src, 4) || !aligned(slot, 4) || !aligned(entry_of, 4) || !aligned(bounds, 4) ||
        !aligned(experts, 4) || !aligned(n_groups, 4) || (grp_ptr && !aligned(grp_ptr, 8)))
        return fail(XS_EINVAL, "prefill_route: a span is missing or misaligned");
    return finish(stream, xs::launch_prefill_route(ids, n_entries, k, n_expert, src, slot, entry_of, bounds, experts,
                                                   n_groups, cache_base, blob, grp_ptr, S(stream)),
                  "prefill_route");
}

size_t xs_moe_prefill_scratch_bytes(int64_t n_tok, int64_t rows, int64_t n_embd, int64_t n_ff) {
    if (n_tok <= 0 || rows <= 0) return 256;
    return up256((size_t)n_tok * (size_t)n_embd * 2) + up256((size_t)rows * (size_t)n_ff * 2) +
           up256((size_t)xs::tile_table_words(rows, rows) * 4) + 256;   // (cap_groups <= rows)
}

namespace {
// the m-tile table inside the experts' scratch: after the f16 copy of x and h
int32_t* prefill_mtile(void* scratch, int64_t n_tok, int64_t rows, const xs_expert_layout_t* L) {
    return (int32_t*)((uint8_t*)scratch + up256((size_t)n_tok * (size_t)L->n_embd * 2) +
                      up256((size_t)rows * (size_t)L->n_ff * 2));
}
// A side stream beside the caller's: per host thread and device (so that calls from several threads, or a graph
// captured on one of them, never share one), made on first use at the default priority and kept until the process
// ends, with two events for a fork (recorded on the caller's stream, waited for by the side stream) and a join
// (recorded on the side stream, waited for by the caller's; under graph capture these become the graph's branch and
// join).
struct SideStream {
    int dev;
    hipStream_t stream;
    hipEvent_t fork, join;
};
hipError_t side_stream_get(SideStream** out) {
    thread_local std::vector<SideStream> sides;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    for (SideStream& x : sides)
        if (x.dev == dev) {
            *out = &x;
            return hipSuccess;
        }
    SideStream x{dev, nullptr, nullptr, nullptr};
    if ((e = hipStreamCreateWithFlags(&x.stream, hipStreamNonBlocking)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&x.fork, hipEventDisableTiming)) != hipSuccess) return e;
    if ((e = hipEventCreateWithFlags(&x.join, hipEventDisableTiming)) != hipSuccess) return e;
    sides.push_back(x);
    *out = &sides.back();
    return hipSuccess;
}
// the side stream, forked from the caller's now
hipError_t side_stream_fork(hipStream_t caller, SideStream** out) {
    SideStream* sd = nullptr;
    hipError_t e = side_stream_get(&sd);
    if (e != hipSuccess) return e;
    if ((e = hipEventRecord(sd->fork, caller)) != hipSuccess) return e;
    if ((e = hipStreamWaitEvent(sd->stream, sd->fork, 0)) != hipSuccess) return e;
    *out = sd;
    return hipSuccess;
}

// the grouped experts writing fp32 parts, or f16 parts when parts_h is set (the whole-layer path); with `split` (a
// side stream of the caller's, and mtile written in the split form) the whole 256-row tiles run on the tall-tile
// GEMMs and the other rows beside them on the side stream
int prefill_experts(const xs_expert_layout_t* L, const float* x, int64_t n_tok, const int32_t* src,
                    const int32_t* entry_of, const int32_t* bounds, const int32_t* n_groups,
                    const unsigned long long* grp_ptr, int64_t cap_groups, int64_t rows, void* scratch, float* parts,
                    uint16_t* parts_h, bool mtile_ready, void* stream, const SideStream* split = nullptr,
                    int32_t* status = nullptr, bool xb_ready = false) {
    if (rows <= 0 || cap_groups <= 0) return ok();
    if (int r = check_layout(L, "moe_prefill_experts")) return r;
    if (cap_groups > rows) return fail(XS_EINVAL, "moe_prefill_experts: cap_groups %lld > rows %lld", (long long)cap_groups,
                                       (long long)rows);
    if (L->n_ff % 128 || L->n_embd % 256)
        return fail(XS_EINVAL, "moe_prefill_experts: n_ff %% 128 and n_embd %% 256 must be 0 (%lld, %lld)",
                    (long long)L->n_ff, (long long)L->n_embd);
    if (cap_groups > 65535 || !aligned(x, 4) || !aligned(src, 4) || !aligned(entry_of, 4) || !aligned(bounds, 4) ||
        !aligned(n_groups, 4) || !aligned(grp_ptr, 8) || !aligned(scratch, 256) ||
        !(parts_h ? aligned(parts_h, 2) : aligned(parts, 4)))
        return fail(XS_EINVAL, "moe_prefill_experts: a span is missing or misaligned");
    xs::PrefillArgs a;
    a.x = x;
    a.src = src;
    a.entry = entry_of;
    a.bounds = bounds;
    a.n_groups = n_groups;
    a.wptr = grp_ptr;
    a.xb = (uint16_t*)scratch;
    a.h = (uint16_t*)((uint8_t*)scratch + up256((size_t)n_tok * (size_t)L->n_embd * 2));
    a.mtile = prefill_mtile(scratch, n_tok, rows, L);
    a.mtile_ready = mtile_ready;
    a.xb_ready = xb_ready;
    // the f16 saturation bit goes to the caller's status word, else to the scratch's own (xs_moe_prefill_status)
    a.err = status ? status : xs_moe_prefill_status(scratch, n_tok, rows, L->n_embd, L->n_ff);
    a.parts = parts;
    a.parts_h = parts_h;
    a.n_tok = n_tok;
    a.rows = rows;
    a.cap_groups = cap_groups;
    a.ld_parts = L->n_embd;
    if (split)
        return finish(stream,
                      xs::launch_prefill_experts_split(to_layout(L), a, S(stream), split->stream, split->fork,
                                                       split->join),
                      "moe_prefill_experts");
    return finish(stream, xs::launch_prefill_experts(to_layout(L), a, S(stream)), "moe_prefill_experts");
}
}  // namespace

int xs_iq_mmq_grouped(int type, const void* w, size_t expert_bytes, int64_t w_rows, int64_t w_cols, int n,
                      const void* xq, int64_t total_rows, const int32_t* bounds, int64_t max_rows, const int32_t* ids,
                      float* dst, int64_t ld_dst, const uint8_t* const* wtab, size_t woff, int64_t rows,
                      void* stream) {
    (void)max_rows;   // the grid covers every row of xq; each work-group finds its tile from bounds on the device
    (void)rows;
    if (n <= 0 || total_rows <= 0) return ok();
    if (type != 8 && type != 12 && type != 14 && type != 23)
        return fail(XS_EINVAL, "iq_mmq_grouped: ggml type %d (this build's products: Q8_0, Q4_K, Q6_K, IQ4_XS)",
                    type);
    const int64_t out_tile = type == 14 ? 128 : 256;   // output columns a work-group: 128, or 256 (two rows a lane)
    if (w_cols <= 0 || w_cols % (type == 8 ? 64 : 256) || w_rows <= 0 || w_rows % out_tile || n > 65535 ||
        ld_dst < w_rows || ld_dst % 4 || total_rows > INT32_MAX / 2)
        return fail(XS_EINVAL,
                    "iq_mmq_grouped: %lld x %lld weights (columns a multiple of %d, rows of %lld), %d experts, "
                    "%lld floats a dst row",
                    (long long)w_rows, (long long)w_cols, type == 8 ? 64 : 256, (long long)out_tile, n,
                    (long long)ld_dst);
    if (!(wtab ? aligned(wtab, 8) : (w && aligned(w, 16) && expert_bytes % 16 == 0)) || !aligned(xq, 16) ||
        !aligned(bounds, 4) || !aligned(ids, 4) || !aligned(dst, 16))
        return fail(XS_EINVAL, "iq_mmq_grouped: a span is missing or misaligned");
    // one launch and no scratch (the reference's contract: no allocation or sync): the GEMM reads the int8 rows and
    // their scales itself, and takes each group's weights and tile from w / wtab and bounds
    xs::ExpertLayout L;
    L.gu_type = L.d_type = type;
    L.n_embd = w_rows;
    L.n_ff = w_cols;
    L.gu_row = L.d_row = L.up_row = (int64_t)xs_iq_row_bytes(type, w_cols);
    L.up_type = type;
    L.up_off = L.down_off = 0;
    L.bytes = (int64_t)expert_bytes;
    xs::PrefillArgs a{};
    a.bounds = bounds;
    a.entry = ids;
    a.parts = dst;
    a.parts_h = nullptr;
    a.n_tok = total_rows;
    a.rows = total_rows;
    a.cap_groups = n;
    a.ld_parts = ld_dst;
    a.xq = (const int8_t*)xq;
    a.wbase = (const uint8_t*)w;
    a.wstride = expert_bytes;
    a.wtab = wtab;
    a.woff = woff;
    return finish(stream, xs::launch_mmq_product(L, a, S(stream)), "iq_mmq_grouped");
}

int xs_moe_prefill_experts(const xs_expert_layout_t* L, const float* x, int64_t n_tok, const int32_t* src,
                           const int32_t* entry_of, const int32_t* bounds, const int32_t* n_groups,
                           const unsigned long long* grp_ptr, int64_t cap_groups, int64_t rows, void* scratch,
                           float* parts, void* stream) {
    return prefill_experts(L, x, n_tok, src, entry_of, bounds, n_groups, grp_ptr, cap_groups, rows, scratch, parts,
                           nullptr, false, stream);
}

int xs_native_moe_combine_multi(const float* parts, const float* weights, const float* shared, float* output,
                                int64_t n_embd, int64_t k, int n_tok, void* stream, const float* shared_gate) {
    if (n_embd <= 0 || k < 1 || k > 15 || n_tok < 1 || (shared_gate && !shared))
        return fail(XS_EINVAL, "native MoE combine (multi) requires a width, 1..15 experts, tokens");
    if (!aligned(parts, 4) || !aligned(weights, 4) || !aligned(output, 4) || (shared && !aligned(shared, 4)))
        return fail(XS_EINVAL, "native MoE combine requires aligned spans");
    const size_t ob = (size_t)n_tok * n_embd * 4;
    if (overlap(output, ob, parts, ob * k) || overlap(output, ob, weights, (size_t)n_tok * k * 4) ||
        overlap(output, ob, shared, ob))
        return fail(XS_EINVAL, "native MoE combine requires disjoint output");
    return finish(stream, xs::launch_combine(parts, weights, shared, shared_gate, nullptr, output, n_embd, (int)k, n_tok,
                                             S(stream)),
                  "native_moe_combine_multi");
}

int xs_native_moe_combine(const float* parts, const float* weights, const float* shared, float* output,
                          int64_t n_embd, int64_t k, void* stream) {
    if (n_embd <= 0 || n_embd > 0x7fffffff || k < 1 || k > 15)
        return fail(XS_EINVAL, "native MoE combine requires a positive width and 1..15 experts");
    return xs_native_moe_combine_multi(parts, weights, shared, output, n_embd, k, 1, stream, nullptr);
}

int xs_native_moe_combine_multi_hits(const float* parts, const float* hits, const int32_t* dst, const int32_t* count,
                                     const float* weights, const float* shared, float* output, int64_t n_embd,
                                     int64_t k, int n_tok, void* stream, const float* shared_gate) {
    if (n_tok <= 0) return ok();
    if (n_embd <= 0 || k < 1 || k > 15 || (shared_gate && !shared) || !hits || !dst || !count)
        return fail(XS_EINVAL, "native MoE combine (hits) requires a width, 1..15 experts, tokens, hits (k %lld)",
                    (long long)k);
    if (!aligned(parts, 4) || !aligned(hits, 4) || !aligned(weights, 4) || !aligned(output, 4) || !aligned(dst, 4) ||
        !aligned(count, 4))
        return fail(XS_EINVAL, "native MoE combine (hits): a span is missing or misaligned");
    const size_t pb = (size_t)n_tok * (size_t)k * (size_t)n_embd * 4, ob = (size_t)n_tok * (size_t)n_embd * 4;
    if (overlap(output, ob, parts, pb) || overlap(output, ob, hits, pb) || (shared && overlap(output, ob, shared, ob)))
        return fail(XS_EINVAL, "native MoE combine (hits): the output overlaps an input");
    return finish(stream, xs::launch_combine_hits(parts, hits, dst, count, weights, shared, shared_gate, output, n_embd,
                                                  (int)k, n_tok, S(stream)),
                  "native_moe_combine_multi_hits");
}

int xs_moe_combine_residual(const float* parts, const float* weights, const float* shared, const float* shared_gate,
                            const float* residual, float* output, int64_t n_embd, int64_t k, int n_tok, void* stream) {
    if (n_embd <= 0 || k < 1 || k > 64 || n_tok < 1 || (shared_gate && !shared))
        return fail(XS_EINVAL, "moe_combine_residual requires a width, 1..64 experts, tokens");
    if (!aligned(parts, 4) || !aligned(weights, 4) || !aligned(output, 4) || !aligned(residual, 4))
        return fail(XS_EINVAL, "moe_combine_residual requires aligned spans");
    const size_t ob = (size_t)n_tok * n_embd * 4;
    if (overlap(output, ob, parts, ob * k)) return fail(XS_EINVAL, "moe_combine_residual: output overlaps parts");
    if (residual != output && overlap(output, ob, residual, ob))
        return fail(XS_EINVAL, "moe_combine_residual: output partly overlaps the residual");
    return finish(stream, xs::launch_combine(parts, weights, shared, shared_gate, residual, output, n_embd, (int)k, n_tok,
                                             S(stream)),
                  "moe_combine_residual");
}

int xs_add_inplace(float* x, const float* y, int64_t n, void* stream) {
    if (n <= 0) return ok();
    if (!aligned(x, 4) || !aligned(y, 4)) return fail(XS_EINVAL, "add_inplace: a span is missing or misaligned");
    return finish(stream, xs::launch_add_inplace(x, y, n, S(stream)), "add_inplace");
}

// ---------------------------------------------------------------- a shared expert (decode)

namespace {
struct SharedWs {
    void* xq;
    unsigned long long* grp_ptr;
    int32_t *start, *n_groups, *idx;
    void* scratch;
    size_t bytes;
};
SharedWs shared_ws(const xs_expert_layout_t* SL, int n_tok, uint8_t* base) {
    SharedWs d;
    size_t off = 0;
    auto take = [&](size_t b) { uint8_t* p = base ? base + off : nullptr; off += up256(b); return p; };
    d.xq = take((size_t)n_tok * (size_t)(SL->n_embd / 32) * 36);
    d.grp_ptr = (unsigned long long*)take(8);
    d.start = (int32_t*)take(8);
    d.n_groups = (int32_t*)take(4);
    d.idx = (int32_t*)take((size_t)n_tok * 4);
    d.scratch = take(xs_native_expert_scratch_bytes(n_tok, SL->n_ff));
    d.bytes = off;
    return d;
}
}  // namespace

size_t xs_shared_expert_decode_workspace_bytes(const xs_expert_layout_t* SL, int n_tok) {
    if (!SL || n_tok <= 0) return 0;
    return shared_ws(SL, n_tok, nullptr).bytes;
}

int xs_shared_expert_decode(const xs_expert_layout_t* SL, const uint8_t* blob, const float* x, int n_tok,
                            const float* w_gate, float* shared, float* gate_logit, void* workspace,
                            size_t workspace_bytes, void* stream) {
    if (n_tok <= 0) return ok();
    if (int r = check_layout(SL, "shared_expert_decode")) return r;
    if (n_tok > 1024) return fail(XS_EINVAL, "shared_expert_decode: %d tokens is past 1024", n_tok);
    if (!aligned(blob, 16) || !aligned(x, 4) || !aligned(shared, 4))
        return fail(XS_EINVAL, "shared_expert_decode: the blob (16-byte aligned), x or shared is missing or misaligned");
    if ((w_gate == nullptr) != (gate_logit == nullptr))
        return fail(XS_EINVAL, "shared_expert_decode: w_gate and gate_logit go together");
    if (!aligned(workspace, 256) || workspace_bytes < xs_shared_expert_decode_workspace_bytes(SL, n_tok))
        return fail(XS_EINVAL, "shared_expert_decode: workspace missing, misaligned or short");
    const SharedWs w = shared_ws(SL, n_tok, (uint8_t*)workspace);
    if (int r = xs_quantize_q8_1_rows(x, n_tok, SL->n_embd, w.xq, stream)) return r;
    if (int r = finish(stream, xs::launch_single_group_plan(w.grp_ptr, w.start, w.n_groups, w.idx, n_tok, blob,
                                                            S(stream)),
                       "shared_expert_decode"))
        return r;
    if (int r = grouped_impl(SL, w.grp_ptr, w.start, w.n_groups, w.idx, w.idx, 1, n_tok, w.xq, w.scratch, shared,
                             stream, 0, n_tok))
        return r;
    if (w_gate) return xs_router_logits_f32(x, w_gate, gate_logit, n_tok, SL->n_embd, 1, stream);
    return ok();
}

// ---------------------------------------------------------------- whole layers

namespace {
struct DecodeWs {
    int32_t* status;   // the error word, first in the workspace
    int32_t* sync;     // the persistent layer's call counters (same 4 KB head, from byte 128)
    uint32_t* marks;   // the persistent layer's unit marks (kMarkWords words after the tagged hand-over words)
    unsigned long long *hx, *px;   // the persistent layer's tagged hand-over words (256 entries)
    int32_t* ids;
    float* w;
    int32_t* plan;
    uint32_t* skip;
    void* xq;
    void* scratch;
    float* parts;
    size_t bytes;
};
// The persistent layer's part of the workspace (head, tagged words) sits at fixed offsets whatever the call's token
// count, ahead of everything else, so one workspace zeroed once serves calls of any size up to the one it was sized
// for and the chained path never writes over tagged words.
bool fused_possible(const xs_expert_layout_t* L, int n_expert, int k) {
    xs::FusedPlan P;
    return xs::fused_decode_plan(to_layout(L), n_expert, k, 1, &P);
}
// fixed_tagged: the tagged words take the regions of the largest layout (xs::kScratchMaxFF, xs::kScratchMaxEmbd) at
// the same offsets for every layout, so that a workspace shared by calls of different layouts (the library's own
// scratch) has nothing but tagged words in those regions
DecodeWs decode_ws(const xs_expert_layout_t* L, int n_expert, int k, int n_tok, uint8_t* base,
                   bool fixed_tagged = false) {
    DecodeWs d;
    const long long capx = (long long)n_tok * k;
    size_t off = 0;
    auto take = [&](size_t b) { uint8_t* p = base ? base + off : nullptr; off += up256(b); return p; };
    d.status = (int32_t*)take(4096);
    d.sync = d.status ? d.status + 32 : nullptr;
    const bool fused = fixed_tagged || fused_possible(L, n_expert, k);
    const int64_t hx_ff = fixed_tagged ? xs::kScratchMaxFF : L->n_ff;
    const int64_t px_embd = fixed_tagged ? xs::kScratchMaxEmbd : L->n_embd;
    d.hx = (unsigned long long*)take(fused ? (size_t)256 * (size_t)hx_ff * 8 : 0);
    d.px = (unsigned long long*)take(fused ? (size_t)256 * (size_t)px_embd * 8 : 0);
    // (after the tagged words, not in the head: the h words' offsets decide which memory channels the polls meet)
    d.marks = (uint32_t*)take(fused ? (size_t)xs::kMarkWords * 4 : 0);
    d.ids = (int32_t*)take((size_t)capx * 4);
    d.w = (float*)take((size_t)capx * 4);
    d.plan = (int32_t*)take(plan_words(capx) * 4);
    d.skip = (uint32_t*)take(4);
    d.xq = take((size_t)n_tok * (size_t)(L->n_embd / 32) * 36);
    d.scratch = take(xs_native_expert_scratch_bytes(capx, L->n_ff));
    d.parts = (float*)take((size_t)capx * (size_t)L->n_embd * 4);
    d.bytes = off;
    return d;
}
struct PrefillWs {
    int32_t* status;   // the workspace's first word (xs_moe_layer_prefill_status)
    int32_t* ids;
    float* w;
    int32_t *src, *slot, *entry, *bounds, *experts, *n_groups;
    unsigned long long* grp_ptr;
    void* scratch;
    uint16_t* parts;   // f16
    int32_t* ghist;    // the split permutation's block histograms
    size_t bytes;
};
PrefillWs prefill_ws(const xs_expert_layout_t* L, int n_expert, int k, int n_tok, uint8_t* base) {
    PrefillWs d;
    const size_t n = (size_t)n_tok * k;
    size_t off = 0;
    auto take = [&](size_t b) { uint8_t* p = base ? base + off : nullptr; off += up256(b); return p; };
    d.status = (int32_t*)take(4);
    d.ids = (int32_t*)take(n * 4);
    d.w = (float*)take(n * 4);
    d.src = (int32_t*)take(n * 4);
    d.slot = (int32_t*)take(n * 4);
    d.entry = (int32_t*)take(n * 4);
    d.bounds = (int32_t*)take((size_t)(n_expert + 1) * 4);
    d.experts = (int32_t*)take((size_t)n_expert * 4);
    d.n_groups = (int32_t*)take(4);
    d.grp_ptr = (unsigned long long*)take((size_t)n_expert * 8);
    d.scratch = take(xs_moe_prefill_scratch_bytes(n_tok, (int64_t)n, L->n_embd, L->n_ff));
    d.parts = (uint16_t*)take(n * (size_t)L->n_embd * 2);
    d.ghist = (int32_t*)take(xs::prefill_route_split_scratch((int64_t)n, n_expert));
    d.bytes = off;
    return d;
}
}  // namespace

int32_t* xs_moe_layer_decode_status(void* workspace) {
    return workspace ? (int32_t*)workspace : nullptr;
}

int32_t* xs_moe_layer_prefill_status(void* workspace) {
    return workspace ? (int32_t*)workspace : nullptr;
}

int32_t* xs_moe_prefill_status(void* scratch, int64_t n_tok, int64_t rows, int64_t n_embd, int64_t n_ff) {
    if (!scratch) return nullptr;
    return (int32_t*)((uint8_t*)scratch + xs_moe_prefill_scratch_bytes(n_tok, rows, n_embd, n_ff) - 256);
}

void xs_moe_set_wait_bound(long long ticks) { g_wait_bound.store(ticks, std::memory_order_relaxed); }

void xs_moe_set_prefill_tall(int on) { g_tall.store(on == 2 ? 2 : on ? 1 : 0, std::memory_order_relaxed); }

int xs_moe_status_check(int32_t* status, void* stream) {
    if (!aligned(status, 4)) return fail(XS_EINVAL, "moe status check: the status word is missing or misaligned");
    hipStream_t s = S(stream);
    int32_t word = 0;
    hipError_t e = hipMemcpyAsync(&word, status, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(XS_EDEVICE, "moe status check: %s", hipGetErrorString(e));
    if (word == 0) return ok();
    const int32_t zero = 0;
    e = hipMemcpyAsync(status, &zero, 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(XS_EDEVICE, "moe status check: %s", hipGetErrorString(e));
    return fail(XS_EDEVICE, "moe layer: status 0x%x:%s%s%s%s", (unsigned)word,
                (word & 2) ? " a bounded wait of the persistent layer expired (its work-groups were not all resident)"
                           : "",
                (word & 4) ? " a token's router produced fewer than k experts (NaN logits; no output written)" : "",
                (word & 8) ? " a prompt value passed the f16 range and was saturated at +-65504 (an activation, h or"
                             " a part: the affected rows are not the fp32 result)"
                           : "",
                (word & ~14) ? " a blob was misaligned" : "");
}

size_t xs_moe_layer_decode_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok) {
    if (!L || k <= 0 || n_tok <= 0 || n_expert <= 0) return 0;
    return decode_ws(L, n_expert, k, n_tok, nullptr).bytes;
}

namespace {
// How a layer routes its tokens: the softmax top-k of the logits (router_top10), or DeepSeek-V3's group-limited
// sigmoid (xs_router_grouped_sigmoid's arguments)
struct Route {
    int kind = XS_ROUTER_SOFTMAX;
    const float* bias = nullptr;
    int n_group = 1, topk_group = 1;
    float scale = 1.0f;
};
int route_of(const xs_router_cfg_t* cfg, int n_expert, int k, Route* r, const char* who) {
    *r = Route{};
    if (!cfg || cfg->kind == XS_ROUTER_SOFTMAX) return XS_OK;
    if (cfg->kind != XS_ROUTER_GROUPED_SIGMOID) return fail(XS_EINVAL, "%s: router kind %d is unknown", who, cfg->kind);
    if (cfg->n_group <= 0 || cfg->n_group > 64 || n_expert % cfg->n_group || cfg->topk_group <= 0 ||
        cfg->topk_group > cfg->n_group || k > (n_expert / cfg->n_group) * cfg->topk_group ||
        (cfg->bias && !aligned(cfg->bias, 4)))
        return fail(XS_EINVAL, "%s: grouped sigmoid router: %d experts, %d groups, top %d groups, k %d", who, n_expert,
                    cfg->n_group, cfg->topk_group, k);
    r->kind = cfg->kind;
    r->bias = cfg->bias;
    r->n_group = cfg->n_group;
    r->topk_group = cfg->topk_group;
    r->scale = cfg->routed_scale;
    return XS_OK;
}

// status: where the persistent layer's error bits go (NULL: the workspace's status word); fixed_tagged: decode_ws's
// the grouped sigmoid router's wave form (xs_route.h route_grouped_sigmoid_wave): the groups on whole lanes, lanes a
// group a power of two (launch_router_grouped_sigmoid's condition)
bool sigmoid_wave_form(int n_expert, int n_group) {
    const int PER = n_expert <= 64 ? 1 : n_expert <= 128 ? 2 : n_expert <= 256 ? 4 : n_expert <= 512 ? 8 : 16;
    const int per = n_group > 0 ? n_expert / n_group : 0;
    const int lpg = per % PER == 0 ? per / PER : 0;
    return n_expert <= 1024 && n_group > 0 && per * n_group == n_expert && lpg > 0 && (lpg & (lpg - 1)) == 0;
}

int layer_decode(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                 const float* x, const float* logits, const float* residual, float* out, int n_tok, void* workspace,
                 size_t workspace_bytes, const float* shared, const float* shared_gate, void* stream,
                 int32_t* status = nullptr, bool fixed_tagged = false, const Route& route = Route{}) {
    if (n_tok <= 0) return ok();
    if (int r = check_layout(L, "moe_layer_decode")) return r;
    if (n_tok * k > 1024) return fail(XS_EINVAL, "moe_layer_decode: %d tokens x top-%d is past 1024 entries", n_tok, k);
    if (blob_bytes < L->bytes || blob_bytes % 16 || !aligned(arena, 16))
        return fail(XS_EINVAL, "moe_layer_decode: the arena must hold 16-byte aligned blobs of at least %zu bytes", L->bytes);
    const size_t need = fixed_tagged ? decode_ws(L, n_expert, k, n_tok, nullptr, true).bytes
                                     : xs_moe_layer_decode_workspace_bytes(L, n_expert, k, n_tok);
    if (!aligned(workspace, 256) || workspace_bytes < need)
        return fail(XS_EINVAL, "moe_layer_decode: workspace missing, misaligned or short");
    if (status && !aligned(status, 4)) return fail(XS_EINVAL, "moe_layer_decode: the status word is misaligned");
    const DecodeWs w = decode_ws(L, n_expert, k, n_tok, (uint8_t*)workspace, fixed_tagged);
    const long long capx = (long long)n_tok * k;
    if (n_expert > 1024 || k > 64 || k > n_expert)
        return fail(XS_EINVAL, "moe_layer_decode: %d experts, top-%d (the router takes up to 1024 and 64)", n_expert, k);
    if (!aligned(logits, 4) || !aligned(x, 4) || !aligned(residual, 4) || !aligned(out, 4))
        return fail(XS_EINVAL, "moe_layer_decode: a span is missing or misaligned");
    const xs::ExpertLayout XL = to_layout(L);
    const bool pre = route.kind == XS_ROUTER_GROUPED_SIGMOID;
    xs::FusedPlan P;
    // 2..16 tokens of a wide layer (hidden >= 4096): the chained path on the weight-stream kernels, measured faster
    // there than the persistent layer (config 4 at 8 tokens: 565 -> ~250 us); narrower layers keep the persistent one
    const bool streamed = n_tok >= 2 && L->n_embd >= 4096 &&
                          xs::stream_usable(XL, n_tok, capx < n_expert ? capx : n_expert, capx);
    const bool fused = !streamed && xs::fused_decode_plan(XL, n_expert, k, n_tok, &P);
    // the grouped sigmoid router inside the persistent layer's routing stage where its groups fall on whole lanes
    // (the wave form) and the layout's instances carry it (the Q4_K pair): one launch less (config 5 T=1: 109.5 ->
    // 105.6 us); otherwise its own launch first, into the workspace's ids and weights
    const bool sig_in = pre && fused && sigmoid_wave_form(n_expert, route.n_group) &&
                        xs::fused_sigmoid_layout(L->gu_type, L->d_type);
    if (pre && !sig_in)
        if (int r = xs_router_grouped_sigmoid(logits, route.bias, n_tok, n_expert, route.n_group, route.topk_group, k,
                                              route.scale, w.ids, w.w, stream))
            return r;
    if (fused) {
        // the whole layer in one persistent launch
        xs::FusedArgs a;
        a.L = XL;
        a.arena = arena;
        a.blob = (long long)blob_bytes;
        a.n_expert = n_expert;
        a.k = k;
        a.n_tok = n_tok;
        a.logits = logits;
        a.x = x;
        a.residual = residual;
        a.out = out;
        a.ids = w.ids;
        a.weights = w.w;
        a.hx = w.hx;
        a.px = w.px;
        a.sync = w.sync;
        a.marks = w.marks;
        a.err = status ? status : w.status;
        a.rh = P.rh;
        a.rd = P.rd;
        a.nu = P.nu;
        a.nj = P.nj;
        a.slab_gu_bytes = P.slab_gu;
        a.slab_dn_bytes = P.slab_dn;
        a.ttab = P.ttab;
        a.direct = P.direct;
        a.slab_alias = P.alias;
        a.spin_ticks = spin_ticks();
        a.help_ticks = help_all() ? -1 : a.spin_ticks / 10000;   // 5 us of the 50 ms bound
        a.shared = shared;
        a.shared_gate = shared_gate;
        a.pre_ids = pre && !sig_in ? w.ids : nullptr;
        a.pre_w = pre && !sig_in ? w.w : nullptr;
        if (sig_in) {
            a.sig_bias = route.bias;
            a.sig_group = route.n_group;
            a.sig_topk_group = route.topk_group;
            a.sig_scale = route.scale;
        }
        if (n_tok == 1) {   // the one-token kernel where the layout fits it
            bool used = false;
            const hipError_t e1 = xs::launch_decode_t1(a, S(stream), &used);
            if (used || e1 != hipSuccess) return finish(stream, e1, "moe_layer_decode");
        }
        return finish(stream, xs::launch_decode_fused(a, P, S(stream)), "moe_layer_decode");
    }
    if (pre) {   // the plan of the given ids, then the activations
        if (int r = xs_resident_plan(w.ids, (int)capx, k, nullptr, n_expert, arena, nullptr, (long long)blob_bytes,
                                     w.plan, capx, w.skip, 1u, stream))
            return r;
        if (int r = xs_quantize_q8_1_rows(x, n_tok, L->n_embd, w.xq, stream)) return r;
    } else {
        // routing, plan and activations in one launch (the reference's router_top10 + resident_plan +
        // quantize_q8_1_rows)
        hipError_t e = xs::launch_decode_route(logits, x, n_tok, n_expert, k, L->n_embd, w.ids, w.w, w.plan, capx,
                                               w.skip, arena, (long long)blob_bytes, w.xq, S(stream));
        if (e != hipSuccess) return hip_status(e, "moe_layer_decode");
    }
    const int64_t cap_groups = capx < n_expert ? capx : n_expert;
    long long o_start, o_dst, o_tok, o_ptr;
    xs_plan_offsets(capx, &o_start, &o_dst, &o_tok, &o_ptr, nullptr);
    if (int r = grouped_impl(L, (const unsigned long long*)(w.plan + o_ptr), w.plan + o_start, w.plan, w.plan + o_dst,
                             w.plan + o_tok, cap_groups, capx, w.xq, w.scratch, w.parts, stream, 0, n_tok))
        return r;
    return xs_moe_combine_residual(w.parts, w.w, shared, shared_gate, residual, out, L->n_embd, k, n_tok, stream);
}
}  // namespace

int xs_moe_layer_decode(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                        const float* x, const float* logits, const float* residual, float* out, int n_tok,
                        void* workspace, size_t workspace_bytes, void* stream) {
    return layer_decode(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, workspace, workspace_bytes,
                        nullptr, nullptr, stream);
}

}  // extern "C"

namespace xs {
size_t layer_decode_fixed_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok) {
    if (!L || k <= 0 || n_tok <= 0 || n_expert <= 0) return 0;
    return decode_ws(L, n_expert, k, n_tok, nullptr, true).bytes;
}
int layer_decode_fixed(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                       const float* x, const float* logits, const float* residual, float* out, int n_tok,
                       void* scratch, size_t scratch_bytes, int32_t* status, void* stream) {
    return layer_decode(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, scratch, scratch_bytes,
                        nullptr, nullptr, stream, status, true);
}
}  // namespace xs

extern "C" {

size_t xs_moe_layer_decode_shared_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok,
                                                  const xs_expert_layout_t* SL) {
    if (!L || !SL || k <= 0 || n_tok <= 0 || n_expert <= 0) return 0;
    return decode_ws(L, n_expert, k, n_tok, nullptr).bytes + up256((size_t)n_tok * (size_t)L->n_embd * 4) +
           up256((size_t)n_tok * 4) + shared_ws(SL, n_tok, nullptr).bytes;
}

}  // extern "C"

namespace {
// the decode layer with an optional shared expert (SL NULL: none) and either router
int layer_decode_shared(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                        const float* x, const float* logits, const float* residual, float* out, int n_tok,
                        const Route& route, const xs_expert_layout_t* SL, const uint8_t* shared_blob,
                        const float* w_gate, void* workspace, size_t workspace_bytes, void* stream, const char* who) {
    if (n_tok <= 0) return ok();
    if (int r = check_layout(L, who)) return r;
    if (!SL)
        return layer_decode(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, workspace,
                            workspace_bytes, nullptr, nullptr, stream, nullptr, false, route);
    if (int r = check_layout(SL, who)) return r;
    if (SL->n_embd != L->n_embd)
        return fail(XS_EINVAL, "%s: the shared expert's n_embd %lld is not the layer's %lld", who,
                    (long long)SL->n_embd, (long long)L->n_embd);
    if (!aligned(workspace, 256) ||
        workspace_bytes < xs_moe_layer_decode_shared_workspace_bytes(L, n_expert, k, n_tok, SL))
        return fail(XS_EINVAL, "%s: workspace missing, misaligned or short", who);
    // the layer's own workspace first (its head and tagged words at the offsets xs_moe_layer_decode uses), then the
    // shared rows, the gate logits and the shared expert's workspace
    const size_t lw = decode_ws(L, n_expert, k, n_tok, nullptr).bytes;
    uint8_t* base = (uint8_t*)workspace;
    float* shared = (float*)(base + lw);
    float* gate = (float*)(base + lw + up256((size_t)n_tok * (size_t)L->n_embd * 4));
    uint8_t* sws = base + lw + up256((size_t)n_tok * (size_t)L->n_embd * 4) + up256((size_t)n_tok * 4);
    const size_t sbytes = shared_ws(SL, n_tok, nullptr).bytes;
    // up to 64 tokens: the shared expert as a one-expert layer in one persistent launch, in the layer's workspace
    // (its head and tagged words, used again by the routed layer after it) - routing given (expert 0, weight 1.0) and
    // no residual, so each row is the expert's own: fl(y x 1) = y, the canonical rows bit for bit.  That replaces
    // four launches (q8_1, plan, gate/up, down).  Otherwise, or where the persistent plan does not take the shared
    // layout or its h would not fit the layer's hand-over region, the shared expert's own chain.
    xs::FusedPlan SP;
    const xs::ExpertLayout SXL = to_layout(SL);
    if (n_tok <= xs::kOneExpertMaxTok && SL->n_ff <= L->n_ff && fused_possible(L, n_expert, k) &&
        xs::fused_decode_plan(SXL, 1, 1, n_tok, &SP) && aligned(shared_blob, 16)) {
        const DecodeWs w = decode_ws(L, n_expert, k, n_tok, base);
        const int32_t* one_ids = nullptr;
        const float* one_w = nullptr;
        if (hipError_t e = xs::one_expert_routing(&one_ids, &one_w)) return hip_status(e, who);
        xs::FusedArgs a;
        a.L = SXL;
        a.arena = shared_blob;
        a.blob = (long long)SL->bytes;
        a.n_expert = 1;
        a.k = 1;
        a.n_tok = n_tok;
        a.logits = nullptr;   // (routing given)
        a.x = x;
        a.residual = nullptr;
        a.out = shared;
        a.ids = w.ids;
        a.weights = w.w;
        a.hx = w.hx;
        a.px = w.px;
        a.sync = w.sync;
        a.marks = w.marks;
        a.err = w.status;
        a.rh = SP.rh;
        a.rd = SP.rd;
        a.nu = SP.nu;
        a.nj = SP.nj;
        a.slab_gu_bytes = SP.slab_gu;
        a.slab_dn_bytes = SP.slab_dn;
        a.ttab = SP.ttab;
        a.direct = SP.direct;
        a.slab_alias = SP.alias;
        a.spin_ticks = spin_ticks();
        a.help_ticks = help_all() ? -1 : a.spin_ticks / 10000;   // 5 us of the 50 ms bound
        a.shared = nullptr;
        a.shared_gate = nullptr;
        a.pre_ids = one_ids;
        a.pre_w = one_w;
        if (int r = finish(stream, xs::launch_decode_fused(a, SP, S(stream)), who)) return r;
        if (w_gate)
            if (int r = xs_router_logits_f32(x, w_gate, gate, n_tok, SL->n_embd, 1, stream)) return r;
    } else if (int r = xs_shared_expert_decode(SL, shared_blob, x, n_tok, w_gate, shared, w_gate ? gate : nullptr, sws,
                                               sbytes, stream)) {
        return r;
    }
    return layer_decode(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, workspace, lw, shared,
                        w_gate ? gate : nullptr, stream, nullptr, false, route);
}
}  // namespace

extern "C" {

int xs_moe_layer_decode_shared(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert,
                               int k, const float* x, const float* logits, const float* residual, float* out,
                               int n_tok, const xs_expert_layout_t* SL, const uint8_t* shared_blob,
                               const float* w_gate, void* workspace, size_t workspace_bytes, void* stream) {
    if (!SL) return fail(XS_EINVAL, "moe_layer_decode_shared: no shared expert");
    return layer_decode_shared(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, Route{}, SL,
                               shared_blob, w_gate, workspace, workspace_bytes, stream, "moe_layer_decode_shared");
}

size_t xs_moe_layer_decode_ex_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok,
                                              const xs_expert_layout_t* SL) {
    return SL ? xs_moe_layer_decode_shared_workspace_bytes(L, n_expert, k, n_tok, SL)
              : xs_moe_layer_decode_workspace_bytes(L, n_expert, k, n_tok);
}

int xs_moe_layer_decode_ex(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                           const float* x, const float* logits, const float* residual, float* out, int n_tok,
                           const xs_router_cfg_t* router, const xs_expert_layout_t* SL, const uint8_t* shared_blob,
                           const float* w_gate, void* workspace, size_t workspace_bytes, void* stream) {
    Route rt;
    if (int r = route_of(router, n_expert, k, &rt, "moe_layer_decode_ex")) return r;
    return layer_decode_shared(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, rt, SL, shared_blob,
                               w_gate, workspace, workspace_bytes, stream, "moe_layer_decode_ex");
}

size_t xs_moe_layer_prefill_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok) {
    if (!L || k <= 0 || n_tok <= 0 || n_expert <= 0) return 0;
    return prefill_ws(L, n_expert, k, n_tok, nullptr).bytes;
}

}  // extern "C"

namespace {
// the prompt layer's shared expert: its single group's plan, its scratch, its fp32 rows and gate logits
struct SharedPrefillWs {
    unsigned long long* grp_ptr;
    int32_t *start, *n_groups, *idx;
    void* scratch;
    float* rows;
    float* gate;
    size_t bytes;
};
SharedPrefillWs shared_prefill_ws(const xs_expert_layout_t* SL, int n_tok, uint8_t* base) {
    SharedPrefillWs d;
    size_t off = 0;
    auto take = [&](size_t b) { uint8_t* p = base ? base + off : nullptr; off += up256(b); return p; };
    d.grp_ptr = (unsigned long long*)take(8);
    d.start = (int32_t*)take(8);
    d.n_groups = (int32_t*)take(4);
    d.idx = (int32_t*)take((size_t)n_tok * 4);
    d.scratch = take(xs_moe_prefill_scratch_bytes(n_tok, n_tok, SL->n_embd, SL->n_ff));
    d.rows = (float*)take((size_t)n_tok * (size_t)SL->n_embd * 4);
    d.gate = (float*)take((size_t)n_tok * 4);
    d.bytes = off;
    return d;
}

int layer_prefill(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                  const float* x, const float* logits, const float* residual, float* out, int n_tok, const Route& route,
                  const xs_expert_layout_t* SL, const uint8_t* shared_blob, const float* w_gate, void* workspace,
                  size_t workspace_bytes, void* stream, const char* who) {
    if (n_tok <= 0) return ok();
    if (int r = check_layout(L, who)) return r;
    if (blob_bytes < L->bytes || blob_bytes % 16 || !aligned(arena, 16))
        return fail(XS_EINVAL, "%s: the arena must hold 16-byte aligned blobs of at least %zu bytes", who, L->bytes);
    if (SL) {
        if (int r = check_layout(SL, who)) return r;
        if (SL->n_embd != L->n_embd || !aligned(shared_blob, 16))
            return fail(XS_EINVAL, "%s: the shared expert (n_embd %lld, blob 16-byte aligned) does not fit the layer",
                        who, (long long)SL->n_embd);
    }
    if (!aligned(workspace, 256) || workspace_bytes < xs_moe_layer_prefill_ex_workspace_bytes(L, n_expert, k, n_tok, SL))
        return fail(XS_EINVAL, "%s: workspace missing, misaligned or short", who);
    const PrefillWs w = prefill_ws(L, n_expert, k, n_tok, (uint8_t*)workspace);
    const int64_t n = (int64_t)n_tok * k;
    // the shared expert first, on a side stream forked from the caller's (its own plan, f16 activations, GEMMs and
    // gate, in its own workspace): its one group of the prompt's rows leaves most of the GPU idle in its GEMMs, which
    // now run beside the routed experts' work; joined before the combine
    const float* shared = nullptr;
    const float* gate = nullptr;
    SideStream* side = nullptr;
    if (SL) {   // every token through the shared expert (one group), its rows in fp32; its gate's logits
        if (hipError_t e = side_stream_fork(S(stream), &side)) return hip_status(e, who);
        void* ss = (void*)side->stream;
        const SharedPrefillWs sw = shared_prefill_ws(SL, n_tok, (uint8_t*)workspace + w.bytes);
        if (int r = finish(ss, xs::launch_single_group_plan(sw.grp_ptr, sw.start, sw.n_groups, sw.idx, n_tok,
                                                            shared_blob, side->stream),
                           who))
            return r;
        if (int r = prefill_experts(SL, x, n_tok, sw.idx, sw.idx, sw.start, sw.n_groups, sw.grp_ptr, 1, n_tok,
                                    sw.scratch, sw.rows, nullptr, false, ss, nullptr, w.status))
            return r;
        if (w_gate) {
            // the prompt path's gate GEMM order (f32_gemm_rows) at every token count
            if (int r = xs_f32_gemm_rows(x, SL->n_embd, w_gate, sw.gate, 1, SL->n_embd, 1, n_tok, ss)) return r;
            gate = sw.gate;
        }
        shared = sw.rows;
        if (hipError_t e = hipEventRecord(side->join, side->stream)) return hip_status(e, who);
    }
    if (route.kind == XS_ROUTER_GROUPED_SIGMOID) {
        if (int r = xs_router_grouped_sigmoid(logits, route.bias, n_tok, n_expert, route.n_group, route.topk_group, k,
                                              route.scale, w.ids, w.w, stream))
            return r;
    } else if (int r = xs_router_top10(logits, n_tok, n_expert, k, w.ids, w.w, stream)) {
        return r;
    }
    const int64_t cap_groups = n < n_expert ? n : n_expert;
    // without a shared expert on the side stream, the whole 256-row tiles of the routed experts take the tall-tile
    // GEMMs and the other rows run beside them there
    SideStream* split = nullptr;
    SideStream serial{0, S(stream), nullptr, nullptr};   // both chains on the caller's stream
    const int tall = g_tall.load(std::memory_order_relaxed);
    if (!SL && tall && xs::tall_usable(to_layout(L)) && n >= 256) {
        if (tall == 2) split = &serial;
        else if (hipError_t e = side_stream_get(&split)) return hip_status(e, who);
    }
    // the permutation's launch also builds the GEMMs' f16 copy of x (at the scratch's start, prefill_experts' xb)
    const xs::ToF16 conv{x, (uint16_t*)w.scratch, (int64_t)n_tok * L->n_embd / 8, w.status};
    if (int r = finish(stream,
                       xs::launch_prefill_route_split(w.ids, n, k, n_expert, w.src, w.slot, w.entry, w.bounds,
                                                      w.experts, w.n_groups, arena, (long long)blob_bytes, w.grp_ptr,
                                                      w.ghist, prefill_mtile(w.scratch, n_tok, n, L), (int)cap_groups,
                                                      S(stream), split != nullptr, &conv),
                       who))
        return r;
    if (int r = prefill_experts(L, x, n_tok, w.src, w.entry, w.bounds, w.n_groups, w.grp_ptr, cap_groups, n, w.scratch,
                                nullptr, w.parts, true, stream, split, w.status, true))
        return r;
    if (side)   // the combine waits for the shared expert's rows
        if (hipError_t e = hipStreamWaitEvent(S(stream), side->join, 0)) return hip_status(e, who);
    return finish(stream,
                  xs::launch_combine_h(w.parts, w.w, shared, gate, residual, out, L->n_embd, k, n_tok, S(stream)), who);
}
}  // namespace

extern "C" {

int xs_moe_layer_prefill(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert,
                         int k, const float* x, const float* logits, const float* residual, float* out, int n_tok,
                         void* workspace, size_t workspace_bytes, void* stream) {
    return layer_prefill(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, Route{}, nullptr, nullptr,
                         nullptr, workspace, workspace_bytes, stream, "moe_layer_prefill");
}

size_t xs_moe_layer_prefill_ex_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok,
                                               const xs_expert_layout_t* SL) {
    if (!L || k <= 0 || n_tok <= 0 || n_expert <= 0) return 0;
    const size_t base = prefill_ws(L, n_expert, k, n_tok, nullptr).bytes;
    return SL ? base + shared_prefill_ws(SL, n_tok, nullptr).bytes : base;
}

int xs_moe_layer_prefill_ex(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                            const float* x, const float* logits, const float* residual, float* out, int n_tok,
                            const xs_router_cfg_t* router, const xs_expert_layout_t* SL, const uint8_t* shared_blob,
                            const float* w_gate, void* workspace, size_t workspace_bytes, void* stream) {
    Route rt;
    if (int r = route_of(router, n_expert, k, &rt, "moe_layer_prefill_ex")) return r;
    return layer_prefill(L, arena, blob_bytes, n_expert, k, x, logits, residual, out, n_tok, rt, SL, shared_blob,
                         w_gate, workspace, workspace_bytes, stream, "moe_layer_prefill_ex");
}

}  // extern "C"
