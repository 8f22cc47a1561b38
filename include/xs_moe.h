/*
 * include/xs_moe.h - the C ABI of the MI355X MoE-layer library (libxsmoe.so).
 *
 * The drop-in boundary for XeStrata's mixture-of-experts hot path.  Each entry point names the reference interface it
 * replaces (paths relative to the reference repository, 32x-k/XeStrata-win).  Conventions, as the reference's:
 *   - every buffer is device memory owned by the caller; no entry point allocates device memory or synchronises,
 *     except where a NULL stream is allowed and documented to synchronise (the reference's `sync_if_needed`);
 *   - `stream` is a hipStream_t passed as void* (the reference's opaque `void* stream`).  NULL is HIP's ordered default
 *     stream everywhere; the entry points the reference lets run on a null queue then also synchronise.  (The
 *     reference's native router, combine and plan reject a null SYCL queue; the C++ wrappers in
 *     xs_strata_kernels.hpp keep that rule for drop-in callers);
 *   - group and entry counts are read on the device, so one captured graph with capacity grids serves every routing;
 *   - blob addresses (expert weights) are 16-byte aligned; float spans 4-byte aligned; outputs do not overlap inputs.
 * Every function returns XS_OK (0) or an error code, with a message for the calling thread in xs_last_error().  The
 * C++ wrappers in xs_strata_kernels.hpp turn a non-zero code back into the reference's exceptions.
 *
 * ggml type ids: Q8_0 = 8, Q4_K = 12, Q6_K = 14, IQ4_XS = 23.
 */
#ifndef XS_MOE_H
#define XS_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XS_OK 0
#define XS_EINVAL 1 /* bad geometry, alignment, overlap or a missing stream: the reference's std::invalid_argument */
#define XS_EDEVICE 2 /* a HIP error: the reference's core::DeviceError */

/* The message of this thread's last failed call ("" if none). */
const char* xs_last_error(void);
/* ABI version (this header's). */
int xs_abi_version(void);

/* One native expert blob: [gate rows | up rows | down rows], raw GGUF blocks.
 * Mirrors NativeExpertLayout (include/strata/kernels/iq_kernels.hpp:66-75). */
typedef struct xs_expert_layout {
    int gu_type, d_type, up_type;
    int64_t n_embd, n_ff;
    size_t gu_row, d_row, up_row;
    size_t up_off, down_off, bytes;
} xs_expert_layout_t;

/* Bytes of one row of n values of `type` (0 when unsupported). Replaces iq_row_bytes (iq_kernels.hpp:22). */
size_t xs_iq_row_bytes(int type, int64_t n);

/* 1 when the grouped expert kernels take this gate/up and down type pair at these dimensions, else 0.
 * Replaces native_expert_supported (include/strata/kernels/iq_kernels.hpp:79). up_type -1: the gate's; another of the
 * four types: a mixed layer, gate and up rows each of its own type (iq_kernels.cpp:2003-2005). */
int xs_native_expert_supported(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, int up_type);

/* Replaces native_expert_layout (iq_kernels.hpp:81). */
int xs_native_expert_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, int up_type,
                            xs_expert_layout_t* out);

/* Scratch bytes xs_native_expert_grouped needs for cap_entries entries. Replaces native_expert_scratch_bytes
 * (iq_kernels.hpp:83): the reference's gate | up | h | hq areas, plus one 256-byte status word area at the end. */
size_t xs_native_expert_scratch_bytes(int64_t cap_entries, int64_t n_ff);

/* q8_1 blocks of n_rows rows of n_cols floats (n_cols a multiple of 32), canonical scale: one a 256 values when
 * n_cols % 256 == 0, else one a 32.  Replaces quantize_q8_1_rows (iq_kernels.hpp:26; iq_kernels.cpp:1850-1879).
 * A NULL stream runs on the default stream and synchronises. */
int xs_quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, void* y, void* stream);

/* Grouped experts in the native format (decode and verify windows).  Group g's blob is at device address
 * grp_ptr[g]; its entries [grp_start[g], grp_start[g+1]) read token ent_tok[e]'s q8_1 row (n_embd/32 blocks a token
 * in x_q8_1) and write row ent_dst[e] of `out` (n_embd floats).  Counts are read on the device; grid_groups (0:
 * cap_groups) rows of work-groups stride over the groups.  Replaces native_expert_grouped
 * (include/strata/kernels/iq_kernels.hpp:90-93; src/kernels/xe/iq_kernels.cpp:2042-2178).  A NULL stream runs on
 * the default stream and synchronises.  A blob address that is not 16-byte aligned is skipped and flagged in the
 * scratch status word (xs_native_expert_status). */
int xs_native_expert_grouped(const xs_expert_layout_t* L, const unsigned long long* grp_ptr,
                             const int32_t* grp_start, const int32_t* n_groups, const int32_t* ent_dst,
                             const int32_t* ent_tok, int64_t cap_groups, int64_t cap_entries, const void* x_q8_1,
                             void* scratch, float* out, void* stream, int64_t grid_groups);
/* The two halves of xs_native_expert_grouped, for callers that schedule them apart (and for timing each): the gate and
 * up rows into scratch (the reference's launch_native_gu, src/kernels/xe/iq_kernels.cpp:997-1031), then SwiGLU +
 * q8_1 of them and the down rows into `out` (its SwiGLU pass :2118-2133 and launch_native_down :1033-1063).  The same
 * scratch and cap_entries must be passed to both. */
int xs_native_expert_gate_up(const xs_expert_layout_t* L, const unsigned long long* grp_ptr, const int32_t* grp_start,
                             const int32_t* n_groups, const int32_t* ent_tok, int64_t cap_groups, int64_t cap_entries,
                             const void* x_q8_1, void* scratch, void* stream, int64_t grid_groups);
int xs_native_expert_down(const xs_expert_layout_t* L, const unsigned long long* grp_ptr, const int32_t* grp_start,
                          const int32_t* n_groups, const int32_t* ent_dst, int64_t cap_groups, int64_t cap_entries,
                          void* scratch, float* out, void* stream, int64_t grid_groups);
/* Device address of the status word inside a scratch of xs_native_expert_scratch_bytes(cap_entries, n_ff) bytes
 * (int32; non-zero once a call met a misaligned blob; the caller clears it). No reference counterpart. */
int32_t* xs_native_expert_status(void* scratch, int64_t cap_entries, int64_t n_ff);

/* Dequantize n values (a whole number of blocks) to fp32: the reference host dequantizers' values bit for bit
 * (include/strata/artifact/dequant.hpp).  Replaces iq_dequant_f32 (iq_kernels.hpp:30). */
int xs_iq_dequant_f32(int type, const void* src, int64_t n, float* dst, void* stream);
/* The same values rounded to bf16 (nearest even): the prompt path's dequantizer.  Replaces dequant_f16 /
 * iq_dequant_f16 (include/strata/kernels/dequant_bf16.hpp:23-25, iq_kernels.hpp:29), which produce FP16. */
int xs_iq_dequant_bf16(int type, const void* src, int64_t n, uint16_t* dst, void* stream);
/* The same values rounded to FP16 (nearest even; IEEE half bits): the reference's iq_dequant_f16
 * (include/strata/kernels/iq_kernels.hpp:29, the FP16 prompt fallback's weights). */
int xs_iq_dequant_f16(int type, const void* src, int64_t n, uint16_t* dst, void* stream);

/* The int8 activations of the reference's MMQ products (include/strata/kernels/iq_mmq.hpp:33-50;
 * src/kernels/xe/iq_mmq.cpp:1264-1341), byte for byte: rows of `cols` values (a multiple of 32; 2 cols when `dup`,
 * every block twice) as int8 q[rows][oc] | float d[rows][oc/32] | float d*sum(q)[rows][oc/32] (the sums written only
 * when `sums`).  d = amax / 127, q = round-half-away(v / d).  xs_iq_mmq_act_bytes replaces iq_mmq_act_bytes;
 * xs_iq_mmq_type_sums / _dup replace iq_mmq_type_sums / iq_mmq_type_dup (iq_mmq.hpp:33-38). */
size_t xs_iq_mmq_act_bytes(int64_t rows, int64_t cols);
int xs_iq_mmq_type_sums(int type);
int xs_iq_mmq_type_dup(int type);
/* Row i of xq from row ids[i] of x (row i when ids is NULL), ld floats a row of x.  Replaces iq_mmq_quantize
 * (iq_mmq.hpp:39-41) and prefill::mmq::quantize (include/strata/prefill/moe_mmq.hpp:46-49). */
int xs_iq_mmq_quantize(const float* x, const int32_t* ids, void* xq, int64_t cols, int64_t ld, int64_t rows, int sums,
                       int dup, void* stream);
/* Token t's row quantized once, stored at rows slot[t * k_used + j] of xq (tokens * k_used rows).  Replaces
 * iq_mmq_quantize_scatter (iq_mmq.hpp:42-47) and prefill::mmq::quantize_scatter (moe_mmq.hpp:50-55). */
int xs_iq_mmq_quantize_scatter(const float* x, const int32_t* slot, void* xq, int64_t cols, int64_t ld,
                               int64_t tokens, int k_used, int sums, int dup, void* stream);
/* n experts in one launch: expert e's weights ([w_rows, w_cols] in ggml `type`'s blocks) at w + e * expert_bytes (or
 * at wtab[e] + woff when wtab, a device table, is given), times its activation rows bounds[e] .. bounds[e + 1] of xq
 * (xs_iq_mmq_quantize's layout, total_rows rows; bounds on the device), into dst rows ids[row], ld_dst floats apart.
 * Replaces iq_mmq_grouped (include/strata/kernels/iq_mmq.hpp:49-58) and prefill::mmq::Context::run
 * (include/strata/prefill/moe_mmq.hpp:57-75).  The products run on the f16 MFMA path of xs_moe_prefill_experts: the
 * int8 activations are taken as q * d rounded to f16, the weights dequantized to f16, fp32 accumulation (within 2e-2
 * of the fp32 product, the reference's int8 path within its own int8 rounding).  Types: Q8_0 (8), Q4_K (12), Q6_K
 * (14), IQ4_XS (23); w_cols a multiple of 256 (64 for Q8_0), w_rows of 256 (128 for Q6_K).  max_rows and rows are
 * not needed (every work-group finds its tile from bounds on the device; the grid covers all total_rows rows).  One
 * launch; no allocation, no scratch and no synchronisation (the reference's contract, native_moe.hpp:18): the GEMM
 * turns the int8 rows to f16 as it stages them, and reads each expert's weights through w or wtab itself.  Calls on
 * different streams share nothing. */
int xs_iq_mmq_grouped(int type, const void* w, size_t expert_bytes, int64_t w_rows, int64_t w_cols, int n,
                      const void* xq, int64_t total_rows, const int32_t* bounds, int64_t max_rows, const int32_t* ids,
                      float* dst, int64_t ld_dst, const uint8_t* const* wtab, size_t woff, int64_t rows, void* stream);
/* h[r, j] = g / (1 + exp(-g)) * u over rows of 2 n_ff floats (gate, up interleaved 2j / 2j+1, or split j / n_ff+j).
 * Replaces prefill::mmq::swiglu (moe_mmq.hpp:106-108; src/prefill/moe_mmq.cpp:128-136). */
int xs_mmq_swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, int interleaved, void* stream);
/* dst[i] = i, i < n.  Replaces prefill::mmq::iota (moe_mmq.hpp:110; moe_mmq.cpp:138-140). */
int xs_mmq_iota(int32_t* dst, int64_t n, void* stream);

/* This library's quantizer: n floats (a whole number of blocks) to `type` blocks.  No reference counterpart (the
 * reference's tests call ggml_quantize_chunk, src/kernels/native_expert_parity.cpp:483-487). */
int xs_quantize_rows(int type, const float* x, int64_t n, void* y, void* stream);

/* Router: logits (n_tokens, n_expert) -> ids (n_tokens, k) int32 and renormalised weights (n_tokens, k) f32, in
 * descending probability rank.  Bit for bit the reference's router_top10 (include/strata/kernels/router_top10.hpp:
 * 20-21; src/kernels/xe/router.cpp:59-308).  n_expert <= 1024, k <= 64 and k <= n_expert.  A NULL stream runs on the
 * default stream and synchronises. */
int xs_router_top10(const float* logits, int n_tokens, int n_expert, int k, int32_t* ids, float* weights,
                    void* stream);

/* DeepSeek-V3 routing: sigmoid scores, selection by score + bias (bias may be NULL), group-limited top-k (n_group
 * groups, the topk_group best by their two best scores), weights normalised over the k and times routed_scale.  No
 * reference counterpart (absent from XeStrata). n_expert <= 1024, n_group <= 64, k <= 64. */
int xs_router_grouped_sigmoid(const float* logits, const float* bias, int n_tokens, int n_expert, int n_group,
                              int topk_group, int k, float routed_scale, int32_t* ids, float* weights, void* stream);

/* Router logits logits[t, e] = x[t] . w[e] in fp32 (w: n_expert rows of n_embd floats, n_embd even): up to 8 tokens
 * in the decode GEMV's order (xs_f32_gemv_fp32_mmvf_multi), more in the prompt GEMM's (xs_f32_gemm_rows), so the
 * logits are the reference's bits (src/core/plain_model.cpp:955 and src/prefill/plain_prompt.cpp:561). */
int xs_router_logits_f32(const float* x, const float* w, float* logits, int n_tokens, int64_t n_embd, int n_expert,
                         void* stream);

/* The reference's projection kernels, each in its own summation order (bit for bit its logits):
 * y[t * ldy + o] = x[t * ldx + .] . w[o * n_in + .].
 * - mmvf: B threads a row (the candidate of 32..256 with the fewest pair iterations), two ordered FMAs a pair, a
 *   32-lane xor butterfly, then one over the B/32 partials; 1..8 tokens, n_in even, x 8-byte aligned.  Replace
 *   f32_gemv_fp32_mmvf(_multi) and bf16_gemv_fp32_mmvf(_multi) (src/kernels/xe/bf16_gemv.cpp:91-147, 440-517).
 * - gemm_rows: one FMA chain a logit over k = 0.. n_in - 1 (then zeros to a multiple of 16), any token count.
 *   Replaces f32_gemm_rows (bf16_gemv.cpp:475-502; the prompt path's router and shared gate). */
int xs_f32_gemv_fp32_mmvf_multi(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in,
                                int64_t n_out, int n_tok, void* stream);
int xs_bf16_gemv_fp32_mmvf_multi(const float* x, int64_t ldx, const uint16_t* w, float* y, int64_t ldy, int64_t n_in,
                                 int64_t n_out, int n_tok, void* stream);
int xs_f32_gemm_rows(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in, int64_t n_out,
                     int64_t n_tok, void* stream);
/* f32 -> bf16 bits, nearest even, a NaN kept and quieted.  Replaces f32_to_bf16_bulk
 * (include/strata/kernels/elementwise.hpp:71; bf16_bits.hpp:39-45). */
int xs_f32_to_bf16_bulk(const float* x, uint16_t* y, int64_t n, void* stream);
/* bf16 x against bf16 rows: bf16_gemv (32 lanes a row for n_out >= 64, one chain a row below) and bf16_gemv_split
 * (32 threads: the same 32-lane rows; another power of two: lane chains then a shared-memory tree).  Replace
 * bf16_gemv / bf16_gemv_split (include/strata/kernels/bf16_gemv.hpp:30-39; bf16_gemv.cpp:50-77, 300-339). */
int xs_bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out, void* stream);
int xs_bf16_gemv_split(const uint16_t* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out,
                       int threads_per_row, void* stream);
/* The BF16 router projection of the engine's moe_route: native -> bf16_gemv_fp32_mmvf (f32 x); else x rounded to
 * x_bf16, then bf16_gemv_split at 32 threads (split) or bf16_gemv.  x_bf16 NULL with split: the rounding is done
 * inside the GEMV (the same bits, one launch, no bf16 copy).  Replaces project_bf16 (src/core/layer.cpp:100-107). */
int xs_project_bf16(const float* x, uint16_t* x_bf16, const uint16_t* w, float* out, int64_t n_in, int64_t n_out,
                    int split, int native, void* stream);

/* The decode / verify-window plan built on the device when every routed expert is resident, in the host pool's
 * layout (counts | start | dst | tok | pad | ptr | ptr2 | start2, capx entries): distinct experts in routing order,
 * their entries ascending; *skip = ring when built, 0 (plan untouched) when a routed expert is not resident.
 * res_layer NULL: every expert resident at slot = its id.  n_entries <= 1024, n_expert <= 16384.
 * Replaces resident_plan (include/strata/kernels/verify_kernels.hpp:81-83; verify_kernels.cpp:819-890). */
int xs_resident_plan(const int32_t* ids, int n_entries, int k, const int32_t* res_layer, int n_expert,
                     const uint8_t* cache_base, const unsigned long long* slot_off, long long blob, int32_t* plan,
                     long long capx, uint32_t* skip, uint32_t ring, void* stream);
/* Offsets (in int32 words) of the plan's parts for a capacity capx: start, dst, tok, ptr, start2. */
void xs_plan_offsets(long long capx, long long* start, long long* dst, long long* tok, long long* ptr,
                     long long* start2);

/* The prompt path's permutation on the device: histogram of n_entries ids, experts ascending, exclusive prefix, a
 * stable fill.  src[row] = entry / k, slot[entry] = row, entry_of[row] = entry; bounds[g] (g < *n_groups, then the
 * total) and experts[g] list the experts with rows.  When grp_ptr is not NULL, grp_ptr[g] = cache_base + experts[g]
 * * blob.  *n_groups = -1 when an id is out of range.  n_expert <= 1024.  Replaces the host grouping of
 * src/prefill/plain_prompt.cpp:576-645 (every expert on the GPU). */
int xs_prefill_route(const int32_t* ids, int64_t n_entries, int k, int n_expert, int32_t* src, int32_t* slot,
                     int32_t* entry_of, int32_t* bounds, int32_t* experts, int32_t* n_groups,
                     const uint8_t* cache_base, long long blob, unsigned long long* grp_ptr, void* stream);

/* Grouped experts for prompt and verify batches: f16 MFMA products (fp32 accumulate) on expert weights dequantized
 * from the raw GGUF blocks.  Rows are the routed rows in expert order (xs_prefill_route): row r reads token src[r] of
 * x (fp32, n_embd a token; taken in f16, saturated) and its down output lands in row entry_of[r] of `parts` (routing
 * order, n_embd floats a row); h = SwiGLU(gate, up) is kept in f16.  scratch: xs_moe_prefill_scratch_bytes.  Replaces the prompt path's mmq::Context::run + swiglu +
 * quantize (include/strata/prefill/moe_mmq.hpp:50-94), iq_mmq_grouped (iq_mmq.hpp:49-58), xmx_gemm_grouped
 * (xmx_gemm.hpp:39-43) and the rocBLAS fallback Gemm::f16_groups (src/prefill/gemm.cpp:371-388). */
int xs_moe_prefill_experts(const xs_expert_layout_t* L, const float* x, int64_t n_tok, const int32_t* src,
                           const int32_t* entry_of, const int32_t* bounds, const int32_t* n_groups,
                           const unsigned long long* grp_ptr, int64_t cap_groups, int64_t rows, void* scratch,
                           float* parts, void* stream);
size_t xs_moe_prefill_scratch_bytes(int64_t n_tok, int64_t rows, int64_t n_embd, int64_t n_ff);
/* Device address of the status word inside xs_moe_prefill_experts' scratch (the same sizes as the call): bit 8 set
 * when an activation, an h value or a part passed the f16 range (|v| > 65504) and was saturated - those rows are not
 * the fp32 result.  The bit stays set until the caller clears the word (xs_moe_status_check reads and clears it); a
 * zero-filled scratch starts clear.  No counterpart in the reference (whose FP16 path overflows to inf). */
int32_t* xs_moe_prefill_status(void* scratch, int64_t n_tok, int64_t rows, int64_t n_embd, int64_t n_ff);

/* The weighted combine: output = fl(p0 w0) + fl(p1 w1) + ... in rank order, + shared (the shared row once; times
 * the sigmoid of shared_gate[t] when given).  k in 1..15.  Replaces native_moe_combine and
 * native_moe_combine_multi (include/strata/kernels/native_moe.hpp:22-25; src/kernels/xe/native_moe.cpp:36-58). */
int xs_native_moe_combine(const float* parts, const float* weights, const float* shared, float* output,
                          int64_t n_embd, int64_t k, void* stream);
int xs_native_moe_combine_multi(const float* parts, const float* weights, const float* shared, float* output,
                                int64_t n_embd, int64_t k, int n_tok, void* stream, const float* shared_gate);
/* combine_multi with the tier path's hit rows folded in: entries dst[0, *count) (entry = token * k + rank) read
 * parts + hits, the sum moe_hit_add would leave, before their product.  Replaces native_moe_combine_multi_hits
 * (include/strata/kernels/native_moe.hpp:27-32; src/kernels/xe/native_moe.cpp:67-110). */
int xs_native_moe_combine_multi_hits(const float* parts, const float* hits, const int32_t* dst, const int32_t* count,
                                     const float* weights, const float* shared, float* output, int64_t n_embd,
                                     int64_t k, int n_tok, void* stream, const float* shared_gate);
/* The combine with the residual add fused: output = residual + combine (output may equal residual).  The reference
 * runs native_moe_combine_multi then add_inplace (src/core/plain_model.cpp:985-987). */
int xs_moe_combine_residual(const float* parts, const float* weights, const float* shared, const float* shared_gate,
                            const float* residual, float* output, int64_t n_embd, int64_t k, int n_tok, void* stream);
/* x += y (n floats).  Replaces add_inplace (src/core/plain_model.cpp:987). */
int xs_add_inplace(float* x, const float* y, int64_t n, void* stream);

/* The whole decode MoE layer on the device, every expert resident in one arena (expert e's blob at
 * arena + e * blob_bytes): router -> plan -> q8_1 -> grouped experts -> combine -> residual.
 * out = residual + MoE(x); out may equal residual.  workspace: xs_moe_layer_decode_workspace_bytes for the largest
 * n_tok it will serve, 256-byte aligned, zeroed once before its first call (every call leaves it ready for the next).
 * The layer runs as one persistent launch when n_tok * k <= 256, n_tok <= 64 and the formats are one of Q4_K/Q6_K,
 * Q4_K/Q4_K, Q8_0/Q8_0, IQ4_XS/IQ4_XS; else as the chain of kernels below.  The engine's moe_route + moe_finish
 * surface (include/strata/core/layer.hpp:108-199) on one GPU, without the host ring. */
int xs_moe_layer_decode(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                        const float* x, const float* logits, const float* residual, float* out, int n_tok,
                        void* workspace, size_t workspace_bytes, void* stream);
size_t xs_moe_layer_decode_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok);
/* Device address of the decode workspace's status word: 0 after good calls; bit 1 a wait of the persistent layer
 * passed its bound (50 ms), bit 2 a token's router produced fewer than k experts (NaN logits) - that call wrote no
 * output.  Bits stay set until the caller clears the word; the workspace itself needs no reset after an error.  No
 * counterpart in the reference (its layer reports through host-side checks of each launch). */
int32_t* xs_moe_layer_decode_status(void* workspace);
/* The checked contract of the persistent layer: synchronises `stream`, reads the status word; 0 -> XS_OK; else clears
 * it and returns XS_EDEVICE with the bits named (an expired bounded wait means other work held CUs the layer's
 * work-groups needed, and that call's output is not to be used).  Call it at the next synchronisation point after
 * a layer call (or a run of them).  Not to be called inside a graph capture.  No counterpart in the reference. */
int xs_moe_status_check(int32_t* status, void* stream);
/* The bound of the persistent layer's waits, in ticks of the device's wall clock (hipDeviceAttributeWallClockRate
 * kHz), for calls made after it, process-wide; 0 restores the default (50 ms); -1 makes every wait expire at once
 * (no hand-over word is taken: the error path forced from the host - every work-group still ends normally, the
 * status word reports bit 1 and the output is not to be used); -2 makes every waiter of the one-token layer compute
 * each unit it would wait on itself (the path taken for units whose owners have not started: the output is the same,
 * bit for bit).  A test and diagnosis hook; no counterpart in the reference. */
void xs_moe_set_wait_bound(long long ticks);
/* The prompt layer's product split, process-wide, for calls made after it: on (the default), a layer without a
 * shared expert whose weights are Q4_K or Q6_K runs every whole 256-row tile of an expert's rows on the tall-tile
 * GEMMs (256 x 256 tiles, weights dequantized once a step into LDS) and the other rows beside them on a side stream;
 * off (0), every row takes the 128/64-row GEMMs; 2 runs the split's two chains one after the other on the caller's
 * stream (each chain's kernels then time alone).  All give the f16 path's results bit for bit (the tiles differ, not
 * the arithmetic of a value).  A test and measurement switch; no counterpart in the reference. */
void xs_moe_set_prefill_tall(int on);

/* xs_moe_layer_decode without a caller workspace, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.  The layer
 * runs in the library's own scratch: a fixed XS_NOALLOC_SCRATCH_BYTES array in device memory that each GPU holds
 * from the library's load until the process ends, zero at load and left ready by every call.  Takes hidden sizes up to
 * 8192 and expert widths up to 4096; a call whose tokens x top-k need more scratch than the array holds fails with
 * XS_EINVAL.  status (optional, device int32): where the persistent layer ORs its error bits (those of
 * xs_moe_layer_decode_status; the caller clears it).  Every call on a GPU shares that GPU's array: calls that overlap
 * on one GPU (other streams, other threads) race, so a caller runs them one at a time.  The first call on each device
 * looks the array's address up and must not be inside a graph capture.  Allocates nothing. */
#define XS_NOALLOC_SCRATCH_BYTES ((size_t)48 << 20)
int xs_moe_layer_decode_noalloc(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert,
                                int k, const float* x, const float* logits, const float* residual, float* out,
                                int n_tok, int32_t* status, void* stream);
/* The current device's status word of that fixed scratch: where xs_moe_layer_decode_noalloc ORs its error bits when
 * its status argument is NULL.  Read and clear it with xs_moe_status_check.  NULL (and the message set) when the
 * device's array cannot be looked up.  The first call on a device must not be inside a graph capture.  No counterpart
 * in the reference. */
int32_t* xs_moe_layer_decode_noalloc_status(void);

/* A shared expert over a decode / verify window: every token through one dense expert in the native format (blob:
 * [gate rows | up rows | down rows] of layout SL, 16-byte aligned), shared[t] = down(SwiGLU(gate x_t, up x_t)) on q8_1
 * activations, canonical rows as the routed experts; with w_gate ([n_embd] fp32), gate_logit[t] = w_gate . x_t (the
 * scalar gate the combine turns into 1 / (1 + exp(-g))).  Replaces the engine's shared-expert decode
 * (src/core/plain_model.cpp:959-973: native_mmvq's Q8_0/Q4_K pair, native_swiglu_q8_1 and the F32 gate GEMV,
 * include/strata/kernels/native_mmvq.hpp:45-52, 128-133).  n_tok <= 1024. */
int xs_shared_expert_decode(const xs_expert_layout_t* SL, const uint8_t* blob, const float* x, int n_tok,
                            const float* w_gate, float* shared, float* gate_logit, void* workspace,
                            size_t workspace_bytes, void* stream);
size_t xs_shared_expert_decode_workspace_bytes(const xs_expert_layout_t* SL, int n_tok);
/* xs_moe_layer_decode with a shared expert: the shared expert (xs_shared_expert_decode) first, then the routed layer,
 * whose combine adds the shared row once after the routed ones, times its gate's sigmoid when w_gate is given
 * (native_moe_combine_multi's shared / shared_gate, native_moe.cpp:36-58; plain_model.cpp:951-988).  The workspace
 * (xs_moe_layer_decode_shared_workspace_bytes, zeroed once) starts with the layer's own: its status word is
 * xs_moe_layer_decode_status(workspace). */
int xs_moe_layer_decode_shared(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert,
                               int k, const float* x, const float* logits, const float* residual, float* out,
                               int n_tok, const xs_expert_layout_t* SL, const uint8_t* shared_blob,
                               const float* w_gate, void* workspace, size_t workspace_bytes, void* stream);
size_t xs_moe_layer_decode_shared_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok,
                                                  const xs_expert_layout_t* SL);

/* How a layer routes its tokens.  XS_ROUTER_SOFTMAX: the softmax top-k of the logits, renormalised
 * (router_top10, include/strata/kernels/router_top10.hpp:20-21).  XS_ROUTER_GROUPED_SIGMOID: DeepSeek-V3's routing
 * (xs_router_grouped_sigmoid: sigmoid scores, selection by score + bias, the topk_group best of n_group groups, weights
 * normalised over the k and times routed_scale); no counterpart in the reference, whose layer wires router_top10
 * (src/core/plain_model.cpp:955-956). */
#define XS_ROUTER_SOFTMAX 0
#define XS_ROUTER_GROUPED_SIGMOID 1
typedef struct xs_router_cfg {
    int kind;
    const float* bias;    /* grouped sigmoid: [n_expert] selection bias, or NULL */
    int n_group, topk_group;
    float routed_scale;
} xs_router_cfg_t;

/* The decode layer with either router and an optional shared expert (SL NULL: none; w_gate NULL: ungated): the
 * engine's whole decode MoE section (src/core/plain_model.cpp:951-988) in one call.  router NULL is the softmax.  With
 * the grouped sigmoid router the routing is its own launch ahead of the layer, whose kernels then take its ids and
 * weights.  workspace: xs_moe_layer_decode_ex_workspace_bytes, 256-byte aligned, zeroed once (as
 * xs_moe_layer_decode's, whose status word it starts with). */
int xs_moe_layer_decode_ex(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                           const float* x, const float* logits, const float* residual, float* out, int n_tok,
                           const xs_router_cfg_t* router, const xs_expert_layout_t* SL, const uint8_t* shared_blob,
                           const float* w_gate, void* workspace, size_t workspace_bytes, void* stream);
size_t xs_moe_layer_decode_ex_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok,
                                              const xs_expert_layout_t* SL);

/* The whole prompt / verify MoE layer on the device (same arena): router -> permutation -> f16 MFMA grouped
 * experts -> combine -> residual.  The engine's prompt MoE section (src/prefill/plain_prompt.cpp:558-797). */
int xs_moe_layer_prefill(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert,
                         int k, const float* x, const float* logits, const float* residual, float* out, int n_tok,
                         void* workspace, size_t workspace_bytes, void* stream);
size_t xs_moe_layer_prefill_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok);
/* Device address of the prompt layer workspace's status word (its first word; _ex's too): 0 after good calls; bit 8 a
 * value of the f16 path (an activation, h or a part, routed or shared) passed the f16 range and was saturated at
 * +-65504 - the affected rows are not the fp32 result.  A zero-filled workspace starts clear; the bits stay until the
 * caller clears the word (xs_moe_status_check).  No counterpart in the reference. */
int32_t* xs_moe_layer_prefill_status(void* workspace);
/* The prompt layer with either router and an optional shared expert: every token through the shared expert (one group
 * of the f16 MFMA GEMMs, rows in fp32) and the combine adding its row once after the routed ones, times the sigmoid of
 * its gate logit w_gate . x when w_gate is given - the reference's prompt layer (src/prefill/plain_prompt.cpp:
 * 788-797: the shared SwiGLU and down projection, then native_moe_combine_multi with shared and sh_g). */
int xs_moe_layer_prefill_ex(const xs_expert_layout_t* L, const uint8_t* arena, size_t blob_bytes, int n_expert, int k,
                            const float* x, const float* logits, const float* residual, float* out, int n_tok,
                            const xs_router_cfg_t* router, const xs_expert_layout_t* SL, const uint8_t* shared_blob,
                            const float* w_gate, void* workspace, size_t workspace_bytes, void* stream);
size_t xs_moe_layer_prefill_ex_workspace_bytes(const xs_expert_layout_t* L, int n_expert, int k, int n_tok,
                                               const xs_expert_layout_t* SL);

/* Measuring kernels for the achieved peaks of the box (no counterpart in the reference; bench.py's roofline lines).
 * xs_bench_hbm_read: reads `bytes` (16-byte aligned, a multiple of 16) at src once with `grid` work-groups of 256
 * threads, nontemporal 16-byte loads; writes grid words to sink.  xs_bench_mfma_f16: `grid` work-groups of two waves,
 * each wave `iters` x 8 back-to-back v_mfma_f32_32x32x16_f16 (32,768 flops each); writes nothing but keeps sink
 * (grid x 128 floats) as its output.  Enqueued on `stream`. */
int xs_bench_hbm_read(const void* src, size_t bytes, unsigned int* sink, int grid, void* stream);
int xs_bench_mfma_f16(int iters, int grid, float* sink, void* stream);
/* grid work-groups of 1024 threads, each thread iters x 8 conflict-free 16-byte LDS reads (ds_read_b128): the LDS
 * read rate, iters x 8 x 16 x 1024 bytes a work-group.  sink: grid words (written only in a case that never happens). */
int xs_bench_lds_read(int iters, int grid, unsigned int* sink, void* stream);
/* n_wg work-groups of 64 threads, each holding lds_bytes of LDS (<= 160 KB: one a compute unit at the most) for `ticks`
 * of the device's wall clock (<= 20 s), then ending: other work owning part of the GPU, for tests of the persistent
 * layers beside it.  sink: n_wg words (written only in a case that never happens). */
int xs_bench_occupy(int n_wg, int lds_bytes, long long ticks, unsigned int* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif
