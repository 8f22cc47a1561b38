/*
 * oracle/xs_oracle.h - CPU restatement of XeStrata's MoE-layer hot path, used ONLY as the checker.
 *
 * TEST INFRASTRUCTURE.  Nothing in the product (the HIP library, its C ABI, bench.py's GPU leg) may include, link
 * or call this code.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load liboracle.so.
 *
 * Every function states the reference file:line whose arithmetic it follows (paths relative to the reference
 * repository root, 32x-k/XeStrata-win).  Block layouts are the GGUF ones (third_party/main/ggml/ggml-common.h):
 *   Q8_0   34 B / 32 values   {fp16 d; int8 qs[32]}
 *   Q8_1   36 B / 32 values   {fp16 d; fp16 s; int8 qs[32]}
 *   Q4_K  144 B / 256 values  {fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]}
 *   Q6_K  210 B / 256 values  {u8 ql[128]; u8 qh[64]; i8 scales[16]; fp16 d}
 *   IQ4_XS 136 B / 256 values {fp16 d; u16 scales_h; u8 scales_l[4]; u8 qs[128]}
 * Type ids are ggml's: Q8_0 = 8, Q4_K = 12, Q6_K = 14, IQ4_XS = 23.
 */
#ifndef XS_ORACLE_H
#define XS_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { XSO_Q8_0 = 8, XSO_Q4_K = 12, XSO_Q6_K = 14, XSO_IQ4_XS = 23 };

/* ---- formats and scalar conversions */
float xso_fp16_to_fp32(uint16_t h);
uint16_t xso_fp32_to_fp16(float f);                  /* round to nearest even, IEEE overflow to inf */
int64_t xso_row_bytes(int type, int64_t n);          /* bytes of n values of `type`; 0 for an unknown type */
int xso_block_values(int type);                      /* values per block */
void xso_dequant_row(int type, const uint8_t* src, int64_t n, float* dst);

/* ---- canonical math (include/strata/kernels/canon_math.hpp) */
float xso_canon_rcp(float v);
float xso_canon_exp(float x);
float xso_canon_silu_mul(float g, float u);
void xso_canon_silu_mul_n(const float* g, const float* u, int64_t n, float* h);
void xso_canon_exp_n(const float* x, int64_t n, float* y);
void xso_canon_rcp_n(const float* x, int64_t n, float* y);

/* ---- q8_1 activations (src/kernels/xe/iq_kernels.cpp:1850-1879 and 1209-1223) */
void xso_quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, uint8_t* y);
void xso_quantize_q8_1_per32(const float* x, int64_t n, uint8_t* y);

/* ---- one row of quantized weights against one q8_1 activation row (iq_kernels.cpp:398-721): xso_vec_dot in the
 * canonical order the HIP kernels take (integer-first units, lane-strided, butterfly; see xs_oracle.c), and
 * xso_vec_dot_calls with the reference's per-call float expressions in call order (a cross-check). */
float xso_vec_dot(int type, const uint8_t* row, const uint8_t* xq, int64_t n, int s256);
float xso_vec_dot_calls(int type, const uint8_t* row, const uint8_t* xq, int64_t n, int s256);
int xso_canon_lanes(int64_t units);

/* ---- the native expert blob: [gate rows | up rows | down rows] (iq_kernels.cpp:2021-2036) */
typedef struct {
    int gu_type, d_type;
    int64_t n_embd, n_ff;
    int64_t gu_row, d_row, up_off, down_off, bytes;
    int64_t up_type, up_row;   /* the up rows' type and row bytes (the gate's, or another: a mixed layer) */
} xso_layout;
int xso_native_layout(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, xso_layout* out);
/* A mixed layer (iq_kernels.cpp:2003-2005, 2021-2036): gate rows of gu_type, up rows of up_type, each read as a
 * gate/up matrix of its own type. */
int xso_native_layout_mixed(int gu_type, int d_type, int64_t n_embd, int64_t n_ff, int up_type, xso_layout* out);

/* Grouped experts (iq_kernels.cpp:2042-2178): group g reads blob blobs[g]; entries [start[g], start[g+1]) read token
 * ent_tok[e]'s q8_1 row of x_q8_1 and write row ent_dst[e] of out (n_embd floats).  gate/up/hq (optional, may be
 * NULL) receive the intermediate rows per entry (cap x n_ff floats; cap x n_ff/32 q8_1 blocks). */
void xso_native_expert_grouped(const xso_layout* L, const uint8_t* const* blobs, const int32_t* start, int n_groups,
                               const int32_t* ent_dst, const int32_t* ent_tok, const uint8_t* x_q8_1, float* out,
                               float* gate, float* up, uint8_t* hq, int n_threads);

/* ---- router (src/kernels/xe/router.cpp:59-145) */
void xso_router_top10(const float* logits, int n_tokens, int n_expert, int k, int32_t* ids, float* weights);
/* DeepSeek-V3 routing (no reference counterpart: the DeepSeek-V3 report's sigmoid + bias, group-limited top-k) */
void xso_router_grouped_sigmoid(const float* logits, const float* bias, int n_tokens, int n_expert, int n_group,
                                int topk_group, int k, float routed_scale, int32_t* ids, float* weights);

/* ---- decode plan (src/kernels/xe/verify_kernels.cpp:819-890; host replay src/kernels/resident_plan_parity.cpp:60-96)
 * Writes counts[0..2], start[0..groups], dst[0..n), tok[0..n) and group_expert[0..groups). Returns groups. */
int xso_decode_plan(const int32_t* ids, int n, int k, int32_t* counts, int32_t* start, int32_t* dst, int32_t* tok,
                    int32_t* group_expert);

/* ---- prefill permutation (src/prefill/plain_prompt.cpp:576-637, every expert on the GPU).  Returns groups. */
int xso_prefill_route(const int32_t* ids, int64_t n_entries, int k, int n_expert, int32_t* src, int32_t* slot,
                      int32_t* entry, int32_t* bounds, int32_t* experts, int32_t* counts);

/* ---- combine (src/kernels/xe/native_moe.cpp:36-58) */
void xso_combine(const float* parts, const float* weights, const float* shared, const float* shared_gate, float* out,
                 int64_t n_embd, int k, int n_tok);

/* ---- float reference of the expert products (src/kernels/native_expert_parity.cpp:104-130): dequantized weights
 * times the activations in double, h = g / (1 + exp(-g)) * u rounded to float, then the down product.  One row of
 * `out` (n_embd floats) per listed (expert blob, token) pair. */
void xso_expert_float(const xso_layout* L, const uint8_t* const* blobs, const float* x, const int32_t* tok, int n,
                      float* out, int n_threads);

/* ---- the whole decode layer on the host (router -> plan -> q8_1 -> grouped experts -> combine -> residual), the
 * CPU baseline's workload.  blobs_by_expert[e] is expert e's blob.  out = residual + combine. */
void xso_moe_layer_decode(const xso_layout* L, const uint8_t* const* blobs_by_expert, int n_expert, int k,
                          const float* x, const float* logits, const float* residual, int n_tok, float* out,
                          int n_threads);
void xso_shared_expert(const xso_layout* SL, const uint8_t* blob, const float* x, int n_tok, float* shared,
                       int n_threads);
void xso_moe_layer_decode_shared(const xso_layout* L, const uint8_t* const* blobs_by_expert, int n_expert, int k,
                                 const float* x, const float* logits, const float* residual, int n_tok,
                                 const xso_layout* SL, const uint8_t* shared_blob, const float* gate_logit, float* out,
                                 int n_threads);

/* ---- the router projections in the reference's orders (src/kernels/xe/bf16_gemv.cpp) */
int xso_mmvf_block(int64_t n_in);
void xso_mmvf(const float* x, int64_t ldx, const float* w_f32, const uint16_t* w_bf16, float* y, int64_t ldy,
              int64_t n_in, int64_t n_out, int n_tok);
void xso_gemm_rows(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in, int64_t n_out,
                   int64_t n_tok);
void xso_bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, int64_t n_in, int64_t n_out, int form, int tpr);

#ifdef __cplusplus
}
#endif
#endif
