// xestrata-win_amd/csrc/xs_kernels.h - launchers of the HIP kernels, called by the C ABI layer (abi.cpp).
// Launchers check nothing the ABI layer has not already checked; they return the launch's hipError_t.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xs {

struct ExpertLayout {   // one native expert blob: [gate rows | up rows | down rows], raw GGUF blocks
    int gu_type, d_type;
    int64_t n_embd, n_ff;
    int64_t gu_row, d_row, up_off, down_off, bytes;
    int up_type = -1;      // the up rows' type: gu_type's, or another gate/up type (a mixed layer; -1: gu_type)
    int64_t up_row = 0;    // bytes of an up row (0: gu_row)
};
// a layer whose up rows are of another type than its gate rows (the paths that take one gate/up type refuse it)
inline bool mixed_gu(const ExpertLayout& L) { return L.up_type >= 0 && L.up_type != L.gu_type; }

// formats.hip
hipError_t launch_quantize_rows(int type, const float* x, int64_t n, void* y, hipStream_t s);
// out: kDequantF32 (float), kDequantBf16 (bf16 bits, nearest even), kDequantF16 (half bits, nearest even)
enum : int { kDequantF32 = 0, kDequantBf16 = 1, kDequantF16 = 2 };
hipError_t launch_dequant(int type, const void* src, int64_t n, void* dst, int out, hipStream_t s);

// quant_act.hip
hipError_t launch_quantize_q8_1_rows(const float* x, int64_t n_rows, int64_t n_cols, void* y, hipStream_t s);

// experts_decode.hip
struct GroupedArgs {
    const unsigned long long* grp_ptr;
    const int32_t* grp_start;
    const int32_t* n_groups;
    const int32_t* ent_dst;
    const int32_t* ent_tok;
    const void* x_q8_1;
    float* gate;   // scratch: [cap_entries, n_ff]
    float* up;     // scratch: [cap_entries, n_ff]
    void* hq;      // scratch: [cap_entries, n_ff / 32] q8_1 blocks
    float* out;
    int32_t* err;  // device word: set non-zero when a blob address is not 16-byte aligned
    int64_t cap_groups, grid_groups;
    int max_entries;   // the most entries a group can have (the call's token count), 0 when not known
    void* hact;        // scratch: the down stream's h activations (int8 values, scales, sums of 16)
    int64_t cap_entries_hint;   // the entries the scratch was sized for
};
hipError_t launch_native_gu(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s);
hipError_t launch_native_down(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s);
// experts_stream.hip: the same products as a weight stream (2..16 tokens, the four formats)
bool stream_usable(const ExpertLayout& L, int n_tok, int64_t cap_groups, int64_t cap_entries);
hipError_t launch_stream_gu(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s);
hipError_t launch_stream_down(const ExpertLayout& L, const GroupedArgs& a, hipStream_t s);

// router.hip
hipError_t launch_router_topk(const float* logits, int n_tokens, int n_expert, int k, int32_t* ids, float* weights,
                              hipStream_t s);
hipError_t launch_router_grouped_sigmoid(const float* logits, const float* bias, int n_tokens, int n_expert,
                                         int n_group, int topk_group, int k, float routed_scale, int32_t* ids,
                                         float* weights, hipStream_t s);

// dispatch.hip
hipError_t launch_resident_plan(const int32_t* ids, int n, int k, const int32_t* res, int n_expert,
                                const uint8_t* cache_base, const unsigned long long* slot_off, long long blob,
                                int32_t* plan, long long capx, uint32_t* skip, uint32_t ring, hipStream_t s);
hipError_t launch_prefill_route(const int32_t* ids, int64_t n, int k, int n_expert, int32_t* src, int32_t* slot,
                                int32_t* entry, int32_t* bounds, int32_t* experts, int32_t* n_groups,
                                const uint8_t* cache_base, long long blob, unsigned long long* grp_ptr, hipStream_t s);

// the prompt GEMMs' f16 copy of x [n_tok, n_embd] (n_chunks = n_tok n_embd / 8), its saturation bit into err
struct ToF16 {
    const float* x;
    uint16_t* y;
    int64_t n_chunks;
    int32_t* err;
};
// the same permutation over ceil(n / 1024) work-groups (ghist: prefill_route_split_scratch bytes), and, when mtile
// is given, the m-tile table launch_prefill_experts would compute (PrefillArgs::mtile_ready), or with split the one
// launch_prefill_experts_split takes (the tall list, and the maps over the rows past each group's tall tiles).  With
// conv, work-groups past the permutation's build the f16 copy of x in the same launch (PrefillArgs::xb_ready).
hipError_t launch_prefill_route_split(const int32_t* ids, int64_t n, int k, int n_expert, int32_t* src, int32_t* slot,
                                      int32_t* entry, int32_t* bounds, int32_t* experts, int32_t* n_groups,
                                      const uint8_t* cache_base, long long blob, unsigned long long* grp_ptr,
                                      int32_t* ghist, int32_t* mtile, int cap_groups, hipStream_t s,
                                      bool split = false, const ToF16* conv = nullptr);
size_t prefill_route_split_scratch(int64_t n, int n_expert);

// decode_layer.hip
hipError_t launch_decode_route(const float* logits, const float* x, int n_tok, int n_expert, int k, int64_t n_embd,
                               int32_t* ids, float* weights, int32_t* plan, long long capx, uint32_t* skip,
                               const uint8_t* arena, long long blob, void* xq, hipStream_t s);

// decode_fused.hip
struct FusedPlan {     // the fused decode layer's unit sizes (a function of the layout alone, save ne and lds)
    int rh, rd;        // SwiGLU outputs a gate/up unit, down rows a down unit
    int nu, nj;        // gate/up units, down units a group
    int slab_gu, slab_dn;
    int ne, lds;       // entries a pass, dynamic LDS bytes
    int ttab;          // tokens of the pipelined gate/up path's activation table (0: that path is off)
    int direct;        // 1: one token, units read their rows from HBM straight into registers (no LDS slabs)
    int alias;         // 1: the down slab lies over the gate/up slabs (no down rows fetched during gate/up units)
};
constexpr int kMarkWords = 1024;
struct FusedArgs {
    ExpertLayout L;
    const uint8_t* arena;
    long long blob;
    int n_expert, k, n_tok;
    const float* logits;    // [n_tok, n_expert]
    const float* x;         // [n_tok, n_embd]
    const float* residual;  // [n_tok, n_embd] (NULL: none, the combined rows alone; the persistent layer only)
    float* out;             // [n_tok, n_embd], may equal residual
    int32_t* ids;           // [n_tok * k]
    float* weights;         // [n_tok * k]
    // hand-over words: a float's bits | the call's tag << 32 (tags never repeat, so no reset is needed)
    unsigned long long* hx; // [256, n_ff] SwiGLU outputs, plan order
    unsigned long long* px; // [256, n_embd] expert outputs, routing order
    int32_t* sync;          // 16 64-bit call counters at sync + 32 i (2 KB, 8-byte aligned; 2^20 a call in all, the
                            // call's tag from their sum >> 20), zero before the first call
    uint32_t* marks;        // [kMarkWords] a word a unit or virtual work-group: the call's tag once its owner runs it
                            // (the waiters' test of whether an owner has started, decode_t1.hip / decode_fused.hip)
    int32_t* err;
    int rh, rd, nu, nj, slab_gu_bytes, slab_dn_bytes, ttab, direct;
    int slab_alias = 0;     // FusedPlan::alias
    long long spin_ticks;   // bound of a wait, in wall-clock ticks
    long long help_ticks = 0;   // how long a waiter waits before it reads the owner's mark (the one-token layer: an
                                // unmarked unit is computed by the waiter); < 0: every waiter computes every unit
                                // (the host's test of that path)
    const float* shared;       // [n_tok, n_embd] the shared expert's rows, added once by the combine (NULL: none)
    const float* shared_gate;  // [n_tok] its gate logits (NULL: ungated)
    // routing already done by another router (DeepSeek's group-limited sigmoid): ids / weights [n_tok, k] in rank
    // order, read instead of routing the logits (NULL: the softmax top-k of the logits)
    const int32_t* pre_ids = nullptr;
    const float* pre_w = nullptr;
    // the group-limited sigmoid router in the routing stage itself (sig_group > 0: n_group; the groups on whole lanes,
    // route_grouped_sigmoid_wave in xs_route.h), instead of softmax top-k, when pre_ids is NULL
    const float* sig_bias = nullptr;
    int sig_group = 0, sig_topk_group = 0;
    float sig_scale = 1.0f;
    // the waves that issue the pipelined (512-thread) instance's loads: 6 where one work-group fills a CU, 4 where two
    // do (launch_decode_fused sets it; the other instances use 3)
    int load_waves = 4;
};
bool fused_decode_plan(const ExpertLayout& L, int n_expert, int k, int n_tok, FusedPlan* P);
hipError_t launch_decode_fused(const FusedArgs& a, const FusedPlan& P, hipStream_t s);
// whether the persistent layer's instances for this layout can run the grouped sigmoid router in their routing stage
// (FusedArgs sig_group): the Q4_K pair's (DeepSeek-V3's layout here); other layouts take the router's own launch
bool fused_sigmoid_layout(int gu_type, int d_type);
// a one-expert layer's routing for the persistent layer's pre_ids / pre_w (expert 0, weight 1.0 for each of up to
// kOneExpertMaxTok tokens): device addresses of this device's arrays
constexpr int kOneExpertMaxTok = 64;
hipError_t one_expert_routing(const int32_t** ids, const float** w);
// decode_t1.hip: the one-token layer (a.n_tok == 1) with the down units over every expert and the combine inside them;
// *used = false (nothing launched) when the layout is not one it takes, and the caller launches launch_decode_fused.
// Needs the same workspace (a.hx holds the q8_1 h words).
hipError_t launch_decode_t1(const FusedArgs& a, hipStream_t s, bool* used);

// the plan of one group of n entries (a shared expert over n tokens): grp_ptr[0] = blob, start = {0, n},
// *n_groups = 1, idx[i] = i (the entries' destination rows and tokens)
hipError_t launch_single_group_plan(unsigned long long* grp_ptr, int32_t* start, int32_t* n_groups, int32_t* idx,
                                    int n, const uint8_t* blob, hipStream_t s);

// combine.hip
hipError_t launch_combine(const float* parts, const float* weights, const float* shared, const float* shared_gate,
                          const float* residual, float* out, int64_t n_embd, int k, int n_tok, hipStream_t s);
hipError_t launch_add_inplace(float* x, const float* y, int64_t n, hipStream_t s);
// the combine over f16 parts, + residual (n_embd % 4 == 0)
// gemv.hip: the router projections in the reference's summation orders
int mmvf_block(int64_t n_in);
template <typename W>
hipError_t launch_mmvf(const float* x, int64_t ldx, const W* w, float* y, int64_t ldy, int64_t n_in, int64_t n_out,
                       int n_tok, hipStream_t s);
hipError_t launch_gemm_rows(const float* x, int64_t ldx, const float* w, float* y, int64_t ldy, int64_t n_in,
                            int64_t n_out, int64_t n_tok, hipStream_t s);
enum : int { kBf16Warp = 0, kBf16Naive = 1, kBf16Tree = 2 };
hipError_t launch_bf16_gemv(const void* x, bool x_f32, const uint16_t* w, float* y, int64_t n_in, int64_t n_out,
                            int form, int tpr, hipStream_t s);
hipError_t launch_to_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t s);

// mmq.hip: the int8 MMQ activations (map: ids of the gathered form, slot of the scatter form), SwiGLU rows, iota
hipError_t launch_mmq_quantize(const float* x, const int32_t* map, void* xq, int64_t cols, int64_t ld, int64_t n_src,
                               int64_t rows, int k_used, bool scatter, bool sums, bool dup, hipStream_t s);
hipError_t launch_mmq_swiglu(const float* gu, float* h, int64_t rows, int64_t n_ff, bool interleaved, hipStream_t s);
hipError_t launch_iota(int32_t* dst, int64_t n, hipStream_t s);

// combine_multi with moe_hit_add folded in: entries dst[0 .. *count) read parts + hits
hipError_t launch_combine_hits(const float* parts, const float* hits, const int32_t* dst, const int32_t* count,
                               const float* weights, const float* shared, const float* shared_gate, float* out,
                               int64_t n_embd, int k, int n_tok, hipStream_t s);
hipError_t launch_combine_h(const uint16_t* parts, const float* weights, const float* shared,
                            const float* shared_gate, const float* residual, float* out, int64_t n_embd, int k,
                            int n_tok, hipStream_t s);

// experts_prefill.hip
struct PrefillArgs {
    const float* x;                 // [n_tok, n_embd] activations (fp32)
    const int32_t* src;             // [rows] token of each routed row (expert-sorted order)
    const int32_t* entry;           // [rows] routing entry each row writes
    const int32_t* bounds;          // [groups + 1] row bounds of each group
    const int32_t* n_groups;        // device count of groups
    const unsigned long long* wptr; // [groups] blob address of each group's expert
    uint16_t* xb;                   // scratch: [n_tok, n_embd] f16 copy of x, in the GEMM's K order
    uint16_t* h;                    // scratch: [rows, n_ff] f16 SwiGLU output, in the GEMM's K order
    float* parts;                   // [n_tok * k, n_embd] routing-order outputs
    uint16_t* parts_h;              // the same in f16 (saturated), written in place of parts when set
    int32_t* mtile;                 // scratch: the m-tile table (tile_table_words words, layout at tile_list)
    bool mtile_ready;               // mtile already holds it (launch_prefill_route_split wrote it)
    bool xb_ready = false;          // xb already holds the f16 copy of x (launch_prefill_route_split built it)
    int32_t* err;
    int64_t n_tok, rows, cap_groups;
    int64_t ld_parts;               // values between the rows of parts / parts_h (n_embd for the layer's own)
    // the standalone product (launch_mmq_product): no scratch.  A rows are the int8 MMQ activations ([rows][K] codes,
    // then a float scale a 32), turned to f16 as they are staged; group g's weights at wtab[g] + woff, or at wbase +
    // g * wstride; each work-group finds its m-tile from bounds (cap_groups groups)
    const int8_t* xq;
    const uint8_t* wbase;
    size_t wstride;
    const uint8_t* const* wtab;
    size_t woff;
};
hipError_t launch_prefill_experts(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s);
// The same products split in two chains: every whole 256-row tile of a group on the tall-tile GEMMs (8 waves over 256
// rows x 256 or 128 weight rows, weights dequantized once a step into LDS) on `s`, the remaining rows on the 128-row
// GEMMs on `side` (which waits for `s` to have built the f16 activations: `fork` is recorded on s, `join` on side;
// side == s runs the chains one after the other).  a.mtile must hold the split form launch_prefill_route_split wrote
// (mtile_ready); only for the layouts tall_usable accepts.
bool tall_usable(const ExpertLayout& L);
hipError_t launch_prefill_experts_split(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s, hipStream_t side,
                                        hipEvent_t fork, hipEvent_t join);
// The grouped product alone (the reference's iq_mmq_grouped), one launch and no scratch: the int8 MMQ activations
// a.xq times every group's [n_embd, n_ff] matrix (the down product's tiles: L.d_type, L.d_row) into
// a.parts[a.entry[row] * a.ld_parts + ...] in fp32.
hipError_t launch_mmq_product(const ExpertLayout& L, const PrefillArgs& a, hipStream_t s);

// The m-tile table of a prompt batch: words 0, 1 the counts of full and of partial tiles of the 128-row map, words
// 2, 3 the same of the 64-row map, then each map's list of tile_cap entries {group | rows << 16, first row}: the full
// tiles from the front (every group's, groups ascending), the partial ones from the back (entry cap - 1 - i for the
// i-th), so that a work-group's m-tile index mt < full is entry mt and is dispatched before every partial tile.
__host__ __device__ inline int64_t tile_cap(int64_t rows, int bm, int64_t cap_groups) {
    return (rows + bm - 1) / bm + cap_groups;
}
__host__ __device__ inline int32_t* tile_list(int32_t* t, int64_t rows, int64_t cap_groups, int bm) {
    return t + 4 + (bm == 128 ? 0 : 2 * tile_cap(rows, 128, cap_groups));
}
// the tall-tile list (experts_prefill.hip, tall_mfma_kernel): after both maps, its count, then {group, first row} of
// every whole 256-row tile of a group (when the maps were written for the rows past those tiles only)
__host__ __device__ inline int32_t* tall_list(int32_t* t, int64_t rows, int64_t cap_groups) {
    return t + 4 + 2 * (tile_cap(rows, 128, cap_groups) + tile_cap(rows, 64, cap_groups));
}
__host__ __device__ inline int64_t tile_table_words(int64_t rows, int64_t cap_groups) {
    return 4 + 2 * (tile_cap(rows, 128, cap_groups) + tile_cap(rows, 64, cap_groups)) + 1 + 2 * (rows / 256 + 1);
}
// the tiles of group g (rows [start, start + n)) in a map of bm-row tiles with `cap` entries, given the full and the
// partial tiles of the groups before it
__device__ inline void write_group_tiles(int32_t* list, int g, int start, int n, int bm, int full_before,
                                         int part_before, int64_t cap) {
    const int nf = n / bm;
    for (int t = 0; t < nf; ++t) {
        list[2 * (full_before + t)] = g | (bm << 16);
        list[2 * (full_before + t) + 1] = start + t * bm;
    }
    if (n % bm) {
        const int64_t e = cap - 1 - part_before;
        list[2 * e] = g | ((n % bm) << 16);
        list[2 * e + 1] = start + nf * bm;
    }
}

// the decode layer over a workspace whose tagged hand-over words sit in fixed regions sized for the largest layout
// (abi.cpp; the library's own scratch of noalloc.hip): hidden sizes up to kScratchMaxEmbd, expert widths up to
// kScratchMaxFF
constexpr int64_t kScratchMaxEmbd = 8192, kScratchMaxFF = 4096;

}  // namespace xs
