/*
 * include/xs_pack.h - a native expert pack's arena in HBM, read from the model's GGUF shards in place.
 *
 * The other side of the expert kernels' boundary: where each routed expert's blob lives and how the arena is filled.
 * A blob is [gate rows | up rows | down rows] in raw GGUF blocks (xs_native_expert_layout's offsets); layer l's n_expert
 * blobs follow one another from the arena offset its table row gives, and the layers follow one another.  The layout
 * comes from a pack's `native_experts.txt` (upstream Strata's v2-v4 and XeStrata's xs1 headers) or from the expert
 * tensors of a GGUF model; the arena is filled from the gate / up / down tensors (blk.<b>.ffn_<role>_exps.weight, each
 * the n_expert experts one after another), each expert's slices landing at their places in its blob.  Paths relative
 * to the reference repository, 32x-k/XeStrata-win.
 *
 * Unlike the kernels' entry points these are host calls: they read files, allocate host memory (the table, and
 * pinned staging buffers while loading) and block until done.  Loading copies into memory the caller owns (device
 * memory, or host memory HIP can address) and allocates no device memory.  Return codes and xs_last_error() are
 * include/xs_moe.h's.
 */
#ifndef XS_PACK_H
#define XS_PACK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A pack's expert layout (opaque).  Mirrors ExpertLayout (include/strata/kernels/cpu/expert_layout.hpp:21-49). */
typedef struct xs_pack xs_pack_t;

typedef struct xs_pack_info {
    int version;              /* native_experts.txt's header version (upstream v2-v4; xs1 reads as 4; 0 none) */
    int has_gguf_off;         /* 1 when the table holds the tensors' absolute GGUF offsets (v2 and later) */
    int64_t n_layers, n_expert;
    uint64_t max_blob;        /* the largest blob of any layer */
    uint64_t total;           /* bytes of the whole arena */
} xs_pack_info_t;

typedef struct xs_pack_layer {
    int gu_type, d_type, up_type;   /* ggml type ids of gate, down and up */
    int64_t block;                  /* the model's block of this MoE layer (blk.<block>.ffn_*_exps) */
    uint64_t offset;                /* arena offset of the layer's first blob */
    uint64_t bytes;                 /* bytes of one blob */
    uint64_t up_off, down_off;      /* the up and down rows' offsets inside a blob */
    uint64_t gguf_off[3];           /* absolute offsets of the gate, up and down tensors in their files (0 unknown) */
    const char* gguf_file[3];       /* their files, names beside the native shard ("" = that shard); valid while the
                                       pack lives */
} xs_pack_layer_t;

typedef struct xs_pack_load_stats {
    uint64_t bytes;                 /* arena bytes written */
    uint64_t layers;
    double seconds;                 /* wall time of the load, files to arena */
} xs_pack_load_stats_t;

/* native_experts.txt of `pack_dir` for n_layers MoE layers of n_expert experts (a header's "(n_expert N" wins, as
 * for a pruned model) at n_embd x n_ff.  Blob sizes must equal what the types make; layers must be contiguous from
 * offset 0; the shard column is one name, "gate,up,down" (an empty field: the native shard) or three names ("-":
 * the native shard).  Refuses versions past v4 / xs1.  A directory without native_experts.txt is refused: the Strata
 * Q2_0 expert form it would mean is not a format these kernels read.
 * Replaces expert_layout_load (include/strata/kernels/cpu/expert_layout.hpp; src/kernels/cpu/expert_layout.cpp:278-393). */
int xs_pack_layout_load(const char* pack_dir, int64_t n_layers, int64_t n_expert, int64_t n_embd, int64_t n_ff,
                        xs_pack_t** out);

/* The layout of a GGUF model's routed experts, read in place: MoE layer i is block moe_blocks[i]; gate and up are
 * [n_embd, n_ff, n_expert], down [n_ff, n_embd, n_expert], in any shard of the model `gguf` belongs to
 * (<name>-0000i-of-0000N.gguf).  Replaces expert_layout_from_gguf (include/strata/core/expert_source.hpp:825-830;
 * src/core/expert_source.cpp:2706-2782). */
int xs_pack_layout_from_gguf(const char* gguf, const int64_t* moe_blocks, int64_t n_layers, int64_t n_expert,
                             int64_t n_embd, int64_t n_ff, xs_pack_t** out);

void xs_pack_free(xs_pack_t* pack);

int xs_pack_info(const xs_pack_t* pack, xs_pack_info_t* out);

/* Layer `layer`'s row of the table.  Mirrors ExpertLayout's per-layer vectors (expert_layout.hpp:22-44). */
int xs_pack_layer(const xs_pack_t* pack, int64_t layer, xs_pack_layer_t* out);

/* Arena offset of (layer, expert)'s blob; ~0 when out of range.  Replaces ExpertLayout::blob_offset
 * (expert_layout.hpp:44-46). */
uint64_t xs_pack_blob_offset(const xs_pack_t* pack, int64_t layer, int64_t expert);

/* Every (layer, role) tensor against the model's files, headers only: present in the file the table names, of the
 * table's type and shape, of the table's bytes per expert, at the table's offset, and not past the end of its file.
 * `native_shard` is the GGUF the table's empty file names mean.  Replaces check_experts_gguf
 * (include/strata/core/expert_source.hpp:824; src/core/expert_source.cpp:2784-2841). */
int xs_pack_check_gguf(const xs_pack_t* pack, const char* native_shard);

/* The whole arena (pack total bytes at `arena`, arena_bytes at least that) from the model's shards: checked as
 * xs_pack_check_gguf first, then each tensor read in chunks of experts into pinned staging on `threads` host threads
 * (0: 4) and copied into the blobs with strided copies, two chunks in flight a thread.  Blocks until the arena holds
 * every byte.  Replaces load_experts_gguf (include/strata/core/expert_source.hpp:831-832;
 * src/core/expert_source.cpp:2843-2916). */
int xs_pack_load_gguf(const xs_pack_t* pack, const char* native_shard, void* arena, uint64_t arena_bytes,
                      int threads, xs_pack_load_stats_t* stats);

/* The same into one destination per layer (layer_dst[l] receives that layer's n_expert blobs).  Replaces the
 * per-layer overload of load_experts_gguf (src/core/expert_source.cpp:2843). */
int xs_pack_load_gguf_layers(const xs_pack_t* pack, const char* native_shard, void* const* layer_dst, int threads,
                             xs_pack_load_stats_t* stats);

#ifdef __cplusplus
}
#endif

#endif /* XS_PACK_H */
