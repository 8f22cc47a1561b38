/*
 * include/xs_tiers.h - the tier protocol's device steps: what lets the engine's CPU and PCIe expert tiers share a
 * layer with the HIP kernels (the reference's verify window, src/core/moe_window.cpp:196-250).
 *
 * The engine's host pool writes a layer's GPU plan (the GpuPlanSink words of include/xs_moe.h's xs_plan_offsets:
 * counts | start | dst | tok | pad | ptr | ptr2 | start2) into mapped host memory and rings a flag.  The device side:
 * wait for the flag, copy the plan in, run the VRAM groups (ptr / start / counts[0]) and the PCIe groups (ptr2 /
 * start2 / counts[2]: staged blobs, or the mapped host blobs read directly) through xs_native_expert_grouped into a
 * hit buffer, take the CPU's rows from mapped memory (zero where the GPU computed the entry), and add the hits in.
 * Every call is one launch on `stream`; a NULL stream is HIP's default stream and the call then synchronises.  Host
 * memory arguments are device-accessible pinned host memory (hipHostMalloc).  A wait meant to be released by this
 * same host thread needs a non-NULL stream: with NULL the call itself waits for the kernel, which then ends only at
 * its bound.  Paths relative to the reference repository, 32x-k/XeStrata-win.  Return codes and xs_last_error() are
 * include/xs_moe.h's.
 */
#ifndef XS_TIERS_H
#define XS_TIERS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Spin until *flag >= value (flag: mapped host memory the host writes), then an acquire at system scope so the work
 * after it on the stream sees what the host wrote before the flag.  Bounded: after limit_us microseconds of the
 * device's wall clock (0: 10 s; at most an hour) the wait gives up and, when `status` (device int32) is given, sets *status = 1.
 * Replaces wait_flag_ge (include/strata/kernels/verify_kernels.hpp:65; src/kernels/xe/verify_kernels.cpp:783-788),
 * which waits without a bound. */
int xs_wait_flag_ge(const uint32_t* flag, uint32_t value, int64_t limit_us, int32_t* status, void* stream);

/* dst[0, n) = src[0, n) with src in mapped host memory: 16-byte reads where both are 16-byte aligned.  Replaces
 * copy_i32_from_mapped (include/strata/kernels/elementwise.hpp:124; src/kernels/xe/elementwise.cpp:236-257). */
int xs_copy_i32_from_mapped(int32_t* dst, const int32_t* src, int64_t n, void* stream);

/* `rows` rows of `width` floats from mapped host memory, except the rows listed in hit_rows[0, *count) (device),
 * which get +0.0 (the entries the GPU computes itself).  width a multiple of 4, both pointers 16-byte aligned.
 * Replaces copy_rows_from_mapped (include/strata/kernels/elementwise.hpp:113-114; elementwise.cpp:196-215). */
int xs_copy_rows_from_mapped(float* dst, const float* src, int64_t rows, int64_t width, const int32_t* hit_rows,
                             const int32_t* count, void* stream);

/* *n (device) blobs of blob_bytes from src[k] (device aliases of mapped host blobs, or device addresses) into
 * dst + k * blob_bytes, 16 bytes a load; launched for a capacity of `cap` blobs (*n is clamped to it).  blob_bytes a
 * multiple of 16; the addresses 16-byte aligned.  Replaces fetch_blobs (include/strata/kernels/verify_kernels.hpp:105;
 * src/kernels/xe/verify_kernels.cpp:1051-1058). */
int xs_fetch_blobs(const unsigned long long* src, const int32_t* n, uint8_t* dst, int64_t blob_bytes, int cap,
                   void* stream);

/* ptr[k] = base + k * blob_bytes for k < *n (at most 128: the PCIe share's group capacity).  Replaces rebase_ptrs
 * (include/strata/kernels/verify_kernels.hpp:110; src/kernels/xe/verify_kernels.cpp:1060-1068). */
int xs_rebase_ptrs(unsigned long long* ptr, const int32_t* n, uint8_t* base, int64_t blob_bytes, void* stream);

/* parts[dst[h] * n_embd + i] += hit_out[dst[h] * n_embd + i] for h < *count (device; launched for `cap` hits): the
 * GPU's rows added into the parts the CPU left at zero there.  Replaces moe_hit_add
 * (include/strata/kernels/s2_expert_grouped.hpp:94-95; src/kernels/xe/s2_expert_grouped.cpp:913-925). */
int xs_moe_hit_add(float* parts, const float* hit_out, const int32_t* dst, const int32_t* count, int64_t cap,
                   int64_t n_embd, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XS_TIERS_H */
