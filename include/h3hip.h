// h3hip: the C ABI of the MI355X (gfx950) attention path.
//
// It replaces the part of h3metal's C API that the DiT attention path uses
// (reference: src/capi.h:17-74, implemented in src/capi.mm). Names, argument
// meaning and the error convention are the reference's: every call that can
// fail returns NULL / a negative value / -1 and leaves a message for
// h3_last_error() on the calling thread. Plain C types only (no torch, no HIP
// types), so ctypes (h3metal_amd/gpu.py) and any other FFI can bind it.
//
// What differs from the reference, and why:
//  * Kernels are compiled ahead of time for gfx950 and looked up by name in a
//    launch table; h3_pipeline() takes the same (file, fn, "K=V;...") triple but
//    selects a precompiled specialisation instead of compiling source text.
//  * Buffers are device memory (hipMalloc, zero-filled like the reference's
//    shared buffers, src/metal_rt.mm:80-83). There is no unified CPU view, so
//    h3_buffer_contents() returns NULL and h3_buffer_read()/h3_buffer_write()
//    copy instead.
//  * A dispatch's grid/threads are chosen by the kernel's launcher from its
//    parameter block (the gfx950 tiles are not the Metal ones); a zero grid is
//    the normal call and a non-zero one is accepted and ignored.
//  * Work runs on one HIP stream per context in submission order. h3_commit()
//    only marks a point; h3_wait() synchronises and returns GPU seconds measured
//    with HIP events on that stream.
// The file-mapping half of the reference API (h3_map_*) is not on this path and
// is not provided.
#ifndef H3HIP_H
#define H3HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct h3_ctx h3_ctx;

// A buffer handle (opaque) and a byte offset into it. Reference: src/capi.h:21-24.
typedef struct {
  void *buf;
  uint64_t offset;
} h3_arg;

// Message of the last failed call on this thread, "" if none. Reference: src/capi.h:27.
const char *h3_last_error(void);

// Opens device 0 (the current HIP device) and creates the context's stream.
// kernel_dir is accepted for signature compatibility and unused (kernels are
// built in). Reference: src/capi.h:29-33.
h3_ctx *h3_open(const char *kernel_dir);
void h3_close(h3_ctx *ctx);
const char *h3_device_name(h3_ctx *ctx);
uint64_t h3_recommended_working_set(h3_ctx *ctx);  // free device memory at open time
uint64_t h3_max_buffer_length(h3_ctx *ctx);        // total device memory

// Zero-filled device buffers. Reference: src/capi.h:35-39.
void *h3_buffer(h3_ctx *ctx, uint64_t bytes);
void *h3_buffer_contents(void *buf);  // always NULL here: device memory has no CPU view
uint64_t h3_buffer_length(void *buf);
void h3_buffer_release(void *buf);
// Additions (no reference counterpart; the reference reads shared memory directly,
// h3metal/gpu.py:137-147): synchronous copies that first drain the context's stream.
// Return 0 on success, -1 on a bad range or a copy failure.
int h3_buffer_write(h3_ctx *ctx, void *buf, uint64_t offset, const void *src, uint64_t bytes);
int h3_buffer_read(h3_ctx *ctx, void *buf, uint64_t offset, void *dst, uint64_t bytes);
// The device address of a buffer (for callers that launch their own HIP work).
void *h3_buffer_device(void *buf);
// Addition (no reference counterpart; a Metal caller copies through shared memory): copies `bytes` from `src` at
// `src_offset` to `dst` at `dst_offset` on the context's stream, in order with the dispatches (asynchronous;
// timed by h3_wait and, in profile mode, recorded like a dispatch). Returns 0, or -1 on a bad range.
int h3_buffer_copy(h3_ctx *ctx, void *dst, uint64_t dst_offset, void *src, uint64_t src_offset, uint64_t bytes);

// Looks up kernel `fn` of module `file` specialised by macros "NAME=value;...".
// Modules: "attention" (fn "attention", "attention_scores") and "ops" (fn
// "qk_norm_rope", "rot_q8") and "gemm" (fn "gemm"; macro WFMT selects the weight
// format as in kernels/gemm.metal:1-40: 1 q8, 4 f16, 5 bf16, 6 h8; other formats
// return NULL); the reference's "attention.metal"/"ops.metal"/"gemm.metal" names are
// also accepted. NULL (with h3_last_error) for an unknown kernel or an unsupported
// specialisation. The handle is owned by the context. Reference: src/capi.h:54-57.
void *h3_pipeline(h3_ctx *ctx, const char *file, const char *fn, const char *macros);
int h3_pipeline_max_threads(void *pso);

// Launches one kernel on the context's stream. bufs[i] binds buffer index i
// (a NULL buf leaves it unbound); params (params_len bytes) is the kernel's
// parameter block, logically at index params_index. Returns 0, or -1 with
// h3_last_error for a missing pipeline, a missing required buffer, a parameter
// block of the wrong size, shapes the kernel does not support, an access that
// would fall outside a bound buffer, or a launch failure. Reference: src/capi.h:59-63.
int h3_dispatch(h3_ctx *ctx, void *pso, const uint32_t grid[3], const uint32_t tg[3], const h3_arg *bufs,
                int nbufs, const void *params, uint32_t params_len, int params_index, uint32_t tg_mem_bytes);

// h3_dispatch without any allocation (no reference counterpart: for callers that cannot allocate device
// memory, such as code under HIP graph capture or a serving loop that forbids it). Same arguments, checks and
// kernels as h3_dispatch, but the scratch memory the kernels use (the attention tail split's partial states,
// the h8 GEMM's widened weights) is a fixed 32 MiB array compiled into the library, one per GPU and held until
// the process ends, instead of the context's workspace; it calls no hipMalloc, hipFree, event creation or other
// allocating routine (per-dispatch profiling is skipped). Work that needs more scratch than 32 MiB: the
// attention split shrinks to fit (down to none), an h8 GEMM with N * K * 2 > 32 MiB fails with a message.
// Calls on one GPU share the array: dispatches through this entry point that may run at the same time on one
// GPU (different contexts or streams) race; on one context's stream they are ordered. Nothing in the array
// needs to start at zero (every kernel writes what it later reads).
int h3_dispatch_static(h3_ctx *ctx, void *pso, const uint32_t grid[3], const uint32_t tg[3], const h3_arg *bufs,
                       int nbufs, const void *params, uint32_t params_len, int params_index, uint32_t tg_mem_bytes);

// Scratch memory of the dispatches (addition, no reference counterpart: Metal
// kernels there keep no scratch). h3_open reserves what the attention's tail
// split needs at most, so h3_dispatch never allocates or synchronises; the h8
// GEMM's widened weights (N * K * 2 bytes) need an explicit h3_reserve_workspace
// first when they exceed it. h3_reserve_workspace drains the stream, then grows
// the buffer (never shrinks it); 0 or -1. h3_workspace_bytes: the current size.
int h3_reserve_workspace(h3_ctx *ctx, uint64_t bytes);
uint64_t h3_workspace_bytes(h3_ctx *ctx);

// Reference: src/capi.h:65-74.
void h3_commit(h3_ctx *ctx);
// Waits for all work on the stream. Returns the GPU seconds between the first
// dispatch after the previous wait and now (HIP events on the stream), or -1.0
// if the stream reported an error.
double h3_wait(h3_ctx *ctx);
// With profiling on, each dispatch is bracketed by its own pair of HIP events;
// h3_profile_take() returns their durations (seconds) since the last call.
void h3_set_profile(h3_ctx *ctx, int on);
int h3_profile_take(h3_ctx *ctx, double *seconds, int max);

#ifdef __cplusplus
}
#endif

#endif
