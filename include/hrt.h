/*
 * hrt — the C-ABI device runtime of the MI355X "vk" PrivateUse1 backend.
 *
 * This is the boundary between the PyTorch shim (C++) and the HIP runtime plus the hand-written gfx950
 * kernels.  It replaces the reference's Rust/Vulkan runtime `vkrt`, whose C ABI is
 * `csrc/vkrt.h:6-32` (implemented at `vkrt/src/lib.rs:975-1244`).  Every function here has the same
 * argument meaning, the same return convention and the same error behaviour as its `vkrt_*` counterpart:
 *
 *   - status-returning calls return 0 on success and -1 on failure;
 *   - value-returning calls return 0 on failure;
 *   - on failure the reason is kept in a process-wide "last error" string (`hrt_last_error`).
 *
 * Memory model: device memory is carved out of hipMalloc'ed slabs; an address returned by `hrt_alloc`
 * is a plain device pointer (it becomes `Tensor::data_ptr()`), so any address inside a live block
 * (a view with a storage offset) may be passed to the transfer calls.  All kernels and copies run in
 * order on ONE HIP stream owned by the runtime; the host only waits at `hrt_download`,
 * `hrt_synchronize`, when a dedicated block is freed and in `hrt_empty_cache`.
 *
 * Thread safety: every call is serialized by one runtime mutex (as `vkrt/src/lib.rs:139, 958-962`).
 */
#ifndef HRT_H_
#define HRT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Initialise the runtime (idempotent): select the device (env HRT_DEVICE: an index, or a case-insensitive
 * substring of a device name, the lowest-numbered match winning; default 0; no match is an error that
 * lists the devices), create the stream, register the kernels.  0 = ok, -1 = error.  Replaces `vkrt_init`
 * (csrc/vkrt.h:7). */
int hrt_init(void);

/* Copy the last error message into buf (NUL-terminated, at most cap bytes) and return its full
 * length.  Replaces `vkrt_last_error` (csrc/vkrt.h:8). */
size_t hrt_last_error(char* buf, size_t cap);

/* Device name (e.g. "AMD Instinct MI355X (gfx950)"); returns the full length.
 * Replaces `vkrt_device_name` (csrc/vkrt.h:9). */
size_t hrt_device_name(char* buf, size_t cap);

/* Largest single allocation in bytes.  Replaces `vkrt_max_alloc` (csrc/vkrt.h:10). */
uint64_t hrt_max_alloc(void);

/* Bytes currently handed out (rounded to the 512-byte block granularity).
 * Replaces `vkrt_live_bytes` (csrc/vkrt.h:11). */
uint64_t hrt_live_bytes(void);

/* out[0] = budget (bytes this process may still reach: device free memory + own reservation),
 * out[1] = device memory in use (all processes), out[2] = device total.  0 = ok.
 * Replaces `vkrt_memory_info` (csrc/vkrt.h:12). */
int32_t hrt_memory_info(uint64_t* out);

/* High-water mark of hrt_live_bytes since the last reset.  Replaces `vkrt_peak_live_bytes`
 * (csrc/vkrt.h:13) and `vkrt_reset_peak_live_bytes` (csrc/vkrt.h:14). */
uint64_t hrt_peak_live_bytes(void);
void hrt_reset_peak_live_bytes(void);

/* Cap on reserved (slab) bytes, 0 = unlimited; simulates a smaller device.  A cap also shrinks the
 * slab size to cap/8 clamped to [64 MiB, 256 MiB].  Replaces `vkrt_set_memory_limit` (csrc/vkrt.h:15). */
void hrt_set_memory_limit(uint64_t bytes);

/* Allocate size bytes (512-byte aligned) and return the device address, 0 on failure (size 0, above
 * hrt_max_alloc, over the memory limit, or out of device memory after one empty_cache retry).
 * Replaces `vkrt_alloc` (csrc/vkrt.h:16). */
uint64_t hrt_alloc(uint64_t size);

/* Free an address returned by hrt_alloc.  Unknown addresses and double frees are rejected (-1).
 * Replaces `vkrt_free` (csrc/vkrt.h:17). */
int hrt_free(uint64_t addr);

/* Host -> device, device -> host, device -> device copies of n bytes.  The whole range must lie inside
 * one live block (-1 otherwise: out-of-range and unknown addresses are rejected, never touched).
 * upload/download return after the data has arrived; copy_d2d is queued on the stream.
 * Replace `vkrt_upload`, `vkrt_download`, `vkrt_copy_d2d` (csrc/vkrt.h:18-20). */
int hrt_upload(uint64_t dst, const void* src, uint64_t n);
int hrt_download(void* dst, uint64_t src, uint64_t n);
int hrt_copy_d2d(uint64_t dst, uint64_t src, uint64_t n);

/* Pinned (page-locked) host memory and asynchronous transfers — the block-swap path (sd-scripts' H2D
 * block offloader streams frozen weights from host to device every step; the reference serves its
 * `non_blocking` copies from pageable memory with synchronous transfers, csrc/shim.cpp:195-198, and has
 * no function of this kind).
 * hrt_host_alloc: `bytes` of pinned host memory (hipHostMalloc), returned as an address, 0 on failure.
 * hrt_host_free: releases it; the memory is reused or returned to the driver only after every transfer
 *   queued before the call has finished, so a buffer may be freed right after an asynchronous copy.
 * hrt_host_is_pinned: 1 if p lies inside a live block from hrt_host_alloc, else 0.
 * hrt_upload_async: queues a host -> device copy from pinned memory on the runtime's copy stream and
 *   returns at once.  The copy starts after all work queued before the call (so it never overwrites data
 *   earlier kernels still read), and the first later kernel or transfer that touches the destination
 *   waits for it; work on other memory overlaps the copy.  src must lie in one pinned block (-1 otherwise).
 * hrt_download_async: queues a device -> host copy into pinned memory in stream order and returns at once;
 *   the data is valid after hrt_synchronize. */
uint64_t hrt_host_alloc(uint64_t bytes);
int hrt_host_free(uint64_t ptr);
int hrt_host_is_pinned(const void* p);
int hrt_upload_async(uint64_t dst, const void* src, uint64_t n);
int hrt_download_async(void* dst, uint64_t src, uint64_t n);

/* Kernel id for a registered kernel name, -1 if unknown.  Names follow the reference's `op_dtype`
 * convention (tools/gen_shaders.py:155-185), e.g. "dq8_bf16", "mm_bf16", "softmax_fwd_f32".
 * The argument block of each kernel is declared in hrt_ops.h.  Replaces `vkrt_kernel_index`
 * (csrc/vkrt.h:21). */
int hrt_kernel_index(const char* name);

/* Queue kernel `kernel` with the argument block args[0..len).  len must equal the kernel's argument
 * size (checked, as `vkrt/src/lib.rs:922-927`).  Raw kernels (only "add_f32") take their workgroup
 * grid from gx/gy/gz; every operator kernel sizes its own grid from its arguments, and for those the
 * caller passes gx = gy = gz = 0 (anything else is rejected).  Asynchronous: returns once queued.
 * Replaces `vkrt_dispatch` (csrc/vkrt.h:22). */
int hrt_dispatch(uint32_t kernel, const void* args, uint32_t len, uint32_t gx, uint32_t gy, uint32_t gz);

/* Queue n operator kernels in order, each exactly as hrt_dispatch(kernels[i], args[i], lens[i], 0, 0, 0).
 * Returns 0 when all are queued; at the first rejected one it stops and returns -(i + 1) with the error
 * set (the ones before it stay queued).  No counterpart function in the reference, whose runtime records
 * its dispatches into command buffers and submits them together (vkrt/src/lib.rs:542-561): this is the
 * batched launch for HIP, one call for a sequence of launches, so that the caller's per-call cost (a
 * Python binding, for instance) does not stall the stream between short kernels. */
int hrt_dispatch_batch(const uint32_t* kernels, const void* const* args, const uint32_t* lens, uint32_t n);

/* Wait until all queued work has finished.  Replaces `vkrt_synchronize` (csrc/vkrt.h:23). */
int hrt_synchronize(void);

/* Return fully idle slabs to the driver; returns how many.  Replaces `vkrt_empty_cache`
 * (csrc/vkrt.h:24). */
size_t hrt_empty_cache(void);

/* Bytes held in slabs (live + cached).  Replaces `vkrt_reserved_bytes` (csrc/vkrt.h:25). */
uint64_t hrt_reserved_bytes(void);

/* Number of live blocks / slabs.  Replace `vkrt_live_blocks`, `vkrt_slab_count` (csrc/vkrt.h:26-27). */
size_t hrt_live_blocks(void);
size_t hrt_slab_count(void);

/* API-misuse errors detected by the runtime (the reference counts Vulkan validation-layer messages;
 * HIP has no validation layer, so this counts rejected calls that would have touched invalid memory:
 * it stays 0 in a correct program).  Replaces `vkrt_validation_errors` (csrc/vkrt.h:28). */
size_t hrt_validation_errors(void);

/* Counters: 0 dispatch host ns, 1 dispatches, 2 transfer ns, 3 transfers, 4 kernel-table setup ns,
 * 5 uploaded bytes, 6 downloaded bytes, 7 ns spent waiting for the GPU.  Replaces `vkrt_stat`
 * (csrc/vkrt.h:29). */
uint64_t hrt_stat(uint32_t i);

/* With env HRT_PROFILE=1 every dispatch is timed with HIP events; this writes
 * "name\tms\tcount\n" lines sorted by total time, returns the full length.
 * Replaces `vkrt_profile_dump` (csrc/vkrt.h:30). */
size_t hrt_profile_dump(char* buf, size_t cap);

/* Matrix-core kernels available: bit0 = f16, bit1 = bf16 (MFMA on gfx950: always 3).
 * Replaces `vkrt_coop_caps` (csrc/vkrt.h:31). */
uint32_t hrt_coop_caps(void);

/* ---- Timing on the runtime's stream (no counterpart in csrc/vkrt.h) --------------------------------
 * Record HIP event `slot` (0..1023) on the runtime stream, and read the elapsed milliseconds between two
 * recorded slots (waits for the later one).  Used by bench.py so that kernel time is measured on the
 * stream the kernels actually run on.  0 / value >= 0 = ok, -1 = error. */
int hrt_event_record(uint32_t slot);
float hrt_event_elapsed_ms(uint32_t start_slot, uint32_t end_slot);

/* ---- HIP graphs on the runtime's stream (no counterpart in csrc/vkrt.h; the reference batches
 * recorded commands instead, vkrt/src/lib.rs:542-643) ---------------------------------------------------
 * Between hrt_graph_begin and hrt_graph_end every hrt_dispatch and hrt_copy_d2d is recorded into a HIP
 * graph instead of being executed; calls that would wait for the GPU (upload, download, synchronize,
 * freeing a dedicated block, empty_cache) and allocations that need a new slab fail while recording.
 * hrt_graph_end returns the graph id (>= 0, -1 on error); hrt_graph_launch queues one replay on the
 * runtime stream (asynchronous), hrt_graph_destroy releases it. */
int hrt_graph_begin(void);
int64_t hrt_graph_end(void);
int hrt_graph_launch(int64_t graph);
int hrt_graph_destroy(int64_t graph);

#ifdef __cplusplus
}
#endif

#endif /* HRT_H_ */
