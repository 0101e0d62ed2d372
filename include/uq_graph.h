/* libuq_hip.so: the MI355X (gfx950) drop-in for the reference's graph ABI.
 *
 * Part 1 is the reference's own C ABI, symbol for symbol, with the same
 * argument meaning, plan format, validation rules and error codes:
 *   runtime/graph.h:39-45   ug_load, ug_run, ug_input_bytes, ug_output_bytes,
 *                           ug_snapshot, ug_profile
 *   runtime/graph.c:425-437 ug_stream_begin, ug_stream_end
 * A host or test that dlopen()s the reference's native library (the
 * UNOQ_NATIVE_LIBRARY pattern of tests/test_residual_add.py:62-69) binds this
 * library unchanged.
 *
 * Part 2 is an additive batch extension with no reference counterpart: it runs
 * a plan on many stacked images (the reference plan format caps one plan at a
 * 16 MiB arena and 2e9 MACs, graph.h:7-9), optionally on device-resident
 * buffers so the caller's data stays in HBM.
 *
 * Plan format (graph.h:15-17): 32-byte header, 48-byte tensor records, 32-byte
 * op records, arena. Little endian. One model per process; not reentrant
 * (graph.c:4-9 keeps the same single global model).
 */
#ifndef UQ_GRAPH_H
#define UQ_GRAPH_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- Part 1: reference ABI -------------------------------------------- */

/* graph.h:39, graph.c:50-262. Copies and validates the plan (the caller keeps
 * the blob), replacing any loaded model. Returns 0 or:
 *   10 blob missing/short  11 header  12 length  13 tensor record
 *   14 constant input      15 operand/use-before-def  16 matmul params
 *   17 add/mul operands    18 op validation  19 unknown op  20 work > 2e9
 *   21 output undefined    25 v3 lifetime overlap
 *   24 no usable GPU (the reference's "worker unavailable" code)
 * Plans that the reference accepts but that use ops outside the INT8 path
 * return 19: the float ops (codes 1-4, 7, 8, 11-13) and the u8 x i8 integer
 * matmuls (6, 9). Every other op code the reference runs loads and runs
 * here: 5, 10, 14-28 (copy, transpose, conv, depthwise, pool, table
 * softmax, add, pack, concat, resize, LUT, pad, mean, mul, slice, bmm,
 * softmax). */
int ug_load(const void *plan, uint32_t len);

/* graph.h:40, graph.c:438-448. Synchronous single-image run from host memory.
 * ni/no must equal ug_input_bytes()/ug_output_bytes(), else 22. A GPU error
 * returns 24 and clears the loaded model (reload required), as graph.c does. */
int ug_run(const void *input, uint32_t ni, void *output, uint32_t no);

/* graph.h:41-42, graph.c:263-264: per-image byte sizes, 0 when not loaded. */
uint32_t ug_input_bytes(void);
uint32_t ug_output_bytes(void);

/* graph.h:44, graph.c:265-268. Tensor contents after the last run (image 0
 * of a batch run); bytes must equal the tensor's size, else 22. */
int ug_snapshot(uint32_t tensor, void *out, uint32_t bytes);

/* graph.h:45, graph.c:269-284. command 0 disable, 1 reset+enable, 2 read.
 * Counters: [0] runs, [1] total ticks, [2+i] ticks of op i. Ticks are GPU
 * nanoseconds from the first start to the last end of an op's kernels (HIP
 * events stamped by the launches themselves). bytes = 514*8, or 130*8
 * when the plan has at most 128 ops. */
int ug_profile(uint32_t command, void *out, uint32_t bytes);

/* graph.c:425-437. Accepted for ABI compatibility; GPU runs need no frame
 * worker. Same return codes: begin 24 if already active, 22 if not loaded. */
int ug_stream_begin(void);
int ug_stream_end(void);

/* ---- Part 2: batch extension (no reference counterpart) ---------------- */

/* Run the loaded plan on `images` images stacked on the leading dimension:
 * input images*ug_input_bytes() bytes, output images*ug_output_bytes().
 * Returns 22 on size mismatch or when not loaded, 24 on a GPU error. */
int ug_run_batch(const void *input, uint64_t ni, void *output, uint64_t no, uint32_t images);

/* The same on device-resident buffers (pointers from ug_device_alloc or any
 * HIP allocation on the current device). ug_run_device returns when the
 * output is complete; ug_enqueue_device only enqueues and ug_synchronize
 * waits for all enqueued work. A batch of at least 128 images runs as two
 * image slices, one on the library stream and one on a side stream; the side
 * stream is left unjoined while identical batches (same images, input and
 * output buffers) follow one another, and any other entry point joins it
 * before it touches the library stream, results or buffers. Between an
 * enqueue and the next synchronize the caller must not free or reuse the
 * buffers. While profiling (ug_profile 1) each profiled batch counts as one
 * run; its times are added by ug_synchronize, by the next enqueue or by a
 * counter read. */
int ug_run_device(const void *d_input, void *d_output, uint32_t images);
int ug_enqueue_device(const void *d_input, void *d_output, uint32_t images);
int ug_synchronize(void);

/* All images of a tensor after the last run: bytes = images * tensor bytes
 * (for constants: the tensor bytes). Activation snapshots return 22 after a
 * ug_enqueue_device_noalloc run and once a caller buffer the last run was
 * bound to has been freed with ug_device_free. After a device-buffer run
 * (ug_run_device, ug_enqueue_device) the output of a stem conv that ran
 * fused with the 3x3 conv after it (it read the caller's input buffer and
 * was never written) returns 22 too, from ug_snapshot as well; after a
 * host-buffer run it is rebuilt from the library's copy of the input. */
int ug_snapshot_images(uint32_t tensor, void *out, uint64_t bytes);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): ug_enqueue_device with every intermediate activation
 * laid out in the library's static per-GPU scratch (UG_NOALLOC_SCRATCH_BYTES,
 * 64 MiB, held by each GPU until the process ends) instead of buffers the
 * library allocates; it calls no allocator. Returns 22 when not loaded, on a
 * null buffer or zero images, or when the plan's activations for `images`
 * (each tensor's images * bytes, 256-byte aligned) exceed the scratch; 24 on
 * a GPU error. Results equal ug_enqueue_device's; ug_synchronize waits for
 * them. Every call on one GPU uses the same scratch, whose contents the last
 * call leaves behind: calls that overlap on one GPU (from other threads, or
 * other streams than the library's) race. Snapshots of activations are not
 * available after it (22). */
#define UG_NOALLOC_SCRATCH_BYTES (64u << 20)
int ug_enqueue_device_noalloc(const void *d_input, void *d_output, uint32_t images);

/* Device buffer helpers for callers without their own HIP allocator. */
void *ug_device_alloc(uint64_t bytes);
int ug_device_free(void *d);
int ug_device_upload(void *d_dst, const void *src, uint64_t bytes);
int ug_device_download(void *dst, const void *d_src, uint64_t bytes);

/* Number of ops of the loaded plan, 0 when not loaded. */
uint32_t ug_op_count(void);

/* Host-buffer batch with transfers overlapped with compute: the batch runs in
 * chunks of `chunk` images (0: chunks of max(256, images/8) images from 512
 * images on, unchunked below); chunk k's host-to-device copy, chunk k-1's
 * kernels and chunk k-2's copy back proceed on three streams at once.
 * Same sizes and codes as ug_run_batch. Afterwards snapshots hold the last
 * chunk. Host buffers from ug_host_alloc transfer by DMA at full rate;
 * ordinary pageable memory also works, with less overlap. */
int ug_run_batch_pipelined(const void *input, uint64_t ni, void *output, uint64_t no, uint32_t images, uint32_t chunk);

/* Pinned host memory for the host-buffer entry points (NULL without a GPU). */
void *ug_host_alloc(uint64_t bytes);
int ug_host_free(void *p);

/* ---- Part 3: .uqmodel bundles (src/unoq_dsp/bundle.py:18-19, 84-141) ---- */

/* Check a bundle image (header, lengths, SHA-256 of manifest || plan, plan
 * magic and version 2/3) and return a pointer into it at the plan. Returns 0,
 * 30 for a bad header or length, 31 for a checksum mismatch, 32 for a plan the
 * bundle format does not admit. The Python loader raises InvalidBundle in
 * these cases; the C ABI reports them as codes above the loader's range. */
int ug_bundle_plan(const void *file, uint64_t len, const void **plan, uint32_t *plan_len);

/* ug_bundle_plan, then ug_load on the plan (returning ug_load's code). A
 * bundle error leaves any previously loaded model in place, as the Python
 * loader fails before reaching the runtime. */
int ug_load_bundle(const void *file, uint64_t len);

/* SHA-256 of a byte string (FIPS 180-4), the bundle checksum. */
void uq_sha256(const void *data, uint64_t len, uint8_t out[32]);

/* ---- Part 4: the reference's host session ABI (runtime/bridge.c) -------- */
/* The entry points the reference's Python HardwareSession binds
 * (src/unoq_dsp/transport.py:35-43), with the same argument checks and codes.
 * One session at a time over the library's single model. */

/* bridge.c:99-125. Load the plan and open a session; NULL on failure with
 * *error = 1 (bad arguments: null plan, more than 17 MiB, pipeline not 0/1),
 * 1001 (a session is open), 1002 (allocation), the ug_load code, or 0 when
 * the plan's input or output exceeds 4 MiB. pipeline 0 is the blocking call
 * per image ("rpc"); 1 ("mailbox") replays one captured graph of the whole
 * plan through pinned staging buffers, for the lowest per-call latency. */
void *ug_open_mode(const void *plan, uint32_t bytes, int pipeline, int *error);

/* bridge.c:126: ug_open_mode(plan, bytes, 0, error). */
void *ug_open(const void *plan, uint32_t bytes, int *error);

/* bridge.c:148-185. One image: 1003 on a null session/buffer or sizes other
 * than the model's; otherwise ug_run's codes. */
int ug_infer(void *session, const void *input, uint32_t ni, void *output, uint32_t no);

/* bridge.c:70-80. Ends the session (the model stays loaded); null is a no-op. */
void ug_close(void *session);

/* bridge.c:127-130. ug_snapshot through the session; 1003 in pipeline mode or
 * for a null session/buffer or bytes outside 1 .. 4 MiB. */
int ug_snapshot_tensor(void *session, uint32_t index, void *out, uint32_t bytes);

/* bridge.c:134-147. ug_profile through the session; 1003 for a null session or
 * buffer, a command above 2, or bytes other than 130*8 or 514*8. */
int ug_profile_control(void *session, uint32_t command, void *out, uint32_t bytes);

#ifdef __cplusplus
}
#endif
#endif
