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
 * Plans that the reference accepts but that use ops outside the INT8 vision
 * path (float ops, transposes, int8 softmax, mul, bmm) return 19. */
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
 * nanoseconds from HIP events on the library stream. bytes = 514*8, or 130*8
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
 * output is complete; ug_enqueue_device only enqueues on the library stream
 * and ug_synchronize waits for all enqueued work. Between an enqueue and the
 * next synchronize the caller must not free or reuse the buffers. */
int ug_run_device(const void *d_input, void *d_output, uint32_t images);
int ug_enqueue_device(const void *d_input, void *d_output, uint32_t images);
int ug_synchronize(void);

/* All images of a tensor after the last run: bytes = images * tensor bytes
 * (for constants: the tensor bytes). */
int ug_snapshot_images(uint32_t tensor, void *out, uint64_t bytes);

/* Device buffer helpers for callers without their own HIP allocator. */
void *ug_device_alloc(uint64_t bytes);
int ug_device_free(void *d);
int ug_device_upload(void *d_dst, const void *src, uint64_t bytes);
int ug_device_download(void *dst, const void *d_src, uint64_t bytes);

/* Number of ops of the loaded plan, 0 when not loaded. */
uint32_t ug_op_count(void);

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

#ifdef __cplusplus
}
#endif
#endif
