/* CPU oracle for the INT8 NHWC vision path: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests, the smoke check and the CPU-baseline leg of the benchmark may
 * load this library, and only as the checker. The GPU library never links it
 * and has no CPU fallback.
 */
#ifndef UQ_ORACLE_H
#define UQ_ORACLE_H
#include <stdint.h>

/* TFLite double-rounding requantisation, qnn.c:61-83. */
int32_t uqo_scale(int32_t v, int32_t m, int32_t shift);

/* Execute a plan (graph.h:15-17 layout) on `images` stacked inputs.
 * input:  images * input_bytes, output: images * output_bytes.
 * If snap_tensor < nt, that tensor's per-run contents (images * bytes for an
 * activation, bytes for a constant) are copied into snap_out.
 * Returns 0, or 10..19 for a plan this restatement cannot execute. */
int uqo_run(const void *plan, uint32_t len, const void *input, uint32_t images,
            void *output, uint32_t snap_tensor, void *snap_out);

#endif
