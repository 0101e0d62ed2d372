// Host-side plumbing shared by the gfx950 kernel files (C++ only): every
// launch takes its stream and timing events from kernels.hip, so that image
// slices, per-op timing and the library's error state cover all kernels.
#ifndef UQK_INTERNAL_H
#define UQK_INTERNAL_H
#include <hip/hip_runtime.h>

// The stream of the next launch and, while an op is timed, the events its
// dispatch stamps (first launch of the op: start and stop; later: stop).
void uqk_next_launch(hipStream_t *stream, hipEvent_t *start, hipEvent_t *stop);
// Records a HIP error as the library's last error; returns it as an int.
int uqk_fail(hipError_t e);
// Image slices whose launches run side by side (launch-shape heuristics).
int uqk_slices_live(void);

#endif
