/*
 * mcop_testing.h -- test and tuning hooks exported by libmcop_norm.so beside its operator entry
 * points (include/mcop_norm.h).  They are not operator interface and have no counterpart in the
 * reference: the tests, the host sanitizer driver and launch-shape sweeps bind them.
 * Conventions as in mcop_norm.h (device pointers, hipStream_t as void*, asynchronous, 0 = ok).
 */
#ifndef MCOP_TESTING_H
#define MCOP_TESTING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The clamp-and-convert step shared by every fp8 epilogue, elementwise:
 *   out[i] = e4m3fn(clamp(in[i] * mul, -448, 448))   (RNE; clamp with fmin/fmax semantics)
 * (the step the reference calls float_to_fp8,
 * op/vllm/quantization/fused_kernels/quant_conversions.cuh:23-28); exported so the hardware
 * conversion can be checked bit for bit against the OCP fp8 definition. */
int mcop_fp8_e4m3fn_from_f32(uint8_t* out, const float* in, int64_t n, float mul, void* stream);

/* Forces the launch shape of the row kernels for later calls made BY THE CALLING THREAD only,
 * for the tests that check results do not depend on the launch shape and for tuning sweeps.
 * Other threads keep the automatic choice. vectors_per_lane in {0,1,2,4,8,16}, lanes_per_row in
 * {0, 16, 32} or a multiple of 64 up to 1024; (0, 0) restores the automatic choice. A request
 * the row does not fit falls back to automatic. Results do not change, only speed. */
int mcop_debug_set_launch_override(int vectors_per_lane, int lanes_per_row);

/* Whether later calls made BY THE CALLING THREAD may run rows too wide for one workgroup's
 * registers on a split-row kernel (the row shared by several co-resident workgroups that
 * exchange partial sums through a device workspace; the default, enabled = 1) or always on the
 * operator's multi-pass kernel (enabled = 0), for the tests that check both kernels and for A/B
 * timing. Results do not change, only speed. */
int mcop_debug_set_split_rows(int enabled);

/* Makes the split-row launches of later calls made BY THE CALLING THREAD (on = 1) start with
 * their workspace's error word already set, as a timed-out exchange leaves it, so that every
 * exchange of the launch fails at once: the grid still drains, and every row's exchanged sum or
 * maximum is NaN (NaN scales; NaN outputs for the norms). For the test of that failure path;
 * on = 0 restores normal launches. Calls that take no split-row kernel are unaffected. */
int mcop_debug_fail_split_waits(int on);

#ifdef __cplusplus
}
#endif

#endif /* MCOP_TESTING_H */
