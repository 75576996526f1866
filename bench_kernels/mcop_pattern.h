/*
 * mcop_pattern.h -- C ABI of bench_kernels/libmcop_pattern.so: compute-free kernels with the HBM
 * access pattern of the operators' register-resident row kernels, plain streaming kernels (copy,
 * read-only, write-only) and an empty kernel. Measurement only, not part of the operator library:
 * they have no counterpart in the reference and compute nothing meaningful; bench.py builds and
 * times them beside the operators to give each operator's practical ceiling (and, for decode
 * shapes, its latency floor) on the GPU it runs on. Conventions as in include/mcop_norm.h
 * (device pointers, hipStream_t as void*, asynchronous, 0 = success).
 */
#ifndef MCOP_PATTERN_H
#define MCOP_PATTERN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  /* reads x, r (bf16 [rows, hidden]) and w (bf16 [hidden]); writes o0 (bf16), q (1 byte per
     element) and scales (fp32 [rows]): rms_norm_dynamic_per_token_quant with a residual */
  MCOP_PATTERN_ADD_NORM_QUANT = 0,
  /* reads x, r, w; writes o0, o1 (bf16; pass x and r to write in place): fused_add_rms_norm */
  MCOP_PATTERN_FUSED_ADD = 1,
  /* reads x, w and smooth (fp32 [hidden]); writes o0, o1 (bf16), q, scales: the SmoothQuant
     rms_norm_dynamic_per_token_quant with after_res and after_norm */
  MCOP_PATTERN_SMOOTH_QUANT = 2,
  /* reads x; writes o0 */
  MCOP_PATTERN_COPY = 3,
  /* reads x; writes practically nothing (a word of `scales` only where a data-dependent test of
     the loaded values holds, so every load is needed) */
  MCOP_PATTERN_READ = 4,
  /* writes o0 */
  MCOP_PATTERN_WRITE = 5,
  /* touches nothing: an empty kernel launched with the given shape's grid and workgroup size
     (the floor under any kernel of that launch shape); no tensor is needed */
  MCOP_PATTERN_EMPTY = 6,
  /* MCOP_PATTERN_ADD_NORM_QUANT in the operators' exact-row form: one row per workgroup and
     every lane in the row (vectors_per_lane * lanes_per_row == hidden / 8, lanes_per_row >=
     256), scalar row bases, no bounds tests -- the form the operator takes for such rows, e.g.
     decode rows of 5120 at two vectors over 320 lanes */
  MCOP_PATTERN_ADD_NORM_QUANT_EXACT = 7
};

enum { MCOP_PATTERN_E_INVALID = -1, MCOP_PATTERN_E_LAUNCH = -3 };

/* One launch of `pattern` over `rows` rows of `hidden` bf16 elements (a multiple of 8), with
 * the launch shape of the operator it models: `vectors_per_lane` (1, 2, 4 or 8 16-byte vectors)
 * and `lanes_per_row` (a multiple of 64 holding the row; rows narrower than 256 lanes are packed
 * several per workgroup, as the operators do). `lds_bytes` (0 to 163840) of dynamic LDS per
 * workgroup, unused by the kernel, caps how many workgroups share a CU (160 KiB of LDS each),
 * to model an operator's occupancy. Tensors the pattern does not touch may be NULL. */
int mcop_pattern(int pattern, const void* x, const void* r, const void* w, const float* smooth,
                 void* o0, void* o1, void* q, float* scales, int64_t rows, int64_t hidden,
                 int vectors_per_lane, int lanes_per_row, int lds_bytes, void* stream);

/* Message of the last failed mcop_pattern call on this host thread. */
const char* mcop_pattern_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MCOP_PATTERN_H */
