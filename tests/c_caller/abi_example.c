/*
 * abi_example.c -- a plain C caller of libmcop_norm.so (include/mcop_norm.h), as a C or C++
 * program that has no torch would use it: device memory from hipMalloc, a stream of its own
 * (hipStreamCreate, not the legacy default stream), raw device pointers into the entry points,
 * copies in and out on that stream, one synchronization at the end.  Each function runs one
 * operator over host buffers and returns MCOP_OK or the failing status, with the message in
 * `err`.  The GPU test tests/test_gpu_c_abi.py loads this file's shared library with ctypes and
 * compares the results with the CPU oracle bit for bit; INTEGRATION.md quotes it.
 *
 * Built by tests/c_caller/Makefile (gcc, against /opt/rocm/include/hip/hip_runtime_api.h).
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "mcop_norm.h"

/* Device buffers and the stream of one call; released by finish(). */
#define MAX_BUF 8
typedef struct {
  hipStream_t stream;
  void* dev[MAX_BUF];
  int n;
  char* err;
  size_t errlen;
  int rc;
} call_t;

static int hip_failed(call_t* c, hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  if (c->rc == MCOP_OK) {
    snprintf(c->err, c->errlen, "%s: %s", what, hipGetErrorString(e));
    c->rc = MCOP_E_LAUNCH;
  }
  return 1;
}

static int start(call_t* c, char* err, size_t errlen) {
  memset(c, 0, sizeof(*c));
  c->err = err;
  c->errlen = errlen;
  c->rc = MCOP_OK;
  if (errlen > 0) err[0] = '\0';
  return !hip_failed(c, hipStreamCreate(&c->stream), "hipStreamCreate");
}

/* A device buffer of `bytes`, filled from `host` (if not NULL) on the call's stream. */
static void* dev_buf(call_t* c, const void* host, size_t bytes) {
  void* d = NULL;
  if (c->rc != MCOP_OK || c->n == MAX_BUF) return NULL;
  if (hip_failed(c, hipMalloc(&d, bytes ? bytes : 1), "hipMalloc")) return NULL;
  c->dev[c->n++] = d;
  if (host != NULL &&
      hip_failed(c, hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, c->stream),
                 "hipMemcpyAsync H2D")) {
    return NULL;
  }
  return d;
}

static void to_host(call_t* c, void* host, const void* d, size_t bytes) {
  if (c->rc != MCOP_OK) return;
  hip_failed(c, hipMemcpyAsync(host, d, bytes, hipMemcpyDeviceToHost, c->stream),
             "hipMemcpyAsync D2H");
}

static void check_op(call_t* c, int rc) {
  if (c->rc == MCOP_OK && rc != MCOP_OK) {
    snprintf(c->err, c->errlen, "%s", mcop_last_error());
    c->rc = rc;
  }
}

static int finish(call_t* c) {
  if (c->stream != NULL) hip_failed(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  for (int i = 0; i < c->n; ++i) hip_failed(c, hipFree(c->dev[i]), "hipFree");
  if (c->stream != NULL) hip_failed(c, hipStreamDestroy(c->stream), "hipStreamDestroy");
  return c->rc;
}

/* H1: residual <- x + residual; x <- RMSNorm(residual) * w, in place (bf16). */
int example_fused_add_rms_norm(uint16_t* x, uint16_t* residual, const uint16_t* w, int64_t T,
                               int64_t H, float eps, char* err, size_t errlen) {
  call_t c;
  if (!start(&c, err, errlen)) return finish(&c);
  const size_t n = (size_t)(T * H) * 2;
  void* xd = dev_buf(&c, x, n);
  void* rd = dev_buf(&c, residual, n);
  void* wd = dev_buf(&c, w, (size_t)H * 2);
  if (c.rc == MCOP_OK) {
    check_op(&c, mcop_fused_add_rms_norm(xd, H, rd, wd, T, H, MCOP_BF16, eps, c.stream));
  }
  to_host(&c, x, xd, n);
  to_host(&c, residual, rd, n);
  return finish(&c);
}

/* H2: (residual add +) RMSNorm + per-token int8 or fp8 (bf16 in; residual may be NULL). */
int example_rms_norm_quant(void* q, int fp8, float* scales, const uint16_t* x, const uint16_t* w,
                           uint16_t* residual, int64_t T, int64_t H, float eps, char* err,
                           size_t errlen) {
  call_t c;
  if (!start(&c, err, errlen)) return finish(&c);
  const size_t n = (size_t)(T * H);
  void* qd = dev_buf(&c, NULL, n);
  void* sd = dev_buf(&c, NULL, (size_t)T * 4);
  void* xd = dev_buf(&c, x, n * 2);
  void* wd = dev_buf(&c, w, (size_t)H * 2);
  void* rd = residual != NULL ? dev_buf(&c, residual, n * 2) : NULL;
  if (c.rc == MCOP_OK) {
    check_op(&c, mcop_rms_norm_dynamic_per_token_quant(qd, fp8 ? MCOP_FP8_E4M3FN : MCOP_I8,
                                                       (float*)sd, xd, wd, NULL, rd, T, H,
                                                       MCOP_BF16, eps, c.stream));
  }
  to_host(&c, q, qd, n);
  to_host(&c, scales, sd, (size_t)T * 4);
  if (residual != NULL) to_host(&c, residual, rd, n * 2);
  return finish(&c);
}

/* H4: SmoothQuant RMSNorm + per-token quant (bf16 x and w, fp32 smooth; residual may be NULL),
 * writing after_res and after_norm. */
int example_rms_norm_smooth_quant(void* q, int fp8, float* scales, const uint16_t* x,
                                  const uint16_t* w, const float* smooth, uint16_t* after_res,
                                  uint16_t* after_norm, const uint16_t* residual, int64_t T,
                                  int64_t H, float eps, char* err, size_t errlen) {
  call_t c;
  if (!start(&c, err, errlen)) return finish(&c);
  const size_t n = (size_t)(T * H);
  void* qd = dev_buf(&c, NULL, n);
  void* sd = dev_buf(&c, NULL, (size_t)T * 4);
  void* xd = dev_buf(&c, x, n * 2);
  void* wd = dev_buf(&c, w, (size_t)H * 2);
  void* smd = dev_buf(&c, smooth, (size_t)H * 4);
  void* ard = dev_buf(&c, NULL, n * 2);
  void* and_ = dev_buf(&c, NULL, n * 2);
  void* rd = residual != NULL ? dev_buf(&c, residual, n * 2) : NULL;
  if (c.rc == MCOP_OK) {
    check_op(&c, mcop_rms_norm_smooth_quant(qd, fp8 ? MCOP_FP8_E4M3FN : MCOP_I8, (float*)sd, xd,
                                            wd, MCOP_BF16, smd, MCOP_F32, ard, and_, rd, T, H,
                                            MCOP_BF16, eps, 0u, c.stream));
  }
  to_host(&c, q, qd, n);
  to_host(&c, scales, sd, (size_t)T * 4);
  to_host(&c, after_res, ard, n * 2);
  to_host(&c, after_norm, and_, n * 2);
  return finish(&c);
}

/* H5: smooth-scale multiply + per-token int8 (bf16 in, fp32 smooth). */
int example_scale_dynamic_quant(int8_t* q, float* scales, const uint16_t* x, const float* smooth,
                                int64_t T, int64_t H, char* err, size_t errlen) {
  call_t c;
  if (!start(&c, err, errlen)) return finish(&c);
  const size_t n = (size_t)(T * H);
  void* qd = dev_buf(&c, NULL, n);
  void* sd = dev_buf(&c, NULL, (size_t)T * 4);
  void* xd = dev_buf(&c, x, n * 2);
  void* smd = dev_buf(&c, smooth, (size_t)H * 4);
  if (c.rc == MCOP_OK) {
    check_op(&c, mcop_scale_dynamic_quant((int8_t*)qd, (float*)sd, xd, (const float*)smd, T, H,
                                          c.stream));
  }
  to_host(&c, q, qd, n);
  to_host(&c, scales, sd, (size_t)T * 4);
  return finish(&c);
}
