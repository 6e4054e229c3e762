/*
 * hip_backend.c — BACKEND_HIP behind the reference's KernelVTable
 * (backend.h:20-39), the MI355X counterpart of cuda_backend.c:43-81.
 *
 * Dense ops (gemm, rmsnorm, softmax, silu, rope, residual, elemwise) stay
 * bound to the CPU backend's kernels, exactly as the CUDA backend binds them
 * (cuda_backend.c:227-234): a HIP backend owns a CPU backend for those and
 * for CPU-resident layers.  The three quantised matvec slots dispatch on
 * Tensor.device_residency (cuda_backend.c:35-40): 0 -> the CPU kernel,
 * 1 -> libgq_hip.so on Tensor.d_data with the host x / y contract and the
 * reference's return codes.  Unlike the CUDA backend, Q6_K and Q8_0 also run
 * on the device (the CUDA vtable leaves them on the CPU, cuda_backend.c:72-73).
 *
 * The vtable functions carry no backend argument, so the live HIP backend is
 * found through one file-scope pointer set by backend_hip_create — the same
 * single-backend-per-process model the reference's g_threadpool global uses
 * (kernels_cpu.c:20-24).  Not thread-safe, like the reference engine.
 */
#include "backend_internal.h"
#include "hip_backend.h"

#include <stdlib.h>

#include "../../include/gq_hip.h"

typedef struct {
  gq_ctx *ctx;
  Backend *cpu; /* dense ops + CPU-resident quant matvecs */
} HipImpl;

static HipImpl *g_hip; /* the live HIP backend (see the file comment) */

static int hip_matvec(int dtype, DataType want, int (*cpu_fn)(const Tensor *, const float *, float *),
                      const Tensor *W, const float *x, float *y) {
  if (!W || !x || !y) return -1;
  if (W->device_residency != 1 || !W->d_data) return cpu_fn ? cpu_fn(W, x, y) : -1;
  if (!g_hip || W->dtype != want || W->ndim != 2) return -1;
  return gq_hip_matvec(g_hip->ctx, dtype, W->d_data, W->shape[0], W->shape[1], W->byte_size, x, y);
}

static int hip_matvec_q4k(const Tensor *W, const float *x, float *y) {
  return hip_matvec(GQ_Q4_K, DTYPE_Q4_K, g_hip ? g_hip->cpu->kernels.matvec_q4k_f32 : NULL, W, x, y);
}

static int hip_matvec_q6k(const Tensor *W, const float *x, float *y) {
  return hip_matvec(GQ_Q6_K, DTYPE_Q6_K, g_hip ? g_hip->cpu->kernels.matvec_q6k_f32 : NULL, W, x, y);
}

static int hip_matvec_q8_0(const Tensor *W, const float *x, float *y) {
  return hip_matvec(GQ_Q8_0, DTYPE_Q8_0, g_hip ? g_hip->cpu->kernels.matvec_q8_0_f32 : NULL, W, x, y);
}

Backend *backend_hip_create(const BackendConfig *cfg) {
  if (!cfg || g_hip) return NULL; /* one HIP backend per process */
  if (gq_hip_device_count() <= cfg->device_id) return NULL;
  gq_ctx *ctx = gq_hip_create(cfg->device_id);
  if (!ctx) return NULL;
  BackendConfig cpu_cfg = *cfg;
  cpu_cfg.kind = BACKEND_CPU;
  Backend *cpu = backend_cpu_create(&cpu_cfg);
  Backend *b = (Backend *)calloc(1, sizeof(Backend));
  HipImpl *impl = (HipImpl *)calloc(1, sizeof(HipImpl));
  if (!cpu || !b || !impl) {
    if (cpu) backend_cpu_destroy(cpu);
    free(b);
    free(impl);
    gq_hip_destroy(ctx);
    return NULL;
  }
  impl->ctx = ctx;
  impl->cpu = cpu;
  b->cfg = *cfg;
  b->cfg.kind = BACKEND_HIP;
  b->kernels = cpu->kernels;
  b->kernels.matvec_q4k_f32 = hip_matvec_q4k;
  b->kernels.matvec_q6k_f32 = hip_matvec_q6k;
  b->kernels.matvec_q8_0_f32 = hip_matvec_q8_0;
  b->impl = impl;
  g_hip = impl;
  return b;
}

void backend_hip_destroy(Backend *b) {
  if (!b) return;
  HipImpl *impl = (HipImpl *)b->impl;
  if (impl) {
    if (g_hip == impl) g_hip = NULL;
    gq_hip_destroy(impl->ctx); /* frees every device weight and buffer */
    backend_cpu_destroy(impl->cpu);
    free(impl);
  }
  free(b);
}

struct gq_ctx *hip_backend_context(const Backend *b) {
  if (!b || b->cfg.kind != BACKEND_HIP || !b->impl) return NULL;
  return ((HipImpl *)b->impl)->ctx;
}

int hip_backend_upload(Backend *b, Tensor *t) {
  gq_ctx *ctx = hip_backend_context(b);
  if (!t) return -1;
  if (!ctx || !t->data || !t->byte_size ||
      (t->dtype != DTYPE_Q4_K && t->dtype != DTYPE_Q6_K && t->dtype != DTYPE_Q8_0)) {
    t->device_residency = 0;
    return -1;
  }
  void *d = gq_hip_upload_weight(ctx, t->data, t->byte_size);
  if (!d) {
    t->device_residency = 0;
    return -1;
  }
  t->d_data = d;
  t->device_residency = 1;
  return 0;
}

int hip_backend_finish(Backend *b) {
  gq_ctx *ctx = hip_backend_context(b);
  return ctx ? gq_hip_sync(ctx) : -1;
}
