/*
 * backend_internal.h — the backend object shared by the backend units
 * (the reference's backend_internal.h:7-17), plus the HIP constructor pair.
 */
#ifndef LLMRT_BACKEND_INTERNAL_H
#define LLMRT_BACKEND_INTERNAL_H

#include "backend.h"

struct Backend {
  BackendConfig cfg;
  KernelVTable kernels;
  void *impl;
};

Backend *backend_cpu_create(const BackendConfig *cfg);
void backend_cpu_destroy(Backend *b);
Backend *backend_cuda_create(const BackendConfig *cfg);
void backend_cuda_destroy(Backend *b);
Backend *backend_hip_create(const BackendConfig *cfg);
void backend_hip_destroy(Backend *b);

#endif
