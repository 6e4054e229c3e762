/*
 * backend.h — backend selection and the kernel vtable (the reference's
 * backend.h:13-52), extended with BACKEND_HIP.  Member order of KernelVTable
 * and BackendConfig is the reference's, so engine code compiled against
 * either header calls the same slots.
 */
#ifndef LLMRT_BACKEND_H
#define LLMRT_BACKEND_H

#include "types.h"

typedef enum {
  BACKEND_AUTO = -1,
  BACKEND_CPU = 0,
  BACKEND_CUDA = 1,
  BACKEND_HIP = 2, /* MI355X path: libgq_hip.so */
} BackendKind;

typedef struct Backend Backend;

typedef struct {
  void (*gemm_f32)(const Tensor *A, const Tensor *B, Tensor *C);
  void (*gemm_f32_nn)(const Tensor *A, const Tensor *B, Tensor *C);
  void (*rmsnorm)(const Tensor *input, const Tensor *weight, Tensor *output, float eps);
  void (*softmax_inplace)(Tensor *scores, int seq_len);
  void (*silu_inplace)(Tensor *x);
  void (*rope)(Tensor *q, Tensor *k, int pos, int head_dim);
  void (*residual_add)(Tensor *x, const Tensor *residual);
  void (*elemwise_mul)(Tensor *a, const Tensor *b);
  int (*matvec_q4k_f32)(const Tensor *W_q4k, const float *x, float *y);
  int (*matvec_q6k_f32)(const Tensor *W_q6k, const float *x, float *y);
  int (*matvec_q8_0_f32)(const Tensor *W_q8_0, const float *x, float *y);
} KernelVTable;

typedef struct {
  BackendKind kind;
  int threads;
  int device_id;
  int n_gpu_layers;
} BackendConfig;

Backend *backend_create(const BackendConfig *cfg);
void backend_destroy(Backend *b);
const KernelVTable *backend_kernels(const Backend *b);
BackendKind backend_kind(const Backend *b);
BackendConfig backend_config(const Backend *b);

#endif
