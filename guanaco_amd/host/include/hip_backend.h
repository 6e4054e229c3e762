/*
 * hip_backend.h — HIP-backend hooks the engine and loader call directly
 * (the CUDA build's direct hooks: cuda_upload_weight, loader.c:701-728;
 * cuda_transformer_layer_gpu, engine.c:315-351; cuda_finish_layer,
 * engine.c:317-322).
 */
#ifndef LLMRT_HIP_BACKEND_H
#define LLMRT_HIP_BACKEND_H

#include "backend.h"

struct gq_ctx;

/* Device context of a HIP backend (NULL for any other kind). */
struct gq_ctx *hip_backend_context(const Backend *b);

/* Upload a quantised weight: on success sets d_data and device_residency = 1
 * and returns 0; on failure leaves the tensor CPU-resident and returns -1
 * (the UPLOAD_IF_GPU fallback, loader.c:711-717). */
int hip_backend_upload(Backend *b, Tensor *t);

/* Wait for queued device work (cuda_finish_layer). */
int hip_backend_finish(Backend *b);

#endif
