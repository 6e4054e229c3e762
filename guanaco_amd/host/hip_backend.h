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

/* Bind the whole model to the device after the loader's uploads
 * (loader.c:701-728): every layer's seven projections must be
 * device-resident or are uploaded here, the F32 norm weights, the embedding
 * and the LM head get device copies, the device KV cache is sized from
 * ModelConfig (θ 500000, kernels_cpu.c:408) and takes the host cache's
 * contents (a restored session's prefix).  After this, gq_hip_forward_token,
 * gq_hip_decode_loop and gq_hip_prefill run on hip_backend_context(b).
 * Returns 0, or -1 (the model stays on its CPU path). */
int hip_backend_bind_model(Backend *b, ModelWeights *mw, KVCache *kv);

/* The gpu_prefill slot (gpu_prefill.h:13-20, same signature): the prompt
 * through every layer on the device (gq_hip_prefill), then the new K/V rows
 * copied into the host cache so the engine's CPU decode (or kv_cache_save)
 * sees them.  Needs hip_backend_bind_model first.  Returns 0, or non-zero
 * for the CPU forward() fallback. */
int hip_backend_prefill(const Backend *backend, ModelWeights *model, KVCache *kv, Scratch *scr,
                        const int *token_ids, int n_tokens, int pos);

/* ---- engine and loader hooks (no Backend argument: the live HIP backend,
 * as the CUDA build's direct hooks use its global device state) ---- */

/* The loader's upload (cuda_upload_weight, loader.c:701-728): Q4_K, Q6_K and
 * Q8_0 go to the device (d_data, device_residency 1); anything else, or a
 * failure, leaves the tensor CPU-resident (device_residency 0), -1. */
int hip_upload_weight(Tensor *t);

/* 1 when a HIP backend is live and all seven projections of the layer are
 * device-resident (the IS_GPU_READY test of engine.c:324-328). */
int hip_layer_ready(const LayerWeights *lw);

/* One decode step (T = 1) of `layer` on the device, as engine.c:330-349 runs
 * cuda_transformer_layer_gpu: hidden (host, hidden_dim floats) in and out,
 * the new K/V row written to the device cache and to the host cache slabs.
 * Needs hip_backend_bind_model.  0, or non-zero for the CPU path. */
int hip_backend_layer(int layer, int pos, float *hidden, KVCache *kv);

/* After the CPU path appended T rows at pos of a device-resident layer (a
 * prompt, or a device error), copy them to the device cache
 * (cuda_sync_kv_cache, engine.c:394-405). */
int hip_backend_kv_sync(KVCache *kv, int layer, int pos, int T, int max_seq);

/* Wait for queued device work before a CPU layer (cuda_finish_layer). */
int hip_backend_sync(void);

#endif
