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

/* Bind the model to the device after the loader's uploads
 * (loader.c:701-728), tensor by tensor: each layer whose seven projections
 * the loader made device-resident runs on the device (with device copies
 * of its F32 norm weights); every other layer (past --n-gpu-layers, or with
 * an F32 projection) stays on the CPU path and nothing of it is uploaded.
 * The LM head joins when the loader put it on the device (a quantised head
 * with --n-gpu-layers > 0; an F32 head stays on the host), the embedding in
 * any dtype the device embeds (F32, Q8_0, Q4_K).  The device KV cache is
 * sized from ModelConfig (θ 500000, kernels_cpu.c:408) and takes the host
 * cache's rows of the device layers (a restored session's prefix).
 * Returns 0, or -1 (the model stays on its CPU path). */
int hip_backend_bind_model(Backend *b, ModelWeights *mw, KVCache *kv);

/* 1 when the bound model is wholly on the device (every layer, the
 * embedding and the LM head): generate.c and chat.c then run prompts and
 * decode steps through the two calls below instead of forward(). */
int hip_backend_whole(const Backend *b);

/* forward(model, kv, scr, tokens, n_tokens, pos) of a whole device model
 * (engine.c:559-595): the prompt through gq_hip_prefill (the bf16 matrix-core
 * GEMM in chunks, or token by token in fp32 with GQ_HIP_PREFILL=steps in the
 * environment), its K/V rows copied into the host cache too.  Returns the
 * logits of the last token as a (1, vocab) F32 tensor owned by the backend
 * (valid until the next call), or NULL. */
Tensor *hip_backend_prompt(Backend *b, KVCache *kv, const int *tokens, int n_tokens, int pos);

/* One decode step of a whole device model and the reference's sampler
 * choice for it (generate.c:294-311): forward(token, pos) + sample_greedy /
 * sample_top_k / sample_top_p / sample_temperature on the device, one
 * replay of the captured step, no logits round trip.  Draws rand() exactly
 * when the reference's sampler would.  The new K/V rows stay on the device
 * until hip_backend_host_kv.  Returns the next token, or < 0 (a position
 * past the device cache: the caller continues on the CPU path, whose host
 * cache this call has brought up to date). */
int hip_backend_forward_sample(Backend *b, KVCache *kv, int token, int pos, float temperature, int top_k,
                               float top_p);

/* The device cache rows hip_backend_forward_sample wrote, into the host
 * cache (before kv_cache_save, or a CPU step). */
int hip_backend_host_kv(Backend *b, KVCache *kv);

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
