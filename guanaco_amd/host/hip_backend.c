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
#include <string.h>

#include "gq_hip.h"

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

static int upload_to(gq_ctx *ctx, Tensor *t) {
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

int hip_backend_upload(Backend *b, Tensor *t) { return upload_to(hip_backend_context(b), t); }

int hip_backend_finish(Backend *b) {
  gq_ctx *ctx = hip_backend_context(b);
  return ctx ? gq_hip_sync(ctx) : -1;
}

/* The reference's KV accessors (kv_cache.c:189-205), as engine.c:307-309
 * declares them. */
extern float *kv_cache_raw_k(KVCache *kv, int layer);
extern float *kv_cache_raw_v(KVCache *kv, int layer);
extern int kv_cache_head_stride(KVCache *kv);

static int gq_dtype(DataType d) {
  switch (d) {
  case DTYPE_F32: return GQ_F32;
  case DTYPE_Q8_0: return GQ_Q8_0;
  case DTYPE_Q4_K: return GQ_Q4_K;
  case DTYPE_Q6_K: return GQ_Q6_K;
  default: return -1;
  }
}

/* A device copy of a tensor: its own d_data when the loader uploaded it,
 * else a fresh upload owned by the device context. */
static const void *device_copy(gq_ctx *ctx, const Tensor *t) {
  if (!t || !t->data) return NULL;
  if (t->device_residency == 1 && t->d_data) return t->d_data;
  size_t bytes = t->byte_size;
  if (!bytes && t->dtype == DTYPE_F32) {
    bytes = sizeof(float);
    for (int i = 0; i < t->ndim; i++) bytes *= (size_t)t->shape[i];
  }
  return bytes ? gq_hip_upload_weight(ctx, t->data, bytes) : NULL;
}

static int weight_of(gq_ctx *ctx, const Tensor *t, gq_weight *w) {
  if (!t || t->ndim != 2 || gq_dtype(t->dtype) < 0) return -1;
  w->data = device_copy(ctx, t);
  w->dtype = gq_dtype(t->dtype);
  w->rows = t->shape[0];
  w->cols = t->shape[1];
  return w->data ? 0 : -1;
}

int hip_backend_bind_model(Backend *b, ModelWeights *mw, KVCache *kv) {
  gq_ctx *ctx = hip_backend_context(b);
  if (!ctx || !mw || !mw->layers || !kv) return -1;
  const ModelConfig *c = &mw->config;
  if (gq_hip_kv_init(ctx, c->n_layers, c->n_kv_heads, c->head_dim, c->max_seq_len, 500000.0f)) return -1;
  gq_layer *layers = (gq_layer *)calloc((size_t)c->n_layers, sizeof(gq_layer));
  if (!layers) return -1;
  int rc = 0;
  for (int l = 0; l < c->n_layers && !rc; l++) {
    const LayerWeights *L = &mw->layers[l];
    gq_layer *g = &layers[l];
    rc = weight_of(ctx, L->wq, &g->wq) || weight_of(ctx, L->wk, &g->wk) || weight_of(ctx, L->wv, &g->wv) ||
         weight_of(ctx, L->wo, &g->wo) || weight_of(ctx, L->w_gate, &g->w_gate) ||
         weight_of(ctx, L->w_up, &g->w_up) || weight_of(ctx, L->w_down, &g->w_down);
    if (!rc) {
      g->rms_att = (const float *)device_copy(ctx, L->rms_att);
      g->rms_ffn = (const float *)device_copy(ctx, L->rms_ffn);
      rc = g->rms_att && g->rms_ffn ? 0 : -1;
    }
  }
  gq_model m;
  memset(&m, 0, sizeof m);
  if (!rc) {
    m.n_layers = c->n_layers, m.hidden = c->hidden_dim, m.ff = c->ff_dim;
    m.n_heads = c->n_heads, m.n_kv_heads = c->n_kv_heads, m.head_dim = c->head_dim, m.vocab = c->vocab_size;
    m.rope_theta = 500000.0f; /* kernels_cpu.c:408 */
    m.rms_eps = 1e-6f;        /* engine.c:359, 524, 582 */
    m.layers = layers;
    m.rms_final = (const float *)device_copy(ctx, mw->rms_final);
    rc = weight_of(ctx, mw->embedding, &m.embed) || weight_of(ctx, mw->lm_head, &m.lm_head) || !m.rms_final;
  }
  if (!rc) rc = gq_hip_model_bind(ctx, &m);
  free(layers); /* gq_hip_model_bind copies the layer array */
  if (rc) return -1;
  /* the host cache may already hold a prefix (a restored session) */
  const int hs = kv_cache_head_stride(kv);
  for (int l = 0; l < c->n_layers; l++)
    if (gq_hip_kv_sync(ctx, l, 0, c->max_seq_len, kv_cache_raw_k(kv, l), kv_cache_raw_v(kv, l), hs,
                       c->max_seq_len))
      return -1;
  return 0;
}

int hip_backend_prefill(const Backend *backend, ModelWeights *model, KVCache *kv, Scratch *scr,
                        const int *token_ids, int n_tokens, int pos) {
  (void)scr;
  gq_ctx *ctx = hip_backend_context(backend);
  if (!ctx || !model || !kv || !token_ids || n_tokens <= 0) return -1;
  if (gq_hip_prefill(ctx, (const int32_t *)token_ids, n_tokens, pos, NULL, NULL, NULL) < 0) return -1;
  const int hs = kv_cache_head_stride(kv);
  for (int l = 0; l < model->config.n_layers; l++)
    if (gq_hip_kv_fetch(ctx, l, pos, n_tokens, kv_cache_raw_k(kv, l), kv_cache_raw_v(kv, l), hs,
                        model->config.max_seq_len))
      return -1;
  return 0;
}

/* ------------------------------------------------------------ engine and loader hooks
 * transformer_layer and load_model see no Backend, as the CUDA build's
 * direct hooks do not (cuda_upload_weight, cuda_transformer_layer_gpu,
 * cuda_sync_kv_cache, cuda_finish_layer): these act on the live HIP
 * backend. */

int hip_upload_weight(Tensor *t) { return upload_to(g_hip ? g_hip->ctx : NULL, t); }

int hip_layer_ready(const LayerWeights *lw) {
  if (!g_hip || !lw) return 0;
  const Tensor *t[7] = {lw->wq, lw->wk, lw->wv, lw->wo, lw->w_gate, lw->w_up, lw->w_down};
  for (int i = 0; i < 7; i++)
    if (!t[i] || t[i]->device_residency != 1 || !t[i]->d_data) return 0;
  return 1;
}

int hip_backend_layer(int layer, int pos, float *hidden, KVCache *kv) {
  if (!g_hip || !hidden || !kv) return -1;
  return gq_hip_transformer_layer(g_hip->ctx, layer, pos, hidden, kv_cache_raw_k(kv, layer),
                                  kv_cache_raw_v(kv, layer), kv_cache_head_stride(kv));
}

int hip_backend_kv_sync(KVCache *kv, int layer, int pos, int T, int max_seq) {
  if (!g_hip || !kv) return -1;
  return gq_hip_kv_sync(g_hip->ctx, layer, pos, T, kv_cache_raw_k(kv, layer), kv_cache_raw_v(kv, layer),
                        kv_cache_head_stride(kv), max_seq);
}

int hip_backend_sync(void) { return g_hip ? gq_hip_sync(g_hip->ctx) : 0; }
