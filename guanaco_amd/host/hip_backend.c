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

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gq_hip.h"
#include "tokenizer.h"

typedef struct {
  gq_ctx *ctx;
  Backend *cpu; /* dense ops + CPU-resident quant matvecs */
  /* the bound model (hip_backend_bind_model) */
  int vocab, max_seq, n_layers;
  float *logits;  /* host logits of the last whole-model prompt */
  Tensor logits_t; /* (1, vocab) F32 view of them, as forward() returns */
  /* device cache rows [dirty_lo, dirty_hi) written by whole-model steps and
   * not yet in the host cache */
  int dirty_lo, dirty_hi;
  int device;
  size_t free0; /* free HBM when the backend was made (before any upload) */
} HipImpl;

static HipImpl *g_hip; /* the live HIP backend (see the file comment) */

/* The reference's samplers draw from the C library's rand() stream
 * (tokenizer.c:187-333, one draw per sampled token), unseeded, so a run is
 * repeatable.  The HIP runtime reseeds that stream when it initialises, so
 * without care --device hip would sample other tokens than --device cpu.
 * Every entry point below that calls into the HIP library therefore hands
 * the stream back as it found it: rng_save copies the generator's state and
 * rng_restore makes a copy of it current.  glibc keeps that state in the
 * array rand() and random() share, with the read position in the array's
 * first word, written there when the array stops being current
 * (initstate(3) / setstate(3)). */
static int32_t rng_snap[64], rng_buf[2][64];
static int rng_next, rng_depth;

static void rng_save(void) {
  if (rng_depth++) return; /* nested: the outermost call keeps the snapshot */
  static const int deg[5] = {0, 7, 15, 31, 63};
  static int32_t probe[32];
  char *cur = initstate(1, (char *)probe, sizeof probe); /* the current array, its position written */
  memcpy(rng_snap, cur, sizeof(int32_t) * (1 + deg[((int32_t *)cur)[0] % 5]));
  (void)setstate(cur);
}

static void rng_restore(void) {
  if (--rng_depth) return;
  /* never the current array: setstate writes the position into that one */
  int32_t *b = rng_buf[rng_next];
  rng_next ^= 1;
  memcpy(b, rng_snap, sizeof rng_snap);
  (void)setstate((char *)b);
}

static int hip_matvec(int dtype, DataType want, int (*cpu_fn)(const Tensor *, const float *, float *),
                      const Tensor *W, const float *x, float *y) {
  if (!W || !x || !y) return -1;
  if (W->device_residency != 1 || !W->d_data) return cpu_fn ? cpu_fn(W, x, y) : -1;
  if (!g_hip || W->dtype != want || W->ndim != 2) return -1;
  rng_save();
  const int rc = gq_hip_matvec(g_hip->ctx, dtype, W->d_data, W->shape[0], W->shape[1], W->byte_size, x, y);
  rng_restore();
  return rc;
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

static Backend *hip_create(const BackendConfig *cfg);

Backend *backend_hip_create(const BackendConfig *cfg) {
  rng_save();
  Backend *b = hip_create(cfg);
  rng_restore();
  return b;
}

static Backend *hip_create(const BackendConfig *cfg) {
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
  impl->device = cfg->device_id;
  size_t total = 0;
  if (gq_hip_mem_info(cfg->device_id, &impl->free0, &total)) impl->free0 = 0;
  /* GQ_HIP_PREFILL=steps: prompts token by token through the fp32 decode
   * step (the reference's precision) instead of the bf16 matrix-core GEMM */
  const char *pm = getenv("GQ_HIP_PREFILL");
  if (pm && strcmp(pm, "steps") == 0) (void)gq_hip_set_prefill_mode(ctx, 1);
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
    rng_save();
    gq_hip_destroy(impl->ctx); /* frees every device weight and buffer */
    rng_restore();
    backend_cpu_destroy(impl->cpu);
    free(impl->logits);
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
  rng_save();
  void *d = gq_hip_upload_weight(ctx, t->data, t->byte_size);
  rng_restore();
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
  if (!ctx) return -1;
  rng_save();
  const int rc = gq_hip_sync(ctx);
  rng_restore();
  return rc;
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

/* A weight the loader made device-resident (d_data); anything else is left
 * out (NULL data), and the tensor's owner stays on the host. */
static void resident_weight(const Tensor *t, gq_weight *w) {
  memset(w, 0, sizeof *w);
  if (!t || t->ndim != 2 || t->device_residency != 1 || !t->d_data || gq_dtype(t->dtype) < 0) return;
  w->data = t->d_data;
  w->dtype = gq_dtype(t->dtype);
  w->rows = t->shape[0];
  w->cols = t->shape[1];
}

static int bind_model(Backend *b, ModelWeights *mw, KVCache *kv);

int hip_backend_bind_model(Backend *b, ModelWeights *mw, KVCache *kv) {
  rng_save();
  const int rc = bind_model(b, mw, kv);
  rng_restore();
  return rc;
}

static int bind_model(Backend *b, ModelWeights *mw, KVCache *kv) {
  gq_ctx *ctx = hip_backend_context(b);
  HipImpl *impl = ctx ? (HipImpl *)b->impl : NULL;
  if (!ctx || !mw || !mw->layers || !kv) return -1;
  const ModelConfig *c = &mw->config;
  if (gq_hip_kv_init(ctx, c->n_layers, c->n_kv_heads, c->head_dim, c->max_seq_len, 500000.0f)) return -1;
  gq_layer *layers = (gq_layer *)calloc((size_t)c->n_layers, sizeof(gq_layer));
  if (!layers) return -1;
  int rc = 0;
  /* Per tensor: a layer goes to the device when the loader made its seven
   * projections device-resident (the --n-gpu-layers split, loader.c:677-728;
   * F32 projections stay on the host); every other layer stays on the CPU
   * path and nothing of it is uploaded. */
  int all_layers = 1;
  for (int l = 0; l < c->n_layers && !rc; l++) {
    const LayerWeights *L = &mw->layers[l];
    if (!hip_layer_ready(L)) {
      all_layers = 0;
      continue;
    }
    gq_layer *g = &layers[l];
    resident_weight(L->wq, &g->wq), resident_weight(L->wk, &g->wk), resident_weight(L->wv, &g->wv);
    resident_weight(L->wo, &g->wo), resident_weight(L->w_gate, &g->w_gate);
    resident_weight(L->w_up, &g->w_up), resident_weight(L->w_down, &g->w_down);
    g->rms_att = (const float *)device_copy(ctx, L->rms_att);
    g->rms_ffn = (const float *)device_copy(ctx, L->rms_ffn);
    rc = g->rms_att && g->rms_ffn ? 0 : -1;
  }
  gq_model m;
  memset(&m, 0, sizeof m);
  if (!rc) {
    m.n_layers = c->n_layers, m.hidden = c->hidden_dim, m.ff = c->ff_dim;
    m.n_heads = c->n_heads, m.n_kv_heads = c->n_kv_heads, m.head_dim = c->head_dim, m.vocab = c->vocab_size;
    m.rope_theta = 500000.0f; /* kernels_cpu.c:408 */
    m.rms_eps = 1e-6f;        /* engine.c:359, 524, 582 */
    m.layers = layers;
    /* With every layer on the device, the whole model: the LM head the
     * loader put there (a quantised head; an F32 one stays on the host),
     * the final norm and the embedding table in any dtype the device embeds
     * (F32, Q8_0, Q4_K).  Otherwise forward() runs on the host and reaches
     * the device layers through the engine hook and the LM head through the
     * vtable, so nothing more is uploaded. */
    if (all_layers) resident_weight(mw->lm_head, &m.lm_head);
    if (m.lm_head.data && !(m.rms_final = (const float *)device_copy(ctx, mw->rms_final))) rc = -1;
    const Tensor *e = mw->embedding;
    if (!rc && m.lm_head.data && e && e->ndim == 2 &&
        (e->dtype == DTYPE_F32 || e->dtype == DTYPE_Q8_0 || e->dtype == DTYPE_Q4_K)) {
      m.embed.data = device_copy(ctx, e);
      m.embed.dtype = gq_dtype(e->dtype);
      m.embed.rows = e->shape[0];
      m.embed.cols = e->shape[1];
    }
  }
  if (!rc) rc = gq_hip_model_bind(ctx, &m);
  free(layers); /* gq_hip_model_bind copies the layer array */
  if (rc) return -1;
  free(impl->logits);
  impl->logits = (float *)calloc((size_t)c->vocab_size, sizeof(float));
  if (!impl->logits) return -1;
  memset(&impl->logits_t, 0, sizeof impl->logits_t);
  impl->logits_t.data = impl->logits;
  impl->logits_t.dtype = DTYPE_F32;
  impl->logits_t.ndim = 2;
  impl->logits_t.shape[0] = 1, impl->logits_t.shape[1] = c->vocab_size;
  impl->logits_t.stride[0] = c->vocab_size, impl->logits_t.stride[1] = 1;
  impl->logits_t.byte_size = sizeof(float) * (size_t)c->vocab_size;
  impl->vocab = c->vocab_size, impl->max_seq = c->max_seq_len, impl->n_layers = c->n_layers;
  impl->dirty_lo = impl->dirty_hi = 0;
  int whole = 0;
  const int n_dev = gq_hip_bound_layers(ctx, &whole);
  const Tensor *lm = mw->lm_head;
  size_t free1 = 0, total = 0;
  const double used = !gq_hip_mem_info(impl->device, &free1, &total) && impl->free0 >= free1
                          ? (double)(impl->free0 - free1) / 1e9 : -1.0;
  fprintf(stderr, "[hip] %d of %d layers on the device, LM head on the %s; %s; %.2f GB of HBM in use\n", n_dev,
          c->n_layers, lm && lm->device_residency == 1 && lm->d_data ? "device" : "host",
          whole ? "prompts and decode steps run whole on the device" : "forward() runs, device layers through the layer hook",
          used);
  /* the host cache may already hold a prefix (a restored session) */
  const int hs = kv_cache_head_stride(kv);
  for (int l = 0; l < c->n_layers; l++)
    if (hip_layer_ready(&mw->layers[l]) &&
        gq_hip_kv_sync(ctx, l, 0, c->max_seq_len, kv_cache_raw_k(kv, l), kv_cache_raw_v(kv, l), hs,
                       c->max_seq_len))
      return -1;
  return 0;
}

int hip_backend_whole(const Backend *b) {
  gq_ctx *ctx = hip_backend_context(b);
  int whole = 0;
  return ctx && gq_hip_bound_layers(ctx, &whole) >= 0 ? whole : 0;
}

/* Rows [p0, p0 + T) of every layer from the device cache into the host
 * cache. */
static int fetch_rows(gq_ctx *ctx, KVCache *kv, int n_layers, int p0, int T, int max_seq) {
  const int hs = kv_cache_head_stride(kv);
  for (int l = 0; l < n_layers; l++)
    if (gq_hip_kv_fetch(ctx, l, p0, T, kv_cache_raw_k(kv, l), kv_cache_raw_v(kv, l), hs, max_seq)) return -1;
  return 0;
}

Tensor *hip_backend_prompt(Backend *b, KVCache *kv, const int *tokens, int n_tokens, int pos) {
  gq_ctx *ctx = hip_backend_context(b);
  HipImpl *impl = ctx ? (HipImpl *)b->impl : NULL;
  if (!ctx || !impl->logits || !kv || !tokens || n_tokens <= 0) return NULL;
  rng_save();
  /* the host cache takes the prompt's rows too: prompt_cache_save and
   * kv_cache_save read it */
  const int ok = gq_hip_prefill(ctx, (const int32_t *)tokens, n_tokens, pos, impl->logits, NULL, NULL) >= 0 &&
                 fetch_rows(ctx, kv, impl->n_layers, pos, n_tokens, impl->max_seq) == 0;
  rng_restore();
  return ok ? &impl->logits_t : NULL;
}

/* Whether the reference's sampler for these settings draws a rand()
 * (generate.c:302-311 picks it; tokenizer.c:187-333): not when greedy, nor
 * for top-p with p <= 0. */
static int draws_rand(int vocab, float temperature, int top_k, float top_p) {
  if (temperature <= 0.0f) return 0;
  if (top_k > 0 && top_k < vocab) return 1;
  if (top_p < 1.0f) return top_p > 0.0f;
  return 1;
}

int hip_backend_forward_sample(Backend *b, KVCache *kv, int token, int pos, float temperature, int top_k,
                               float top_p) {
  gq_ctx *ctx = hip_backend_context(b);
  HipImpl *impl = ctx ? (HipImpl *)b->impl : NULL;
  if (!ctx || !impl->logits || !kv) return -1;
  int next;
  if (pos < 0 || pos >= impl->max_seq) { /* past the device cache: the CPU path, which wraps */
    next = -5;
  } else if (temperature > 0.0f && top_k > 1024 && top_k < impl->vocab) {
    /* a top-k the device sampler does not take: the reference's own sampler
     * on the device logits (it draws its own rand()) */
    rng_save();
    next = gq_hip_forward_token(ctx, token, pos, impl->logits, NULL);
    rng_restore();
    if (next >= 0) next = sample_top_k(impl->logits, impl->vocab, top_k, temperature);
  } else {
    const int rnd = draws_rand(impl->vocab, temperature, top_k, top_p) ? rand() : 0;
    rng_save();
    next = gq_hip_forward_sample(ctx, token, pos, temperature, top_k, top_p, rnd);
    rng_restore();
  }
  if (next >= 0) {
    if (impl->dirty_hi <= impl->dirty_lo) impl->dirty_lo = pos, impl->dirty_hi = pos;
    if (pos < impl->dirty_lo) impl->dirty_lo = pos;
    if (pos + 1 > impl->dirty_hi) impl->dirty_hi = pos + 1;
  } else {
    (void)hip_backend_host_kv(b, kv); /* the caller's CPU path continues from the host cache */
  }
  return next;
}

int hip_backend_host_kv(Backend *b, KVCache *kv) {
  gq_ctx *ctx = hip_backend_context(b);
  HipImpl *impl = ctx ? (HipImpl *)b->impl : NULL;
  if (!ctx || !kv) return -1;
  if (impl->dirty_hi <= impl->dirty_lo) return 0;
  rng_save();
  const int rc = fetch_rows(ctx, kv, impl->n_layers, impl->dirty_lo, impl->dirty_hi - impl->dirty_lo,
                            impl->max_seq);
  rng_restore();
  if (!rc) impl->dirty_lo = impl->dirty_hi = 0;
  return rc;
}

int hip_backend_prefill(const Backend *backend, ModelWeights *model, KVCache *kv, Scratch *scr,
                        const int *token_ids, int n_tokens, int pos) {
  (void)scr;
  gq_ctx *ctx = hip_backend_context(backend);
  if (!ctx || !model || !kv || !token_ids || n_tokens <= 0) return -1;
  rng_save();
  const int ok = gq_hip_prefill(ctx, (const int32_t *)token_ids, n_tokens, pos, NULL, NULL, NULL) >= 0 &&
                 fetch_rows(ctx, kv, model->config.n_layers, pos, n_tokens, model->config.max_seq_len) == 0;
  rng_restore();
  return ok ? 0 : -1;
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
  rng_save();
  const int rc = gq_hip_transformer_layer(g_hip->ctx, layer, pos, hidden, kv_cache_raw_k(kv, layer),
                                          kv_cache_raw_v(kv, layer), kv_cache_head_stride(kv));
  rng_restore();
  return rc;
}

int hip_backend_kv_sync(KVCache *kv, int layer, int pos, int T, int max_seq) {
  if (!g_hip || !kv) return -1;
  rng_save();
  const int rc = gq_hip_kv_sync(g_hip->ctx, layer, pos, T, kv_cache_raw_k(kv, layer), kv_cache_raw_v(kv, layer),
                                kv_cache_head_stride(kv), max_seq);
  rng_restore();
  return rc;
}

int hip_backend_sync(void) {
  if (!g_hip) return 0;
  rng_save();
  const int rc = gq_hip_sync(g_hip->ctx);
  rng_restore();
  return rc;
}
