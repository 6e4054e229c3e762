/*
 * gq_oracle.c — CPU restatement of the reference decode path (TEST
 * INFRASTRUCTURE ONLY: the parity checker and the "port" CPU baseline; the
 * product library never links it).
 *
 * Reference = animeshkumarmaitreya/Guanaco.  Every function names the
 * reference lines whose arithmetic order it restates.  Build flags
 * (oracle/Makefile) match the reference's: -std=c11 -O2 -mavx2 -mfma with
 * FP contraction off, so every product/sum here is rounded exactly where the
 * reference rounds it; fused operations are spelled out as fmaf() or as the
 * AVX2 FMA intrinsics, exactly where the reference uses _mm256_fmadd_ps /
 * _mm256_fmsub_ps.
 */
#define _GNU_SOURCE
#include "gq_oracle.h"

#include "../guanaco_amd/csrc/gq_synth.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* A small persistent worker pool: the caller takes part, work is handed out
 * in fixed chunks from an atomic counter (the reference's scheme,
 * threadpool.c:37-54, 177-219).  Only timing depends on it. */

typedef void (*orc_range_fn)(int start, int end, void *ctx);

static struct {
  pthread_mutex_t mu;
  pthread_cond_t go, done;
  pthread_t th[64];
  int n_workers, n_threads, started, stop;
  unsigned gen;
  int busy;
  orc_range_fn fn;
  void *ctx;
  int end, grain;
  int next;
} g_pool = {.mu = PTHREAD_MUTEX_INITIALIZER, .go = PTHREAD_COND_INITIALIZER, .done = PTHREAD_COND_INITIALIZER};

static int g_faithful = 1;

static void pool_run_chunks(orc_range_fn fn, void *ctx, int end, int grain) {
  for (;;) {
    int s = __atomic_fetch_add(&g_pool.next, grain, __ATOMIC_RELAXED);
    if (s >= end) break;
    int e = s + grain < end ? s + grain : end;
    fn(s, e, ctx);
  }
}

static void *pool_worker(void *arg) {
  (void)arg;
  unsigned seen = 0;
  pthread_mutex_lock(&g_pool.mu);
  for (;;) {
    while (!g_pool.stop && g_pool.gen == seen) pthread_cond_wait(&g_pool.go, &g_pool.mu);
    if (g_pool.stop) break;
    seen = g_pool.gen;
    orc_range_fn fn = g_pool.fn;
    void *ctx = g_pool.ctx;
    int end = g_pool.end, grain = g_pool.grain;
    pthread_mutex_unlock(&g_pool.mu);
    pool_run_chunks(fn, ctx, end, grain);
    pthread_mutex_lock(&g_pool.mu);
    if (--g_pool.busy == 0) pthread_cond_broadcast(&g_pool.done);
  }
  pthread_mutex_unlock(&g_pool.mu);
  return NULL;
}

static void pool_stop(void) {
  if (!g_pool.started) return;
  pthread_mutex_lock(&g_pool.mu);
  g_pool.stop = 1;
  pthread_cond_broadcast(&g_pool.go);
  pthread_mutex_unlock(&g_pool.mu);
  for (int i = 0; i < g_pool.n_workers; i++) pthread_join(g_pool.th[i], NULL);
  g_pool.started = 0;
  g_pool.stop = 0;
  g_pool.n_workers = 0;
}

void orc_set_threads(int n) {
  if (n < 1) n = 1;
  if (n > 64) n = 64;
  pool_stop();
  g_pool.n_threads = n;
  g_pool.n_workers = n - 1;
  for (int i = 0; i < g_pool.n_workers; i++) pthread_create(&g_pool.th[i], NULL, pool_worker, NULL);
  g_pool.started = 1;
}

int orc_get_threads(void) { return g_pool.n_threads > 0 ? g_pool.n_threads : 1; }

void orc_set_faithful(int on) { g_faithful = on; }

static void parallel_for(int end, int grain, orc_range_fn fn, void *ctx) {
  if (grain < 1) grain = 1;
  if (g_pool.n_workers == 0 || end <= grain) {
    fn(0, end, ctx);
    return;
  }
  pthread_mutex_lock(&g_pool.mu);
  g_pool.fn = fn;
  g_pool.ctx = ctx;
  g_pool.end = end;
  g_pool.grain = grain;
  g_pool.next = 0;
  g_pool.busy = g_pool.n_workers;
  g_pool.gen++;
  pthread_cond_broadcast(&g_pool.go);
  pthread_mutex_unlock(&g_pool.mu);
  pool_run_chunks(fn, ctx, end, grain);
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.busy) pthread_cond_wait(&g_pool.done, &g_pool.mu);
  pthread_mutex_unlock(&g_pool.mu);
}

/* ------------------------------------------------------------------------ */
/* binary16 -> binary32, exact: subnormals renormalised, inf/NaN kept
 * (quant_matvec_q4_k.c:18-45). */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 31u, m = h & 1023u, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      int sh = 0;
      while (!(m & 1024u)) { m <<= 1; sh++; }
      bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 1023u) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  return gq_bits_f32(bits);
}

uint16_t orc_f32_to_f16(float f) { return gq_f32_to_f16(f); }

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Q4_K 6-bit (scale, min) of sub-block j (quant_matvec_q4_k.c:47-56). */
static inline void q4k_scale_min(const uint8_t *s, int j, float *sc, float *mn) {
  int a, b;
  if (j < 4) {
    a = s[j] & 63;
    b = s[j + 4] & 63;
  } else {
    a = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    b = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
  *sc = (float)a;
  *mn = (float)b;
}

/* ------------------------------------------------------------------------ */
/* Q4_K matvec, arithmetic order of quant_matvec_q4_k.c:65-140: per row one
 * scalar sum; per block an 8-lane FMA accumulator, lane i taking, for each
 * 64-weight chunk c and step s, the low nibble of qs[32c+8s+i] then the high
 * nibble, each weight formed as fmsub(d*sc, q, dmin*m); the 8 lanes are summed
 * left to right and added to the row sum. */
typedef struct {
  const uint8_t *w;
  const float *x;
  float *y;
  int nb;
} mv_ctx;

static void q4k_rows(int r0, int r1, void *vctx) {
  const mv_ctx *c = (const mv_ctx *)vctx;
  const __m256i lo_mask = _mm256_set1_epi32(15);
  for (int r = r0; r < r1; r++) {
    float sum = 0.0f;
    const uint8_t *blk = c->w + (size_t)r * c->nb * 144;
    for (int b = 0; b < c->nb; b++, blk += 144) {
      const float d = orc_f16_to_f32(rd16(blk)), dmin = orc_f16_to_f32(rd16(blk + 2));
      const uint8_t *sc = blk + 4, *qs = blk + 16;
      const float *x = c->x + (size_t)b * 256;
      __m256 acc = _mm256_setzero_ps();
      for (int ch = 0; ch < 4; ch++) {
        float s0, m0, s1, m1;
        q4k_scale_min(sc, 2 * ch, &s0, &m0);
        q4k_scale_min(sc, 2 * ch + 1, &s1, &m1);
        const __m256 dl = _mm256_set1_ps(d * s0), ml = _mm256_set1_ps(dmin * m0);
        const __m256 dh = _mm256_set1_ps(d * s1), mh = _mm256_set1_ps(dmin * m1);
        for (int st = 0; st < 4; st++) {
          __m256i q = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qs + 32 * ch + 8 * st)));
          __m256 wl = _mm256_fmsub_ps(dl, _mm256_cvtepi32_ps(_mm256_and_si256(q, lo_mask)), ml);
          __m256 wh = _mm256_fmsub_ps(dh, _mm256_cvtepi32_ps(_mm256_srli_epi32(q, 4)), mh);
          acc = _mm256_fmadd_ps(wl, _mm256_loadu_ps(x + 64 * ch + 8 * st), acc);
          acc = _mm256_fmadd_ps(wh, _mm256_loadu_ps(x + 64 * ch + 32 + 8 * st), acc);
        }
      }
      float t[8];
      _mm256_storeu_ps(t, acc);
      sum += t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];
    }
    c->y[r] = sum;
  }
}

static int check_args(const void *w, const float *x, const float *y, int rows, int cols, int qk,
                      size_t block_bytes, size_t bytes) {
  if (!w || !x || !y || rows <= 0 || cols <= 0) return -1;
  if (cols % qk != 0) return -2;
  if (bytes != 0 && (size_t)rows * (size_t)(cols / qk) * block_bytes > bytes) return -3;
  return 0;
}

int orc_matvec_q4k(const uint8_t *w, size_t bytes, int rows, int cols, const float *x, float *y) {
  int rc = check_args(w, x, y, rows, cols, 256, 144, bytes);
  if (rc) return rc;
  mv_ctx c = {w, x, y, cols / 256};
  int nt = orc_get_threads();
  if (nt > 1 && rows >= 32) { /* chunking of quant_matvec_q4_k.c:162-170 */
    int chunk = rows / nt;
    if (chunk < 8) chunk = 8;
    parallel_for(rows, chunk, q4k_rows, &c);
  } else {
    q4k_rows(0, rows, &c);
  }
  return 0;
}

/* Q6_K matvec, order of quant_matvec_q6_k.c:62-95: one fp32 sum per row; for
 * each block, half and l, four terms added in order, each evaluated as
 * ((d*sc)*q)*x with separate roundings. */
static void q6k_rows(int r0, int r1, void *vctx) {
  const mv_ctx *c = (const mv_ctx *)vctx;
  for (int r = r0; r < r1; r++) {
    float sum = 0.0f;
    const uint8_t *blk = c->w + (size_t)r * c->nb * 210;
    for (int b = 0; b < c->nb; b++, blk += 210) {
      const float d = orc_f16_to_f32(rd16(blk + 208));
      const float *x = c->x + (size_t)b * 256;
      for (int h = 0; h < 2; h++) {
        const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
        const float *xh = x + 128 * h;
        for (int l = 0; l < 32; l++) {
          const int s = l / 16;
          const int q0 = ((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32;
          const int q1 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
          const int q2 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
          const int q3 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
          sum += d * (float)sc[s] * (float)q0 * xh[l];
          sum += d * (float)sc[s + 2] * (float)q1 * xh[l + 32];
          sum += d * (float)sc[s + 4] * (float)q2 * xh[l + 64];
          sum += d * (float)sc[s + 6] * (float)q3 * xh[l + 96];
        }
      }
    }
    c->y[r] = sum;
  }
}

int orc_matvec_q6k(const uint8_t *w, size_t bytes, int rows, int cols, const float *x, float *y) {
  int rc = check_args(w, x, y, rows, cols, 256, 210, bytes);
  if (rc) return rc;
  mv_ctx c = {w, x, y, cols / 256};
  int nt = orc_get_threads();
  if (!g_faithful && nt > 1 && rows >= 32)
    parallel_for(rows, rows / nt > 8 ? rows / nt : 8, q6k_rows, &c);
  else
    q6k_rows(0, rows, &c);
  return 0;
}

/* Q8_0 matvec, order of quant_matvec_q8_0.c:60-75: per 32-block an in-order
 * sum of q*x, then sum += block_sum * scale. */
static void q8_rows(int r0, int r1, void *vctx) {
  const mv_ctx *c = (const mv_ctx *)vctx;
  for (int r = r0; r < r1; r++) {
    float sum = 0.0f;
    const uint8_t *blk = c->w + (size_t)r * c->nb * 34;
    for (int b = 0; b < c->nb; b++, blk += 34) {
      const float scale = orc_f16_to_f32(rd16(blk));
      const int8_t *q = (const int8_t *)(blk + 2);
      const float *x = c->x + (size_t)b * 32;
      float bs = 0.0f;
      for (int i = 0; i < 32; i++) bs += (float)q[i] * x[i];
      sum += bs * scale;
    }
    c->y[r] = sum;
  }
}

int orc_matvec_q8_0(const uint8_t *w, size_t bytes, int rows, int cols, const float *x, float *y) {
  int rc = check_args(w, x, y, rows, cols, 32, 34, bytes);
  if (rc) return rc;
  mv_ctx c = {w, x, y, cols / 32};
  int nt = orc_get_threads();
  if (!g_faithful && nt > 1 && rows >= 32)
    parallel_for(rows, rows / nt > 8 ? rows / nt : 8, q8_rows, &c);
  else
    q8_rows(0, rows, &c);
  return 0;
}

int orc_matvec(const orc_tensor *t, const float *x, float *y) {
  if (!t) return -1;
  switch (t->dtype) {
  case ORC_Q4_K: return orc_matvec_q4k(t->data, t->bytes, t->rows, t->cols, x, y);
  case ORC_Q6_K: return orc_matvec_q6k(t->data, t->bytes, t->rows, t->cols, x, y);
  case ORC_Q8_0: return orc_matvec_q8_0(t->data, t->bytes, t->rows, t->cols, x, y);
  default: return -1;
  }
}

/* ------------------------------------------------------------------------ */
/* 8-lane FMA dot product, lanes summed left to right (kernels_cpu.c:35-71). */
float orc_dot8(const float *a, const float *b, int k) {
  __m256 acc = _mm256_setzero_ps();
  int i = 0;
  for (; i + 8 <= k; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
  float t[8];
  _mm256_storeu_ps(t, acc);
  float sum = 0.0f;
  sum += t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];
  for (; i < k; i++) sum += a[i] * b[i];
  return sum;
}

/* RMSNorm (kernels_cpu.c:199-265): 8-lane FMA sum of squares, /dim, +eps,
 * 1/sqrtf, out = w * (x * r). */
void orc_rmsnorm(const float *x, const float *w, float *out, int dim, float eps) {
  __m256 acc = _mm256_setzero_ps();
  int j = 0;
  for (; j + 8 <= dim; j += 8) {
    __m256 v = _mm256_loadu_ps(x + j);
    acc = _mm256_fmadd_ps(v, v, acc);
  }
  float t[8];
  _mm256_storeu_ps(t, acc);
  float ss = t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];
  for (; j < dim; j++) ss += x[j] * x[j];
  ss /= (float)dim;
  ss += eps;
  ss = 1.0f / sqrtf(ss);
  for (int i = 0; i < dim; i++) out[i] = (w ? w[i] : 1.0f) * (x[i] * ss);
}

/* Softmax (kernels_cpu.c:271-310): serial max; all -inf -> zeros; expf(x-max)
 * with a serial sum clamped below at 1e-10; divide. */
void orc_softmax(float *x, int n) {
  float mx = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  if (isinf(mx) && mx < 0) {
    for (int i = 0; i < n; i++) x[i] = 0.0f;
    return;
  }
  float s = 0.0f;
  for (int i = 0; i < n; i++) {
    x[i] = expf(x[i] - mx);
    s += x[i];
  }
  if (s < 1e-10f) s = 1e-10f;
  for (int i = 0; i < n; i++) x[i] /= s;
}

/* SiLU (kernels_cpu.c:312-341): x * (1/(1+expf(-x))) over whole groups of 8,
 * x / (1+expf(-x)) on the tail. */
void orc_silu(float *x, int n) {
  const int nv = (n / 8) * 8;
  int i = 0;
  for (; i < nv; i++) {
    float sig = 1.0f / (1.0f + expf(0.0f - x[i]));
    x[i] = x[i] * sig;
  }
  for (; i < n; i++) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* RoPE table for one position (kernels_cpu.c:409-413): f = 1/powf(theta,
 * i/hd) for even i; angle = (float)pos * f; cosf/sinf. */
void orc_rope_table(float *cos_out, float *sin_out, int head_dim, int pos, float theta) {
  for (int i = 0; i < head_dim; i += 2) {
    float f = 1.0f / powf(theta, (float)i / (float)head_dim);
    float a = (float)pos * f;
    cos_out[i / 2] = cosf(a);
    sin_out[i / 2] = sinf(a);
  }
}

/* Adjacent-pair rotation of every Q head then every K head
 * (kernels_cpu.c:391-431), products and differences rounded separately. */
void orc_rope(float *q, float *k, int n_heads, int n_kv_heads, int head_dim, int pos, float theta) {
  float cs[512], sn[512];
  orc_rope_table(cs, sn, head_dim, pos, theta);
  for (int i = 0; i < head_dim; i += 2) {
    const float c = cs[i / 2], s = sn[i / 2];
    for (int h = 0; h < n_heads; h++) {
      float *p = q + (size_t)h * head_dim;
      const float a = p[i], b = p[i + 1];
      p[i] = a * c - b * s;
      p[i + 1] = a * s + b * c;
    }
    for (int h = 0; h < n_kv_heads; h++) {
      float *p = k + (size_t)h * head_dim;
      const float a = p[i], b = p[i + 1];
      p[i] = a * c - b * s;
      p[i + 1] = a * s + b * c;
    }
  }
}

/* Offset of (layer, head, pos) in a KV slab (kv_cache.c:90-93). */
static inline size_t kv_off(const orc_kv *kv, int layer, int head, int pos) {
  return (((size_t)layer * kv->n_kv_heads + head) * kv->max_seq + pos) * kv->head_dim;
}

/* Append one K/V row per KV head at pos % max_seq (kv_cache.c:95-128). */
int orc_kv_append(orc_kv *kv, int layer, int pos, const float *k, const float *v) {
  if (!kv || !k || !v) return -1;
  if (layer < 0 || layer >= kv->n_layers) return -1;
  int p = pos % kv->max_seq;
  for (int h = 0; h < kv->n_kv_heads; h++) {
    memcpy(kv->k + kv_off(kv, layer, h, p), k + (size_t)h * kv->head_dim, sizeof(float) * kv->head_dim);
    memcpy(kv->v + kv_off(kv, layer, h, p), v + (size_t)h * kv->head_dim, sizeof(float) * kv->head_dim);
  }
  return 0;
}

/* Single-query GQA attention of one layer (engine.c:433-509): per Q head h,
 * kv_h = h / (n_heads/n_kv); s_j = dot8(q_h, K_j) * (1/sqrtf(hd)) for
 * j <= pos; softmax; o_h[d] = in-order FMA chain of p_j * V_j[d] (the 8-column
 * blocks of kernels_cpu.c:82-112). */
void orc_attention(const float *q, const orc_kv *kv, int layer, int n_heads, int pos, float *out) {
  const int hd = kv->head_dim, n_kv = kv->n_kv_heads;
  int L = pos + 1;
  if (L > kv->max_seq) L = kv->max_seq;
  const float scale = 1.0f / sqrtf((float)hd);
  float *p = (float *)malloc(sizeof(float) * (size_t)L);
  for (int h = 0; h < n_heads; h++) {
    const int g = h / (n_heads / n_kv);
    const float *K = kv->k + kv_off(kv, layer, g, 0);
    const float *V = kv->v + kv_off(kv, layer, g, 0);
    const float *qh = q + (size_t)h * hd;
    for (int j = 0; j < L; j++) {
      float s = orc_dot8(qh, K + (size_t)j * hd, hd) * scale;
      if (j > pos) s = -INFINITY;
      p[j] = s;
    }
    orc_softmax(p, L);
    float *o = out + (size_t)h * hd;
    for (int d = 0; d < hd; d++) {
      float acc = 0.0f;
      if (d < (hd / 8) * 8) {
        for (int j = 0; j < L; j++) acc = fmaf(p[j], V[(size_t)j * hd + d], acc);
      } else {
        for (int j = 0; j < L; j++) acc += p[j] * V[(size_t)j * hd + d];
      }
      o[d] = acc;
    }
  }
  free(p);
}

/* Embedding row: F32 copy, Q8_0 q*scale, Q4_K d*sc*q - dmin*m with separate
 * roundings (engine.c:214-283). */
void orc_embed(const orc_tensor *e, int token, float *out) {
  const int H = e->cols;
  if (e->dtype == ORC_F32) {
    memcpy(out, (const float *)e->data + (size_t)token * H, sizeof(float) * H);
  } else if (e->dtype == ORC_Q8_0) {
    const uint8_t *row = e->data + (size_t)token * (H / 32) * 34;
    for (int b = 0; b < H / 32; b++) {
      const float s = orc_f16_to_f32(rd16(row + 34 * b));
      const int8_t *q = (const int8_t *)(row + 34 * b + 2);
      for (int i = 0; i < 32; i++) out[32 * b + i] = (float)q[i] * s;
    }
  } else if (e->dtype == ORC_Q4_K) {
    const uint8_t *row = e->data + (size_t)token * (H / 256) * 144;
    for (int b = 0; b < H / 256; b++) {
      const uint8_t *blk = row + 144 * b;
      const float d = orc_f16_to_f32(rd16(blk)), dmin = orc_f16_to_f32(rd16(blk + 2));
      for (int ch = 0; ch < 4; ch++) {
        float s0, m0, s1, m1;
        q4k_scale_min(blk + 4, 2 * ch, &s0, &m0);
        q4k_scale_min(blk + 4, 2 * ch + 1, &s1, &m1);
        const float d1 = d * s0, n1 = dmin * m0, d2 = d * s1, n2 = dmin * m1;
        const uint8_t *q = blk + 16 + 32 * ch;
        float *o = out + 256 * b + 64 * ch;
        for (int l = 0; l < 32; l++) o[l] = d1 * (float)(q[l] & 15) - n1;
        for (int l = 0; l < 32; l++) o[32 + l] = d2 * (float)(q[l] >> 4) - n2;
      }
    }
  }
}

/* Greedy argmax, ties to the lowest index (tokenizer.c:175-185). */
int orc_argmax(const float *x, int n) {
  int best = 0;
  float bv = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > bv) {
      bv = x[i];
      best = i;
    }
  return best;
}

static void matvec_or_die(const orc_tensor *t, const float *x, float *y) {
  if (orc_matvec(t, x, y) != 0) abort(); /* linear_dispatch aborts (engine.c:125-151) */
}

/* One decode layer, T = 1 (engine.c:353-554). */
int orc_layer(const orc_model *m, orc_kv *kv, int l, int pos, float *hidden) {
  const int H = m->hidden, hd = m->head_dim, kvd = m->n_kv_heads * hd, F = m->ff;
  float *buf = (float *)malloc(sizeof(float) * ((size_t)6 * H + 2 * kvd + 2 * F));
  float *res = buf, *nrm = res + H, *Q = nrm + H, *K = Q + H, *V = K + kvd, *att = V + kvd;
  float *proj = att + H, *nrm2 = proj + H, *gate = nrm2 + H, *up = gate + F;
  memcpy(res, hidden, sizeof(float) * H);
  orc_rmsnorm(hidden, m->rms_att[l], nrm, H, m->rms_eps);
  matvec_or_die(&m->wq[l], nrm, Q);
  matvec_or_die(&m->wk[l], nrm, K);
  matvec_or_die(&m->wv[l], nrm, V);
  orc_rope(Q, K, m->n_heads, m->n_kv_heads, hd, pos, m->rope_theta);
  orc_kv_append(kv, l, pos, K, V);
  orc_attention(Q, kv, l, m->n_heads, pos, att);
  matvec_or_die(&m->wo[l], att, proj);
  for (int i = 0; i < H; i++) proj[i] = proj[i] + res[i];
  memcpy(res, proj, sizeof(float) * H);
  orc_rmsnorm(proj, m->rms_ffn[l], nrm2, H, m->rms_eps);
  matvec_or_die(&m->wg[l], nrm2, gate);
  matvec_or_die(&m->wu[l], nrm2, up);
  orc_silu(gate, F);
  for (int i = 0; i < F; i++) gate[i] = gate[i] * up[i];
  matvec_or_die(&m->wd[l], gate, hidden);
  for (int i = 0; i < H; i++) hidden[i] = hidden[i] + res[i];
  free(buf);
  return 0;
}

/* embed -> layers -> final RMSNorm -> LM head (engine.c:559-594). */
int orc_forward_token(const orc_model *m, orc_kv *kv, int token, int pos, float *logits,
                      float *hidden_per_layer) {
  const int H = m->hidden;
  float *h = (float *)malloc(sizeof(float) * 2 * (size_t)H), *n = h + H;
  orc_embed(&m->embed, token, h);
  for (int l = 0; l < m->n_layers; l++) {
    orc_layer(m, kv, l, pos, h);
    if (hidden_per_layer) memcpy(hidden_per_layer + (size_t)l * H, h, sizeof(float) * H);
  }
  orc_rmsnorm(h, m->rms_final, n, H, m->rms_eps);
  matvec_or_die(&m->lm_head, n, logits);
  free(h);
  return orc_argmax(logits, m->lm_head.rows);
}

/* ------------------------------------------------------------------------ */
/* .lctx image: 64-byte header {magic "LCTX", version 1, n_layers, n_kv_heads,
 * head_dim, max_seq, current_pos, n_tokens, 32 reserved zero bytes}, int32
 * tokens, then K of every layer, then V of every layer, each layer at the full
 * max_seq stride (session.c:33-103). */
size_t orc_lctx_size(const orc_kv *kv, int n_tokens) {
  size_t slab = (size_t)kv->n_layers * kv->n_kv_heads * kv->max_seq * kv->head_dim * sizeof(float);
  return 64 + 4 * (size_t)(n_tokens > 0 ? n_tokens : 0) + 2 * slab;
}

static void put32(uint8_t *p, uint32_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
  p[2] = (uint8_t)(v >> 16);
  p[3] = (uint8_t)(v >> 24);
}

static uint32_t get32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

int orc_lctx_write(const orc_kv *kv, int current_pos, const int32_t *tokens, int n_tokens,
                   uint8_t *out, size_t out_size) {
  size_t need = orc_lctx_size(kv, n_tokens);
  if (!out || out_size < need) return -1;
  memset(out, 0, 64);
  put32(out + 0, 0x5843544Cu);
  put32(out + 4, 1u);
  put32(out + 8, (uint32_t)kv->n_layers);
  put32(out + 12, (uint32_t)kv->n_kv_heads);
  put32(out + 16, (uint32_t)kv->head_dim);
  put32(out + 20, (uint32_t)kv->max_seq);
  put32(out + 24, (uint32_t)current_pos);
  put32(out + 28, (uint32_t)n_tokens);
  size_t o = 64;
  if (n_tokens > 0 && tokens) {
    memcpy(out + o, tokens, 4 * (size_t)n_tokens);
    o += 4 * (size_t)n_tokens;
  }
  size_t slab = (size_t)kv->n_layers * kv->n_kv_heads * kv->max_seq * kv->head_dim * sizeof(float);
  memcpy(out + o, kv->k, slab);
  memcpy(out + o + slab, kv->v, slab);
  return 0;
}

/* Restore: validate magic, version, geometry and max_seq (session.c:107-188). */
int orc_lctx_read(orc_kv *kv, const uint8_t *img, size_t size, int *current_pos, int *n_tokens) {
  if (!kv || !img || size < 64) return -1;
  if (get32(img) != 0x5843544Cu || get32(img + 4) != 1u) return -1;
  if ((int)get32(img + 8) != kv->n_layers || (int)get32(img + 12) != kv->n_kv_heads ||
      (int)get32(img + 16) != kv->head_dim)
    return -1;
  if ((int)get32(img + 20) != kv->max_seq) return -1;
  int nt = (int)get32(img + 28);
  size_t slab = (size_t)kv->n_layers * kv->n_kv_heads * kv->max_seq * kv->head_dim * sizeof(float);
  size_t o = 64 + 4 * (size_t)(nt > 0 ? nt : 0);
  if (size < o + 2 * slab) return -1;
  memcpy(kv->k, img + o, slab);
  memcpy(kv->v, img + o + slab, slab);
  if (current_pos) *current_pos = (int)get32(img + 24);
  if (n_tokens) *n_tokens = nt;
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Synthetic inputs from gq_synth.h (byte-identical to the device fill). */
typedef struct {
  uint64_t seed;
  uint8_t *out;
  int nb_row;
  int kind;
  float *fout;
  int zero_mean; /* Q4_K: the zero-mean rule (gq_q4k_zm_byte) */
} synth_ctx;

static void synth_rows(int r0, int r1, void *vctx) {
  const synth_ctx *c = (const synth_ctx *)vctx;
  const int bb = c->kind == ORC_Q4_K ? 144 : c->kind == ORC_Q6_K ? 210 : 34;
  for (int r = r0; r < r1; r++) {
    for (int b = 0; b < c->nb_row; b++) {
      uint64_t bi = (uint64_t)r * c->nb_row + b;
      uint8_t *o = c->out + bi * bb;
      for (int k = 0; k < bb; k++) {
        o[k] = c->kind == ORC_Q4_K ? (c->zero_mean ? gq_q4k_zm_byte(c->seed, bi, (uint32_t)k)
                                                   : gq_q4k_byte(c->seed, bi, (uint32_t)k))
               : c->kind == ORC_Q6_K ? gq_q6k_byte(c->seed, bi, (uint32_t)k)
                                     : gq_q8_0_byte(c->seed, bi, (uint32_t)k);
      }
    }
  }
}

void orc_synth_q4k(uint64_t seed, int rows, int cols, uint8_t *out) {
  synth_ctx c = {seed, out, cols / 256, ORC_Q4_K, NULL, 0};
  parallel_for(rows, 64, synth_rows, &c);
}

void orc_synth_q4k_zm(uint64_t seed, int rows, int cols, uint8_t *out) {
  synth_ctx c = {seed, out, cols / 256, ORC_Q4_K, NULL, 1};
  parallel_for(rows, 64, synth_rows, &c);
}

void orc_synth_q6k(uint64_t seed, int rows, int cols, uint8_t *out) {
  synth_ctx c = {seed, out, cols / 256, ORC_Q6_K, NULL, 0};
  parallel_for(rows, 64, synth_rows, &c);
}

void orc_synth_q8_0(uint64_t seed, int rows, int cols, uint8_t *out) {
  synth_ctx c = {seed, out, cols / 32, ORC_Q8_0, NULL, 0};
  parallel_for(rows, 64, synth_rows, &c);
}

static void normal_chunk(int c0, int c1, void *vctx) {
  const synth_ctx *c = (const synth_ctx *)vctx;
  size_t n = (size_t)c->nb_row;
  for (size_t i = (size_t)c0 * 4096; i < (size_t)c1 * 4096 && i < n; i++) c->fout[i] = gq_normal(c->seed, i);
}

void orc_synth_normal(uint64_t seed, size_t n, float *out) {
  synth_ctx c = {seed, NULL, (int)n, 0, out, 0};
  if (n > 0x7fffffffULL) abort();
  parallel_for((int)((n + 4095) / 4096), 16, normal_chunk, &c);
}

void orc_synth_norm_weight(uint64_t seed, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) out[i] = gq_norm_weight(seed, i);
}

uint64_t orc_tensor_seed(uint64_t model_seed, int layer, int slot) {
  return gq_tensor_seed(model_seed, layer, slot);
}

/* KV pre-fill: seeded N(0,1) history at positions 0..n_pos-1 of every layer and
 * KV head, element index from gq_kv_index (independent of max_seq). */
typedef struct {
  uint64_t seed;
  float *slab;
  int n_kv, hd, max_seq, n_pos;
} kvfill_ctx;

static void kvfill_rows(int r0, int r1, void *vctx) {
  const kvfill_ctx *c = (const kvfill_ctx *)vctx;
  for (int r = r0; r < r1; r++) { /* r = layer * n_kv + head */
    const int layer = r / c->n_kv, h = r % c->n_kv;
    float *base = c->slab + (size_t)r * c->max_seq * c->hd;
    for (int p = 0; p < c->n_pos; p++)
      for (int d = 0; d < c->hd; d++)
        base[(size_t)p * c->hd + d] = gq_normal(c->seed, gq_kv_index(layer, c->n_kv, h, p, c->hd, d));
  }
}

void orc_synth_kv(uint64_t seed, float *slab, int n_layers, int n_kv_heads, int head_dim,
                  int max_seq, int n_pos) {
  kvfill_ctx c = {seed, slab, n_kv_heads, head_dim, max_seq, n_pos};
  parallel_for(n_layers * n_kv_heads, 1, kvfill_rows, &c);
}
