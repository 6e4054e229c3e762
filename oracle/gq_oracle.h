/*
 * gq_oracle.h — CPU restatement of the reference's decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X path and the "port" CPU baseline.  Only tests/, the smoke check in
 * __graft_entry__.py and bench.py's cpu_baseline leg may load it; the
 * product library (libgq_hip.so) never links or calls it.
 *
 * Each function restates, in its own code, the arithmetic ORDER of the
 * reference CPU path (animeshkumarmaitreya/Guanaco, src/...), cited per
 * function in gq_oracle.c, so that its fp32 results are bit-identical to the
 * reference's on the same inputs.  How each function is pinned (golden
 * vectors from the compiled reference, the reference's own known-answer
 * tests, closed forms, fp64 brute force) is listed in oracle/README.md.
 */
#ifndef GQ_ORACLE_H
#define GQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: the reference's DataType values (types.h:16-24). */
enum { ORC_F32 = 0, ORC_Q8_0 = 2, ORC_Q4_K = 4, ORC_Q6_K = 5 };

typedef struct {
  int dtype;
  int rows; /* out_features */
  int cols; /* in_features */
  const uint8_t *data;
  size_t bytes;
} orc_tensor;

typedef struct {
  int n_layers, hidden, ff, n_heads, n_kv_heads, head_dim, vocab, max_seq;
  float rope_theta, rms_eps;
  /* per layer */
  orc_tensor *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  const float **rms_att, **rms_ffn;
  /* global */
  orc_tensor embed, lm_head;
  const float *rms_final;
} orc_model;

/* KV slabs, layout [layer][kv_head][max_seq][head_dim] fp32 (kv_cache.c:25-32). */
typedef struct {
  float *k, *v;
  int n_layers, n_kv_heads, head_dim, max_seq;
} orc_kv;

/* --- threading (timing faithfulness only; results are thread-count invariant) --- */
void orc_set_threads(int n);
int orc_get_threads(void);
/* 1: Q6_K/Q8_0 single-threaded like the reference (default); 0: row-parallel. */
void orc_set_faithful(int on);

/* --- scalar pieces --- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* --- matvecs: y[rows] = W[rows, cols] . x[cols]; return 0 / -1 / -2 / -3 --- */
int orc_matvec_q4k(const uint8_t *w, size_t bytes, int rows, int cols, const float *x, float *y);
int orc_matvec_q6k(const uint8_t *w, size_t bytes, int rows, int cols, const float *x, float *y);
int orc_matvec_q8_0(const uint8_t *w, size_t bytes, int rows, int cols, const float *x, float *y);
int orc_matvec(const orc_tensor *t, const float *x, float *y);

/* --- layer glue --- */
void orc_rmsnorm(const float *x, const float *w, float *out, int dim, float eps);
float orc_dot8(const float *a, const float *b, int k);
void orc_softmax(float *x, int n);
void orc_silu(float *x, int n);
void orc_rope(float *q, float *k, int n_heads, int n_kv_heads, int head_dim, int pos, float theta);
void orc_rope_table(float *cos_out, float *sin_out, int head_dim, int pos, float theta);
void orc_attention(const float *q, const orc_kv *kv, int layer, int n_heads, int pos, float *out);
void orc_embed(const orc_tensor *e, int token, float *out);
int orc_argmax(const float *x, int n);

/* --- KV cache (kv_cache.c) --- */
int orc_kv_append(orc_kv *kv, int layer, int pos, const float *k, const float *v);

/* --- one decode token through the whole model (engine.c:287-594) ---
 * hidden_per_layer (optional): n_layers * hidden floats, the residual stream
 * after each layer.  logits: vocab floats.  Returns the greedy token. */
int orc_layer(const orc_model *m, orc_kv *kv, int layer, int pos, float *hidden);
int orc_forward_token(const orc_model *m, orc_kv *kv, int token, int pos, float *logits,
                      float *hidden_per_layer);

/* --- .lctx session image (session.c:33-103) --- */
size_t orc_lctx_size(const orc_kv *kv, int n_tokens);
int orc_lctx_write(const orc_kv *kv, int current_pos, const int32_t *tokens, int n_tokens,
                   uint8_t *out, size_t out_size);
int orc_lctx_read(orc_kv *kv, const uint8_t *img, size_t size, int *current_pos, int *n_tokens);

/* --- synthetic inputs (gq_synth.h) --- */
void orc_synth_q4k(uint64_t seed, int rows, int cols, uint8_t *out);
void orc_synth_q4k_zm(uint64_t seed, int rows, int cols, uint8_t *out); /* zero-mean rule */
void orc_synth_q6k(uint64_t seed, int rows, int cols, uint8_t *out);
void orc_synth_q8_0(uint64_t seed, int rows, int cols, uint8_t *out);
void orc_synth_normal(uint64_t seed, size_t n, float *out);
void orc_synth_norm_weight(uint64_t seed, size_t n, float *out);
uint64_t orc_tensor_seed(uint64_t model_seed, int layer, int slot);
void orc_synth_kv(uint64_t seed, float *slab, int n_layers, int n_kv_heads, int head_dim,
                  int max_seq, int n_pos);

#ifdef __cplusplus
}
#endif
#endif
