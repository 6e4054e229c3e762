/*
 * types.h — the data contract the backend boundary is written against.
 *
 * Restates, field for field, the reference's shared types (types.h:16-147 of
 * animeshkumarmaitreya/Guanaco): the DataType codes, Tensor (with the GPU
 * residency flag and device pointer), ModelConfig, LayerWeights and
 * ModelWeights.  The layouts must stay identical so hip_backend.c compiles
 * unchanged inside the reference tree and this repository's tests can hand
 * these structs to the reference's compiled engine.
 */
#ifndef LLMRT_TYPES_H
#define LLMRT_TYPES_H

#include <stddef.h>
#include <stdint.h>

typedef enum {
  DTYPE_F32 = 0,
  DTYPE_F16 = 1,
  DTYPE_Q8_0 = 2,
  DTYPE_Q4_0 = 3,
  DTYPE_Q4_K = 4,
  DTYPE_Q6_K = 5,
  DTYPE_UNKNOWN = 99,
} DataType;

#define MAX_DIMS 4

typedef struct {
  void *data;               /* host bytes (mmap'd weights or scratch) */
  int shape[MAX_DIMS];      /* shape[0] outermost; weights are [rows=out][cols=in] */
  int stride[MAX_DIMS];     /* in elements */
  int ndim;
  DataType dtype;
  uint32_t ggml_type;
  size_t byte_size;         /* authoritative size of quantised tensors; 0 = unknown */
  int device_residency;     /* 0 host, 1 device */
  void *d_data;             /* device copy when device_residency == 1 */
} Tensor;

typedef struct {
  int hidden_dim, n_heads, n_kv_heads, head_dim, n_layers, vocab_size;
  int bos_token_id, eos_token_id, ff_dim, max_seq_len;
  char **vocab_strings;
  float *vocab_scores;
} ModelConfig;

typedef struct {
  Tensor *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down, *rms_att, *rms_ffn;
} LayerWeights;

typedef struct {
  ModelConfig config;
  LayerWeights *layers;
  Tensor *embedding, *rms_final, *lm_head;
} ModelWeights;

typedef struct Arena Arena;
typedef struct Scratch Scratch;
typedef struct KVCache KVCache;

#endif
