/*
 * gq_hip.h — C ABI of libgq_hip.so, the MI355X (gfx950) decode hot path.
 *
 * Plain C types only: opaque context, device pointers as void*, host
 * pointers, sizes and int status codes.  Every entry point names the
 * reference interface it replaces (animeshkumarmaitreya/Guanaco, src/...).
 * A host-side KernelVTable binding (guanaco_amd/host/hip_backend.c) and the
 * ctypes mirror (guanaco_amd/hip.py) sit on top of it.
 *
 * Status codes: 0 success; -1 bad argument / NULL / bad dtype / not
 * initialised (the reference's matvec code -1, quant_matvec_q4_k.c:143-146);
 * -2 cols not a multiple of the block length (:150-151); -3 byte_size too
 * small for the shape (:154-158); -4 HIP runtime error or out of device
 * memory (the caller falls back to the CPU path, as engine.c:347-350 does
 * for cuda_transformer_layer_gpu's -1); -5 position outside the KV cache.
 * gq_hip_last_error() returns a message for the last failure on a context.
 *
 * Threading: a context owns one HIP stream; calls on one context are not
 * thread-safe (matches the reference's single-threaded engine,
 * engine.c:287-594).  Entry points that return host data synchronise the
 * stream before returning; *_dev entry points are asynchronous on the
 * context stream until gq_hip_sync().
 */
#ifndef GQ_HIP_H
#define GQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes = the reference's DataType values (types.h:16-24) */
#define GQ_F32 0
#define GQ_Q8_0 2
#define GQ_Q4_K 4
#define GQ_Q6_K 5

typedef struct gq_ctx gq_ctx;

/* ---------------------------------------------------------------- lifecycle
 * Replaces the CUDA backend's device bring-up (cuda_backend.c:43-81) and the
 * hidden static streams (matvec_q4k_cuda.cu:83, cuda_layer_kernels.cu:314). */
int gq_hip_device_count(void);                 /* 0 when no usable GPU */
gq_ctx *gq_hip_create(int device_id);          /* NULL when unavailable */
void gq_hip_destroy(gq_ctx *ctx);              /* frees every device buffer */
const char *gq_hip_last_error(const gq_ctx *ctx);
/* Replaces cuda_finish_layer (cuda_layer_kernels.cu:715-717). */
int gq_hip_sync(gq_ctx *ctx);
/* Number of compute units and the device name (for reports). */
int gq_hip_device_info(gq_ctx *ctx, int *n_cu, char *name, int name_len);

/* ------------------------------------------------------- device memory
 * Replaces cuda_upload_weight (matvec_q4k_cuda.cu:115-133): allocates and
 * copies `bytes` from host memory, returns the device pointer or NULL (the
 * loader then keeps the tensor CPU-resident, loader.c:711-717).  The copy
 * goes through two 32 MiB pinned staging slots of the context (CPU copy of
 * one chunk overlapping the DMA of the previous one), so the source may be a
 * private file mapping, which the reference stages through a heap copy for.
 * Allocations carry 256 bytes of tail padding so block loads never leave the
 * buffer. */
void *gq_hip_upload_weight(gq_ctx *ctx, const void *host, size_t bytes);
/* hipMemGetInfo of a device: free and total bytes (no counterpart in the
 * reference; shows that gq_hip_destroy returns every byte). */
int gq_hip_mem_info(int device_id, size_t *free_bytes, size_t *total_bytes);
void *gq_hip_malloc(gq_ctx *ctx, size_t bytes);
void gq_hip_free(gq_ctx *ctx, void *dev);
int gq_hip_h2d(gq_ctx *ctx, void *dev, const void *host, size_t bytes);
int gq_hip_d2h(gq_ctx *ctx, void *host, const void *dev, size_t bytes);

/* ------------------------------------------------------- synthetic inputs
 * Device fill with the generator of csrc/gq_synth.h (bit-identical to the
 * host generator the parity oracle uses).  dtype Q4_K/Q6_K/Q8_0: rows x cols
 * blocks; GQ_Q4_K | GQ_SYNTH_Q4K_ZERO_MEAN: Q4_K blocks whose sub-block mins
 * cancel the scales' mean (m_j = sc_j, dmin = fp16(7.5 d)), so the weights
 * are zero-mean; normal: n fp32 ~ N(0,1); norm_weight: n fp32
 * 1 + N(0,1)/64. */
#define GQ_SYNTH_Q4K_ZERO_MEAN 0x100
int gq_hip_synth_quant(gq_ctx *ctx, void *dev, int dtype, int rows, int cols, uint64_t seed);
int gq_hip_synth_normal(gq_ctx *ctx, float *dev, size_t n, uint64_t seed);
int gq_hip_synth_norm_weight(gq_ctx *ctx, float *dev, size_t n, uint64_t seed);

/* ------------------------------------------------------- quantised matvec
 * y[rows] = W[rows, cols] . x[cols]; W device-resident in the reference's
 * on-disk block layout.  Replaces the vtable slots matvec_q4k_f32 /
 * matvec_q6k_f32 / matvec_q8_0_f32 (backend.h:36-38) and the CUDA host
 * wrapper cuda_matvec_q4k_f32_impl (matvec_q4k_cuda.cu:85-113): x and y are
 * HOST pointers (engine scratch), the call returns after y is written.
 * byte_size 0 skips the size check, as the reference does. */
int gq_hip_matvec(gq_ctx *ctx, int dtype, const void *w_dev, int rows, int cols,
                  size_t byte_size, const float *x, float *y);
/* Same, device x / y, asynchronous on the context stream. */
int gq_hip_matvec_dev(gq_ctx *ctx, int dtype, const void *w_dev, int rows, int cols,
                      const float *x_dev, float *y_dev);
/* y = W (rmsnorm(x) * norm_w): the reference's cpu_rmsnorm followed by its
 * matvec (engine.c:356-366, :582-590), with the norm fused into the matvec's
 * x staging as the decode step runs it.  Device pointers, asynchronous. */
int gq_hip_matvec_norm_dev(gq_ctx *ctx, int dtype, const void *w_dev, int rows, int cols,
                           const float *x_dev, const float *norm_w_dev, float eps, float *y_dev);

/* ------------------------------------------------------- KV cache
 * Device-resident fp32 cache in the reference layout
 * [layer][kv_head][max_seq][head_dim], K and V in separate slabs
 * (kv_cache.c:25-32, offset formula :90-93), zeroed at init
 * (kv_cache_create, :34-84).  Also uploads the RoPE (cos, sin) table for
 * positions 0..max_seq-1, computed on the host with the reference's fp32
 * expressions (kernels_cpu.c:409-413) for the given theta. */
int gq_hip_kv_init(gq_ctx *ctx, int n_layers, int n_kv_heads, int head_dim, int max_seq,
                   float rope_theta);
float *gq_hip_kv_k(gq_ctx *ctx, int layer); /* device pointer of a layer's K slab */
float *gq_hip_kv_v(gq_ctx *ctx, int layer);
/* Append one token's K and V rows (n_kv_heads x head_dim each, host memory)
 * at pos % max_seq — kv_cache_append (kv_cache.c:95-128).  Bit copies. */
int gq_hip_kv_append(gq_ctx *ctx, int layer, int pos, const float *k, const float *v);
/* Copy a layer's whole K/V slabs device -> host / host -> device
 * (kv_cache_raw_k / raw_v + memcpy, kv_cache.c:189-205). */
int gq_hip_kv_read_layer(gq_ctx *ctx, int layer, float *k, float *v);
int gq_hip_kv_write_layer(gq_ctx *ctx, int layer, const float *k, const float *v);
/* T new host rows from position pos of one layer -> device; arguments as
 * cuda_sync_kv_cache (cuda_layer_kernels.cu:585-603). */
int gq_hip_kv_sync(gq_ctx *ctx, int layer, int pos, int T, const float *h_k, const float *h_v,
                   int head_stride, int max_seq);
/* The reverse of gq_hip_kv_sync: rows pos .. pos+T-1 of every KV head of
 * `layer` from the device cache into the host slabs (head_stride floats
 * between heads, kv_cache_head_stride), so a CPU layer or a host-side
 * kv_cache_save after a device prefill sees them.  Synchronous. */
int gq_hip_kv_fetch(gq_ctx *ctx, int layer, int pos, int T, float *h_k, float *h_v, int head_stride,
                    int max_seq);
/* Seeded N(0,1) history at positions 0..n_pos-1 (gq_synth.h gq_kv_index). */
int gq_hip_kv_prefill_synth(gq_ctx *ctx, uint64_t seed_k, uint64_t seed_v, int n_pos);

/* ------------------------------------------------------- sessions (.lctx)
 * Byte-identical to kv_cache_save / kv_cache_load (session.c:52-188): 64-byte
 * header, int32 tokens, K of all layers, V of all layers at full max_seq
 * stride.  Save gathers from the DEVICE cache (the device cache is the source
 * of truth); load validates magic, version, geometry and max_seq and
 * restores into the device cache.  *tokens is malloc'ed (caller frees) when
 * the file holds tokens and tokens != NULL. */
int gq_hip_lctx_save(gq_ctx *ctx, const char *path, int current_pos, const int32_t *tokens,
                     int n_tokens);
int gq_hip_lctx_load(gq_ctx *ctx, const char *path, int *current_pos, int32_t **tokens,
                     int *n_tokens);
/* Frozen-prefix prompt cache (prompt_cache_save / prompt_cache_load,
 * session.c:192-251): the .lctx format with current_pos = prefix_len and
 * n_tokens = 0, gathered from / restored into the device cache; save
 * rejects prefix_len <= 0 with -1 as the reference does. */
int gq_hip_prompt_cache_save(gq_ctx *ctx, int prefix_len, const char *path);
int gq_hip_prompt_cache_load(gq_ctx *ctx, const char *path, int *prefix_len);
/* Restore K/V from a .lctx image already in host memory (e.g. pinned),
 * returns the milliseconds the host->device copy took (HIP events). */
int gq_hip_lctx_restore_image(gq_ctx *ctx, const void *image, size_t size, int *current_pos,
                              float *ms);
void *gq_hip_host_alloc_pinned(size_t bytes); /* hipHostMalloc */
void gq_hip_host_free_pinned(void *p);

/* ------------------------------------------------------- model + decode
 * Device-resident model description: the GPU side of LayerWeights /
 * ModelWeights (types.h:127-147).  Weight pointers are device pointers from
 * gq_hip_upload_weight / gq_hip_malloc; norm weights are device fp32. */
typedef struct {
  const void *data;
  int dtype;
  int rows, cols;
} gq_weight;

typedef struct {
  gq_weight wq, wk, wv, wo, w_gate, w_up, w_down;
  const float *rms_att, *rms_ffn;
} gq_layer;

typedef struct {
  int n_layers, hidden, ff, n_heads, n_kv_heads, head_dim, vocab;
  float rope_theta, rms_eps;
  const gq_layer *layers; /* host array, copied */
  gq_weight embed, lm_head;
  const float *rms_final;
} gq_model;

/* Bind a model (after gq_hip_kv_init with matching geometry) and allocate
 * the decode workspace.  A layer whose seven weights and two norm weights
 * are all NULL stays on the host (the --n-gpu-layers split, loader.c:677-728,
 * or a projection the device does not take, such as F32); so may the
 * embedding and the LM head (an F32 LM head stays on the host, as
 * loader.c:575-585 allows).  The per-layer entry points (decode_layer,
 * transformer_layer, qkv_rope) then serve the bound layers; the
 * whole-model ones (forward_token, forward_sample, decode_loop, prefill,
 * chat_turn, profile_step, time_op) need every layer, the embedding and the
 * LM head on the device and return -1 otherwise. */
int gq_hip_model_bind(gq_ctx *ctx, const gq_model *m);
/* Layers the bound model holds on the device (0 when none is bound); *whole
 * (may be NULL) is 1 when the whole-model entry points can run.  No
 * reference counterpart: the engine's IS_GPU_READY test per layer
 * (engine.c:324-328) asked once for the model. */
int gq_hip_bound_layers(gq_ctx *ctx, int *whole);

/* One decode layer on a device hidden vector (hidden -> hidden): RMSNorm,
 * QKV, RoPE + KV append, split-K GQA attention, o-proj + residual, RMSNorm,
 * gate/up + SwiGLU, down + residual.  The device-side equivalent of
 * transformer_layer for T = 1 (engine.c:353-554). */
int gq_hip_decode_layer_dev(gq_ctx *ctx, int layer, int pos, float *hidden_dev);

/* Drop-in for cuda_transformer_layer_gpu (kernels.h:46-58, called at
 * engine.c:334): host hidden in/out for one bound layer; also writes the new
 * K/V rows into the host cache (h_k_cache / h_v_cache with the given head
 * stride, may be NULL) so a later kv_cache_save sees them.  Returns 0, or
 * non-zero so the engine falls back to its CPU path. */
int gq_hip_transformer_layer(gq_ctx *ctx, int layer, int pos, float *h_hidden, float *h_k_cache,
                             float *h_v_cache, int head_stride);

/* Whole-model decode of one token at position pos on the device: embedding,
 * every layer, final RMSNorm, LM head, greedy argmax (ties to the lowest
 * index, tokenizer.c:175-185) — forward() + sample_greedy (engine.c:559-594).
 * logits (host, vocab floats) and hidden_per_layer (host, n_layers*hidden)
 * may be NULL.  Returns the next token, or a negative status. */
int gq_hip_forward_token(gq_ctx *ctx, int token, int pos, float *logits, float *hidden_per_layer);

/* Greedy decode loop of n_steps tokens from (token, pos): the generate.c
 * decode loop (generate.c:266-325) with sampling on the device.  Each step
 * is one replay of a captured HIP graph when use_graph != 0.  tokens_out
 * receives the n_steps generated tokens.  *ms (may be NULL) receives the
 * device time of the loop (HIP events around it). */
int gq_hip_decode_loop(gq_ctx *ctx, int token, int pos, int n_steps, int use_graph,
                       int32_t *tokens_out, float *ms);

/* ------------------------------------------------------- measurement
 * Runs one eager decode step with HIP events after every kernel launch and
 * accumulates per-class device time and launch counts.  Classes by role:
 * 0 q/k/v projections (RMSNorm, RoPE and K/V append fused), 1 attention
 * (partial + merge), 2 o-projection + residual, 3 gate/up + SwiGLU, 4 down
 * projection + residual, 5 final RMSNorm + LM head, 6 other (embedding,
 * argmax).  Per-class algorithmic bytes (weights, activations in and out,
 * KV read) are accumulated in bytes[]. */
#define GQ_NCLASS 7
int gq_hip_profile_step(gq_ctx *ctx, int token, int pos, double ms[GQ_NCLASS],
                        int launches[GQ_NCLASS], double bytes[GQ_NCLASS]);
/* Average device time (ms) of one op (a GQ_NCLASS class index 0..5) of the
 * bound model, launched n_iter times back to back on the context stream
 * (layer i % n_layers for launch i, so no two consecutive launches share
 * weights) between two HIP events.  The ops write their usual outputs (the
 * q/k/v op appends K/V at pos; o and down add into the hidden state). */
float gq_hip_time_op(gq_ctx *ctx, int op, int pos, int n_iter);
/* Average device time (ms) of n back-to-back launches of one matvec, timed
 * with HIP events on the context stream; rotating over n_w weight buffers
 * (to defeat the MALL) with per-buffer outputs. */
float gq_hip_time_matvec(gq_ctx *ctx, int dtype, const void *const *w_devs, int n_w, int rows,
                         int cols, const float *x_dev, float *y_dev, int n_iter);
/* Selects the matvec kernels for later launches in this process: 1
 * (default) the int8 matrix-core kernel for gate/up + SwiGLU and the LM head
 * (where the bound model has their tile-interleaved copies) and the
 * vector-ALU kernel for every other launch; 0 the vector-ALU kernel for
 * every launch; 2 the matrix-core kernel wherever it fits (the op-level
 * entry points then tile their weights per call), else the vector-ALU
 * kernel; 3 as 1, with the Q6_K down projection read from the reference
 * layout instead of the unit-layout copy gq_hip_model_bind makes for the
 * vector-ALU kernel.  Returns the previous setting.  No reference counterpart: a switch
 * for the parity tests (each kernel against the oracle) and for timing. */
int gq_hip_set_matvec_path(int path);
/* Device time of n launches of the attention kernels for one layer. */
float gq_hip_time_attention(gq_ctx *ctx, int layer, int pos, const float *q_dev, float *out_dev,
                            int n_iter);

/* ------------------------------------------------------- op-level entry points
 * (device pointers, asynchronous) used by the parity tests. */
int gq_hip_rmsnorm_dev(gq_ctx *ctx, const float *x, const float *w, float *out, int dim,
                       float eps);
/* RoPE on q (n_heads x hd) and k (n_kv x hd) at pos, then append k and v to
 * the cache of `layer` at pos (the step 4 + 5 of transformer_layer,
 * engine.c:372-392). q, k, v are device buffers; q is rotated in place. */
int gq_hip_rope_append_dev(gq_ctx *ctx, int layer, int pos, int n_heads, float *q, const float *k,
                           const float *v);
/* Split-K single-query GQA attention of `layer` over positions 0..pos
 * (engine.c:433-509): q (n_heads x hd) -> out (n_heads x hd). */
int gq_hip_attention_dev(gq_ctx *ctx, int layer, int pos, int n_heads, const float *q,
                         float *out);
/* Allocation-free form of gq_hip_attention_dev.  It has no counterpart in
 * the reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split-K partials go to a static 8 MiB device array that
 * the library holds on every GPU it runs on until the process ends, so the
 * call allocates nothing.  They take n_heads x nch x (head_dim + 2) floats,
 * nch = ceil(max_seq / 32) up to max_seq 12288 and ceil(max_seq / 128) past
 * it (the 8B shape fits up to max_seq 64512); -1 with an error message when
 * they do not fit.  Every call on one GPU shares that array and leaves its
 * partials there: calls that overlap on one GPU (other streams or contexts
 * of the same device) race. */
int gq_hip_attention_dev_noalloc(gq_ctx *ctx, int layer, int pos, int n_heads, const float *q,
                                 float *out);
/* q/k/v projections of a bound layer from a device hidden vector with the
 * layer's RMSNorm, RoPE and K/V append: fused != 0 runs the decode path's
 * single fused epilogue, fused == 0 plain matvecs followed by the standalone
 * RoPE+append kernel (the two must agree bit for bit). */
int gq_hip_qkv_rope_dev(gq_ctx *ctx, int layer, int pos, const float *hidden, float *q_out,
                        int fused);
int gq_hip_embed_dev(gq_ctx *ctx, int dtype, const void *table, int hidden, int token,
                     float *out);
int gq_hip_argmax_dev(gq_ctx *ctx, const float *x, int n, int *out_index_dev);

/* Sampling on the device, replacing the reference's sampler choice
 * (generate.c:302-311) and sample_greedy / sample_top_k / sample_top_p /
 * sample_temperature (tokenizer.c:175-333) without copying the logits to the
 * host: temperature <= 0 -> greedy; 0 < top_k < vocab -> top-k (top_k at most
 * 1024); top_p < 1 -> top-p (top_p <= 0 greedy); else temperature.  rnd is
 * the value of the caller's rand() for this token (the reference draws one
 * per sampled token; unused for greedy).  logits: vocab floats in device
 * memory.  Returns the token, or -1 bad argument, -2 top_k above 1024, -4 HIP
 * error.  Every mode follows the reference's arithmetic order (plain
 * temperature sampling sums on one device thread, ~0.3 ms at 128256
 * entries); exponentials come from the device's expf. */
int gq_hip_sample_dev(gq_ctx *ctx, const float *logits, int vocab, float temperature, int top_k, float top_p,
                      int rnd);
/* forward() of one token (gq_hip_forward_token) followed by on-device
 * sampling of the next one as above: generate.c:294-311 without the logits
 * round trip.  Returns the sampled token or < 0 (as gq_hip_forward_token). */
int gq_hip_forward_sample(gq_ctx *ctx, int token, int pos, float temperature, int top_k, float top_p, int rnd);
int gq_hip_silu_mul_dev(gq_ctx *ctx, float *gate, const float *up, int n);
/* ------------------------------------------------------- prefill chunk
 * y[t][n] = sum_k x[t][k] w[n][k] for t < T tokens at once on the bf16
 * matrix cores, fp32 accumulation: the projections of a prefill chunk, which
 * the reference runs as T sequential matvecs (linear_dispatch,
 * engine.c:119-152).  w: rows x cols Q4_K, Q6_K or Q8_0 on the device
 * (rows % 128 == 0, cols % 256 == 0, Q6_K cols % 512 == 0: -2 otherwise);
 * x: T x cols fp32, y: T x rows fp32, device pointers.  mode 0 stores, mode 1 adds r (T x rows, may alias y).
 * x and the dequantized weights are rounded to bf16 (nearest even) before
 * the products.  Q6_K weights with cols % 2048 == 0 are read through a
 * unit-layout copy made for the call (a bound model keeps its copies from
 * gq_hip_model_bind); results equal the reference layout's bit for bit.
 * Asynchronous on the context stream. */
int gq_hip_prefill_gemm_dev(gq_ctx *ctx, int dtype, int mode, const void *w, int rows, int cols,
                            const float *x, int T, float *y, const float *r);
/* Average device time (ms) of n_iter back-to-back launches of that GEMM
 * (mode 0), timed with HIP events on the context stream; the bf16 copy of
 * x and any Q6_K unit-layout copy are made before the timed region.  No
 * reference counterpart: a measurement entry, as gq_hip_time_matvec. */
float gq_hip_time_prefill_gemm(gq_ctx *ctx, int dtype, const void *w, int rows, int cols, const float *x, int T,
                               float *y, int n_iter);
/* act[t][n] = bf16(silu(g) * u) with g = x w_gate^T and u = x w_up^T on the
 * matrix cores in one launch (silu_inplace + elemwise_mul after the two
 * linear_dispatch calls, engine.c:524-549): w_gate and w_up rows x cols of
 * one dtype (Q4_K, Q8_0, or Q6_K with cols % 512 == 0), rows % 64 == 0; x T x
 * cols fp32, act T x rows bf16 (uint16 bit patterns), device pointers. */
int gq_hip_prefill_gate_up_dev(gq_ctx *ctx, int dtype, const void *w_gate, const void *w_up, int rows,
                               int cols, const float *x, int T, uint16_t *act);
/* Steps 4-10 of transformer_layer for T tokens at pos .. pos+T-1
 * (engine.c:372-509): RoPE of q (T x n_heads*hd, in place) and k
 * (T x n_kv*hd), append of every token's k and v to the cache of `layer`,
 * then causal attention, token t over positions 0 .. pos+t, into out
 * (T x n_heads*hd).  Device pointers, asynchronous; -5 when pos+T passes
 * the cache. */
int gq_hip_prefill_attention_dev(gq_ctx *ctx, int layer, int pos, int T, int n_heads, float *q,
                                 const float *k, const float *v, float *out);
/* One turn of the chat REPL (chat_repl, chat.c:157-263) on the bound model
 * (its prompt through gq_hip_prefill, so with the precision of the context's
 * prefill mode: gq_hip_set_prefill_mode),
 * KV reused across turns: tokens (BOS first only on a conversation's first
 * turn, as chat.c:157-163 tokenizes) go through the prefill at
 * *current_pos; the reply is sampled until max_tokens, 512 tokens
 * (CHAT_MAX_OUTPUT_TOKENS) or eos_token, greedy when temperature <= 0, else
 * as gq_hip_sample_dev with rnd[i] the i-th rand() value (max_tokens
 * values).  reply receives the tokens (eos included when sampled, up to
 * min(max_tokens, 512)); *current_pos advances as chat.c's current_pos
 * does (the prompt, then every reply token, the last of which is never
 * fed).  Returns the reply length; -6 when *current_pos + n_tokens >=
 * max_seq - 1, where chat.c restarts the conversation (:169-190: the caller
 * sets *current_pos = 0 and re-tokenizes with BOS); -5 when the reply runs
 * past the cache (the reference wraps, kv_cache.c:101; the device does not). */
int gq_hip_chat_turn(gq_ctx *ctx, const int32_t *tokens, int n_tokens, int *current_pos, int max_tokens,
                     int eos_token, float temperature, int top_k, float top_p, const int *rnd, int32_t *reply);
/* forward(model, kv, scr, tokens, n_tokens, pos) of the bound model
 * (engine.c:559-595): the whole prompt through every layer in chunks of
 * up to 512 tokens, filling the device KV cache at pos .. pos+n_tokens-1;
 * the slot of gpu_prefill (gpu_prefill.h:13-20).  tokens and the optional
 * outputs are host pointers: logits (vocab floats) and hidden_last (the
 * last token's final hidden state before the final RMSNorm) of the last
 * token, ms the device time.  Returns the greedy next token (>= 0) or a
 * negative error (-5: positions outside the cache). */
int gq_hip_prefill(gq_ctx *ctx, const int32_t *tokens, int n_tokens, int pos, float *logits,
                   float *hidden_last, float *ms);
/* How gq_hip_prefill (and gq_hip_chat_turn's prompt) runs a prompt on this
 * context: 0 (default) the chunked matrix-core GEMM path above, whose
 * products round x and the weights to bf16 (logits within ~5e-3 relative
 * of an fp32 forward); 1 token by token through the fp32 decode step, the
 * reference's own precision (forward() over T tokens equals T single-token
 * steps up to fp32 rounding), at the decode step's speed per token.
 * Returns the previous mode, or -1.  No reference counterpart: the
 * reference has no prompt GEMM (linear_dispatch loops over tokens,
 * engine.c:119-152). */
int gq_hip_set_prefill_mode(gq_ctx *ctx, int mode);
/* Device-to-device copy by a plain streaming kernel (bytes and both pointers
 * multiples of 16), asynchronous.  No reference counterpart: the known-size
 * workload that scales the HBM byte counters of the profiles. */
int gq_hip_copy_dev(gq_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Average device time (ms) of one launch of a read-only streaming kernel
 * over `bytes` (a multiple of 16): eight 16-byte loads per thread issued
 * before use, a grid that covers the bytes in one pass, nothing stored.  Launch i reads src + (i mod n_buf) * stride,
 * so src must hold (n_buf - 1) * stride + bytes bytes (stride >= bytes when
 * n_buf > 1, a multiple of 16); 1 untimed + n_iter timed launches between
 * HIP events on the context stream.  No reference counterpart: the floor a
 * single launch reading that many bytes reaches, beside which the decode
 * kernels' durations are set (-1 on a bad argument). */
float gq_hip_time_read(gq_ctx *ctx, const void *src, size_t bytes, size_t stride, int n_buf, int n_iter);

#ifdef __cplusplus
}
#endif
#endif /* GQ_HIP_H */
