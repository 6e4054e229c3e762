/*
 * gq_runtime.hip — the C ABI of libgq_hip.so (include/gq_hip.h): device
 * context and stream, memory, the device KV cache and .lctx sessions, model
 * binding, the per-token decode step (eager or replayed from a captured HIP
 * graph) and event-based measurement.
 *
 * Device memory plan for one context (sized for 288 GB of HBM):
 *   weights     as uploaded, reference block layout, 256 B tail padding;
 *   K, V slabs  [layer][kv_head][max_seq][head_dim] fp32, one allocation each
 *               (8B shape at max_seq 8320: 2 x 1.09 GB);
 *   RoPE table  [max_seq][head_dim/2] (cos, sin) fp32 pairs;
 *   workspace   hidden, q|k|v, attention output, SwiGLU activation, logits,
 *               split-K partials, argmax partials, device token/pos/step.
 */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "gq_internal.h"

namespace {

constexpr size_t kPad = 256;

struct Workspace {
  float *hidden = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *act2 = nullptr;
  float *logits = nullptr, *part_o = nullptr, *part_ml = nullptr, *amax = nullptr;
  int *d_token = nullptr, *d_pos = nullptr, *d_step = nullptr, *d_tokens = nullptr;
  int tokens_cap = 0, nch = 0, s_max = 0, amax_blocks = 0;
  size_t part_cap = 0, part_ml_cap = 0; /* floats in part_o / part_ml */
};

/* Prefill-chunk activations, T x width row-major, allocated on first use
 * for up to `cap` tokens; attention partials grow with the context. */
struct PrefillWs {
  int cap = 0;
  int H = 0, F = 0, kvd = 0; /* hidden, ff and n_kv_heads * head_dim the buffers were sized for */
  float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr; /* fp32: hidden, q/k/v for RoPE */
  __bf16 *xn = nullptr, *att = nullptr, *act = nullptr;          /* bf16 GEMM inputs */
  __bf16 *xb = nullptr; /* op-level entry: bf16 copy of its fp32 x */
  int *tok = nullptr;
  size_t xb_cap = 0;
  float *part = nullptr; /* the GEMM's K-part sums (PgArgs.part) */
  size_t part_cap = 0;
};

/* tokens per prefill chunk */
constexpr int kPrefillChunk = 512;

} // namespace

struct gq_ctx {
  int dev = 0;
  hipStream_t stream = nullptr;
  char err[512] = {0};
  int n_cu = 0;
  char name[128] = {0};
  std::vector<void *> allocs;
  /* host-pointer op staging */
  float *sx = nullptr, *sy = nullptr;
  size_t sx_cap = 0, sy_cap = 0;
  /* KV cache */
  int kv_layers = 0, kv_heads = 0, kv_hd = 0, kv_max_seq = 0;
  float theta = 0.f;
  float *kslab = nullptr, *vslab = nullptr;
  float2 *rope = nullptr;
  /* model: `bound` once gq_hip_model_bind succeeded; layer_on[l] for the
   * layers it holds (the rest stay on the host); `whole` when every layer,
   * the embedding and the LM head are on the device, which the whole-model
   * entry points need */
  bool bound = false, whole = false;
  gq_model m{};
  std::vector<gq_layer> layers;
  std::vector<char> layer_on;
  /* prompts through gq_hip_prefill: 0 the matrix-core GEMM in chunks, 1 token
   * by token through the fp32 decode step (gq_hip_set_prefill_mode) */
  int prefill_mode = 0;
  /* tile-interleaved copies of the bound model's gate+up pairs and LM head
   * for the matrix-core matvec (gq_launch_mm_tile), owned by the context;
   * NULL where a weight does not take that layout */
  struct MmLayer {
    const uint8_t *gu = nullptr;
    const uint8_t *dx = nullptr; /* Q6_K down in the vector-ALU unit layout (gq_launch_q6k_units) */
    /* Q6_K projections in the same unit layout for the prefill GEMM (cols %
     * 2048): wq, wk, wv, wo, gate, up, down; ux[6] is dx itself */
    const uint8_t *ux[7] = {};
  };
  std::vector<MmLayer> mm;
  const uint8_t *mm_lm = nullptr;
  Workspace ws;
  PrefillWs pf;
  float *scratch = nullptr; /* this device's address of the file-scope `scratch` array */
  /* host -> device staging: two pinned slots, allocated on first upload */
  void *stage[2] = {nullptr, nullptr};
  hipEvent_t stage_ev[2] = {nullptr, nullptr};
  SampleWs sw;
  int *d_sample = nullptr; /* sampled token (device) */
  /* graph */
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  /* the device state a graph replay left behind (graph_step): w.hidden holds
   * the embedding of g_token, to be decoded at g_pos */
  bool g_valid = false;
  int g_token = -1, g_pos = -1;
  int *st_pinned = nullptr; /* pinned (token, pos, step) for graph_step */
  /* measurement hooks for eager steps */
  bool prof = false;
  std::vector<hipEvent_t> ev;
  std::vector<int> ev_class;
  std::vector<double> ev_bytes;
};

static int fail(gq_ctx *c, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
static void pf_release(gq_ctx *c);
static int fail(gq_ctx *c, int code, const char *fmt, ...) {
  if (c) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(c->err, sizeof c->err, fmt, ap);
    va_end(ap);
  }
  return code;
}

#define HIPCHK(c, call)                                                                         \
  do {                                                                                          \
    hipError_t e_ = (call);                                                                     \
    if (e_ != hipSuccess) return fail((c), -4, "%s: %s", #call, hipGetErrorString(e_));         \
  } while (0)

/* A start/stop pair of timing events, destroyed on every exit path. */
struct EventPair {
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t create() {
    const hipError_t e = hipEventCreate(&e0);
    return e != hipSuccess ? e : hipEventCreate(&e1);
  }
  float ms() const {
    float t = 0.f;
    (void)hipEventElapsedTime(&t, e0, e1);
    return t;
  }
  ~EventPair() {
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
  }
};

static size_t block_bytes(int dtype, int *qk) {
  switch (dtype) {
  case GQ_Q4_K: *qk = 256; return 144;
  case GQ_Q6_K: *qk = 256; return 210;
  case GQ_Q8_0: *qk = 32; return 34;
  default: *qk = 0; return 0;
  }
}

/* profile classes (gq_hip.h) */
enum { PC_QKV = 0, PC_ATTN, PC_O, PC_GATE_UP, PC_DOWN, PC_LM_HEAD, PC_OTHER };

/* ------------------------------------------------------------ lifecycle */
extern "C" int gq_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

/* ------------------------------------------------------------ scratch
 * Device memory of gq_hip_attention_dev_noalloc (split-K partials): a
 * file-scope array that every GPU the library runs on holds until the
 * process ends, so that entry point needs no allocation.  On the host the
 * name is only a stand-in for the symbol, never an address: each device's
 * address comes from hipGetSymbolAddress, taken once per device with that
 * device current (at its first context creation) and kept in scratch_addr. */
constexpr size_t kScratchFloats = (size_t)2 << 20; /* 8 MiB */
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
static std::mutex scratch_mu;
static float *scratch_addr[kMaxDevices];

/* the calling thread's current device is `dev` */
static float *scratch_setup(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(scratch_mu);
  if (!scratch_addr[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    scratch_addr[dev] = (float *)p;
  }
  return scratch_addr[dev];
}

extern "C" gq_ctx *gq_hip_create(int device_id) {
  int n = gq_hip_device_count();
  if (device_id < 0 || device_id >= n) return nullptr;
  if (hipSetDevice(device_id) != hipSuccess) return nullptr;
  gq_ctx *c = new gq_ctx();
  c->dev = device_id;
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return nullptr;
  }
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, device_id) == hipSuccess) {
    c->n_cu = p.multiProcessorCount;
    snprintf(c->name, sizeof c->name, "%s", p.gcnArchName);
    gq_matvec_set_cus(c->n_cu);
  }
  c->scratch = scratch_setup(device_id); /* NULL: the allocation-free entry point reports it */
  return c;
}

static void free_graph(gq_ctx *c) {
  if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
  if (c->graph) (void)hipGraphDestroy(c->graph);
  c->gexec = nullptr;
  c->graph = nullptr;
  c->g_valid = false;
}

extern "C" void gq_hip_destroy(gq_ctx *c) {
  if (!c) return;
  (void)hipSetDevice(c->dev);
  (void)hipStreamSynchronize(c->stream);
  free_graph(c);
  if (c->st_pinned) (void)hipHostFree(c->st_pinned);
  for (hipEvent_t e : c->ev) (void)hipEventDestroy(e);
  for (void *p : c->allocs) (void)hipFree(p);
  for (int i = 0; i < 2; i++) {
    if (c->stage[i]) (void)hipHostFree(c->stage[i]);
    if (c->stage_ev[i]) (void)hipEventDestroy(c->stage_ev[i]);
  }
  (void)hipStreamDestroy(c->stream);
  delete c;
}

extern "C" const char *gq_hip_last_error(const gq_ctx *c) { return c ? c->err : "no context"; }

extern "C" int gq_hip_sync(gq_ctx *c) {
  if (!c) return -1;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_device_info(gq_ctx *c, int *n_cu, char *name, int name_len) {
  if (!c) return -1;
  if (n_cu) *n_cu = c->n_cu;
  if (name && name_len > 0) snprintf(name, (size_t)name_len, "%s", c->name);
  return 0;
}

/* ------------------------------------------------------------ memory */
static void *dev_alloc(gq_ctx *c, size_t bytes) {
  void *p = nullptr;
  if (hipMalloc(&p, bytes + kPad) != hipSuccess) {
    fail(c, -4, "hipMalloc(%zu) failed", bytes + kPad);
    return nullptr;
  }
  c->allocs.push_back(p);
  return p;
}

extern "C" void *gq_hip_malloc(gq_ctx *c, size_t bytes) {
  if (!c) return nullptr;
  (void)hipSetDevice(c->dev);
  return dev_alloc(c, bytes);
}

extern "C" void gq_hip_free(gq_ctx *c, void *p) {
  if (!c || !p) return;
  auto it = std::find(c->allocs.begin(), c->allocs.end(), p);
  if (it == c->allocs.end()) return;
  (void)hipStreamSynchronize(c->stream);
  (void)hipFree(p);
  c->allocs.erase(it);
}

extern "C" int gq_hip_h2d(gq_ctx *c, void *dev, const void *host, size_t bytes) {
  if (!c || !dev || !host) return -1;
  HIPCHK(c, hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_d2h(gq_ctx *c, void *host, const void *dev, size_t bytes) {
  if (!c || !dev || !host) return -1;
  HIPCHK(c, hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

/* Host -> device through two pinned staging slots of kStageBytes: the CPU
 * copies chunk i + 1 into one slot while the DMA of chunk i drains the
 * other.  The source is only ever read by the CPU, so a private file mapping
 * (the loader's mmap) never meets the DMA engine, which is why the reference
 * stages through a heap copy (matvec_q4k_cuda.cu:115-133). */
constexpr size_t kStageBytes = (size_t)32 << 20;

static int staged_h2d(gq_ctx *c, void *dst, const void *src, size_t bytes) {
  for (int i = 0; i < 2; i++) {
    if (!c->stage[i] && hipHostMalloc(&c->stage[i], kStageBytes, hipHostMallocDefault) != hipSuccess) {
      c->stage[i] = nullptr;
      return fail(c, -4, "upload: pinned staging buffer");
    }
    if (!c->stage_ev[i] && hipEventCreateWithFlags(&c->stage_ev[i], hipEventDisableTiming) != hipSuccess) {
      c->stage_ev[i] = nullptr;
      return fail(c, -4, "upload: staging event");
    }
  }
  size_t off = 0;
  for (int k = 0; off < bytes; k ^= 1) {
    const size_t n = std::min(kStageBytes, bytes - off);
    HIPCHK(c, hipEventSynchronize(c->stage_ev[k])); /* the slot's previous DMA is done */
    memcpy(c->stage[k], (const char *)src + off, n);
    HIPCHK(c, hipMemcpyAsync((char *)dst + off, c->stage[k], n, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipEventRecord(c->stage_ev[k], c->stream));
    off += n;
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" void *gq_hip_upload_weight(gq_ctx *c, const void *host, size_t bytes) {
  if (!c || !host || !bytes) return nullptr;
  (void)hipSetDevice(c->dev);
  void *d = dev_alloc(c, bytes);
  if (!d) return nullptr;
  if (staged_h2d(c, d, host, bytes) || hipMemsetAsync((char *)d + bytes, 0, kPad, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess) {
    gq_hip_free(c, d);
    fail(c, -4, "weight upload of %zu bytes failed", bytes);
    return nullptr;
  }
  return d;
}

extern "C" int gq_hip_mem_info(int device_id, size_t *free_bytes, size_t *total_bytes) {
  if (device_id < 0 || device_id >= gq_hip_device_count() || hipSetDevice(device_id) != hipSuccess) return -1;
  size_t f = 0, t = 0;
  if (hipMemGetInfo(&f, &t) != hipSuccess) return -4;
  if (free_bytes) *free_bytes = f;
  if (total_bytes) *total_bytes = t;
  return 0;
}

extern "C" void *gq_hip_host_alloc_pinned(size_t bytes) {
  void *p = nullptr;
  if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) return nullptr;
  return p;
}

extern "C" void gq_hip_host_free_pinned(void *p) {
  if (p) (void)hipHostFree(p);
}

/* ------------------------------------------------------------ synthetic */
extern "C" int gq_hip_synth_quant(gq_ctx *c, void *dev, int dtype, int rows, int cols, uint64_t seed) {
  if (!c || !dev || rows <= 0 || cols <= 0) return -1;
  int rc = gq_launch_synth_quant(dev, dtype, rows, cols, seed, c->stream);
  if (rc) return fail(c, rc, "synth_quant: bad dtype/shape");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_synth_normal(gq_ctx *c, float *dev, size_t n, uint64_t seed) {
  if (!c || !dev) return -1;
  if (gq_launch_synth_normal(dev, n, seed, 0, c->stream)) return fail(c, -4, "synth_normal");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_synth_norm_weight(gq_ctx *c, float *dev, size_t n, uint64_t seed) {
  if (!c || !dev) return -1;
  if (gq_launch_synth_normal(dev, n, seed, 1, c->stream)) return fail(c, -4, "synth_norm_weight");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

/* ------------------------------------------------------------ matvec */
static int check_mv(gq_ctx *c, int dtype, const void *w, int rows, int cols, size_t byte_size,
                    const void *x, const void *y) {
  int qk;
  const size_t bb = block_bytes(dtype, &qk);
  if (!w || !x || !y || !bb || rows <= 0 || cols <= 0) return fail(c, -1, "matvec: bad argument");
  if (cols % qk) return fail(c, -2, "matvec: cols %d not a multiple of %d", cols, qk);
  if (byte_size && (size_t)rows * (size_t)(cols / qk) * bb > byte_size)
    return fail(c, -3, "matvec: byte_size %zu too small", byte_size);
  return 0;
}

static int launch_one_mv(gq_ctx *c, int dtype, const void *w, int rows, int cols, const float *x,
                         float *y, const uint8_t *mm = nullptr) {
  MvArgs a{};
  a.seg[0] = MvSeg{(const uint8_t *)w, y, nullptr, rows};
  a.nseg = 1;
  a.cols = cols;
  a.x = x;
  a.mm = mm;
  return gq_launch_matvec(dtype, MV_STORE, a, c->stream);
}

/* The op-level entry points take weights in the reference layout; with the
 * matrix-core kernel selected explicitly (path 2) they tile a copy for the
 * call (freed by the caller with gq_hip_free after the stream is done). */
static const uint8_t *op_tile(gq_ctx *c, int dtype, const void *w, int rows, int cols) {
  if (!gq_matvec_mm_forced() || (dtype != GQ_Q4_K && dtype != GQ_Q6_K)) return nullptr;
  const size_t bytes = gq_mm_tile_bytes(dtype, rows, cols, false);
  if (!bytes) return nullptr;
  uint8_t *d = (uint8_t *)dev_alloc(c, bytes);
  if (d && gq_launch_mm_tile(d, dtype, w, nullptr, rows, cols, c->stream)) {
    gq_hip_free(c, d);
    return nullptr;
  }
  return d;
}

extern "C" int gq_hip_matvec(gq_ctx *c, int dtype, const void *w, int rows, int cols,
                             size_t byte_size, const float *x, float *y) {
  if (!c) return -1;
  int rc = check_mv(c, dtype, w, rows, cols, byte_size, x, y);
  if (rc) return rc;
  if (c->sx_cap < (size_t)cols) {
    float *p = (float *)dev_alloc(c, sizeof(float) * cols);
    if (!p) return -4;
    if (c->sx) gq_hip_free(c, c->sx);
    c->sx = p, c->sx_cap = cols;
  }
  if (c->sy_cap < (size_t)rows) {
    float *p = (float *)dev_alloc(c, sizeof(float) * rows);
    if (!p) return -4;
    if (c->sy) gq_hip_free(c, c->sy);
    c->sy = p, c->sy_cap = rows;
  }
  HIPCHK(c, hipMemcpyAsync(c->sx, x, sizeof(float) * cols, hipMemcpyHostToDevice, c->stream));
  const uint8_t *mm = op_tile(c, dtype, w, rows, cols);
  rc = launch_one_mv(c, dtype, w, rows, cols, c->sx, c->sy, mm);
  if (mm) gq_hip_free(c, (void *)mm);
  if (rc) return fail(c, rc, "matvec launch failed");
  HIPCHK(c, hipMemcpyAsync(y, c->sy, sizeof(float) * rows, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_matvec_dev(gq_ctx *c, int dtype, const void *w, int rows, int cols,
                                 const float *x, float *y) {
  if (!c) return -1;
  int rc = check_mv(c, dtype, w, rows, cols, 0, x, y);
  if (rc) return rc;
  const uint8_t *mm = op_tile(c, dtype, w, rows, cols);
  rc = launch_one_mv(c, dtype, w, rows, cols, x, y, mm);
  if (mm) gq_hip_free(c, (void *)mm);
  return rc ? fail(c, rc, "matvec launch failed") : 0;
}

/* y = W (rmsnorm(x) * norm_w) with the RMSNorm fused into the matvec's x
 * staging, as the decode step runs it before q/k/v, gate/up and the LM head
 * (cpu_rmsnorm + linear_dispatch, engine.c:356-366, :582-590). */
extern "C" int gq_hip_matvec_norm_dev(gq_ctx *c, int dtype, const void *w, int rows, int cols,
                                      const float *x, const float *norm_w, float eps, float *y) {
  if (!c) return -1;
  int rc = check_mv(c, dtype, w, rows, cols, 0, x, y);
  if (rc) return rc;
  if (!norm_w) return fail(c, -1, "matvec_norm: no norm weight");
  const uint8_t *mm = op_tile(c, dtype, w, rows, cols);
  MvArgs a{};
  a.seg[0] = MvSeg{(const uint8_t *)w, y, nullptr, rows};
  a.nseg = 1, a.cols = cols, a.x = x, a.norm_w = norm_w, a.eps = eps, a.mm = mm;
  rc = gq_launch_matvec(dtype, MV_STORE, a, c->stream);
  if (mm) gq_hip_free(c, (void *)mm);
  return rc ? fail(c, rc, "matvec_norm launch failed") : 0;
}

/* ------------------------------------------------------------ KV cache */
static size_t layer_floats(const gq_ctx *c) {
  return (size_t)c->kv_heads * c->kv_max_seq * c->kv_hd;
}

/* Free the K/V slabs and the RoPE table and forget the cache geometry: every
 * entry point that checks c->kslab then sees no cache. */
static void kv_release(gq_ctx *c) {
  (void)hipStreamSynchronize(c->stream);
  if (c->kslab) gq_hip_free(c, c->kslab);
  if (c->vslab) gq_hip_free(c, c->vslab);
  if (c->rope) gq_hip_free(c, c->rope);
  c->kslab = c->vslab = nullptr;
  c->rope = nullptr;
  c->kv_layers = c->kv_heads = c->kv_hd = c->kv_max_seq = 0;
  c->bound = c->whole = false;
}

extern "C" int gq_hip_kv_init(gq_ctx *c, int n_layers, int n_kv_heads, int head_dim, int max_seq,
                              float rope_theta) {
  if (!c || n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 || (head_dim & 1) || max_seq <= 0)
    return fail(c, -1, "kv_init: bad geometry");
  (void)hipSetDevice(c->dev);
  kv_release(c);
  free_graph(c);
  c->bound = c->whole = false;
  const size_t bytes = sizeof(float) * (size_t)n_kv_heads * max_seq * head_dim * n_layers;
  const size_t half = (size_t)head_dim / 2;
  c->kslab = (float *)dev_alloc(c, bytes);
  c->vslab = (float *)dev_alloc(c, bytes);
  c->rope = (float2 *)dev_alloc(c, sizeof(float2) * half * max_seq);
  if (!c->kslab || !c->vslab || !c->rope) { /* nothing half-made stays behind */
    kv_release(c);
    return fail(c, -4, "kv_init: out of device memory for %zu-byte K/V slabs", bytes);
  }
  c->kv_layers = n_layers, c->kv_heads = n_kv_heads, c->kv_hd = head_dim, c->kv_max_seq = max_seq;
  c->theta = rope_theta;
  /* zeroed like kv_cache_create (kv_cache.c:73-75) */
  if (hipMemsetAsync(c->kslab, 0, bytes, c->stream) != hipSuccess ||
      hipMemsetAsync(c->vslab, 0, bytes, c->stream) != hipSuccess) {
    kv_release(c);
    return fail(c, -4, "kv_init: clearing the K/V slabs failed");
  }
  /* RoPE table with the reference's fp32 expressions (kernels_cpu.c:409-413) */
  std::vector<float2> tab(half * max_seq);
  std::vector<float> freq(half);
  for (size_t i = 0; i < half; i++)
    freq[i] = 1.0f / powf(rope_theta, (float)(2 * i) / (float)head_dim);
  for (int p = 0; p < max_seq; p++)
    for (size_t i = 0; i < half; i++) {
      const float a = (float)p * freq[i];
      tab[(size_t)p * half + i] = make_float2(cosf(a), sinf(a));
    }
  if (hipMemcpyAsync(c->rope, tab.data(), sizeof(float2) * tab.size(), hipMemcpyHostToDevice, c->stream) !=
          hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess) {
    kv_release(c);
    return fail(c, -4, "kv_init: uploading the RoPE table failed");
  }
  return 0;
}

extern "C" float *gq_hip_kv_k(gq_ctx *c, int layer) {
  if (!c || !c->kslab || layer < 0 || layer >= c->kv_layers) return nullptr;
  return c->kslab + layer_floats(c) * layer;
}

extern "C" float *gq_hip_kv_v(gq_ctx *c, int layer) {
  if (!c || !c->vslab || layer < 0 || layer >= c->kv_layers) return nullptr;
  return c->vslab + layer_floats(c) * layer;
}

extern "C" int gq_hip_kv_append(gq_ctx *c, int layer, int pos, const float *k, const float *v) {
  if (!c || !c->kslab || !k || !v) return fail(c, -1, "kv_append: not initialised / NULL");
  if (layer < 0 || layer >= c->kv_layers) return fail(c, -1, "kv_append: bad layer %d", layer);
  if (pos < 0) return fail(c, -5, "kv_append: negative position %d", pos);
  const int p = pos % c->kv_max_seq; /* ring wrap of kv_cache.c:101 */
  const size_t hd = c->kv_hd, row = sizeof(float) * hd, pitch = row * c->kv_max_seq;
  float *kd = gq_hip_kv_k(c, layer) + (size_t)p * hd, *vd = gq_hip_kv_v(c, layer) + (size_t)p * hd;
  HIPCHK(c, hipMemcpy2DAsync(kd, pitch, k, row, row, c->kv_heads, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipMemcpy2DAsync(vd, pitch, v, row, row, c->kv_heads, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_kv_read_layer(gq_ctx *c, int layer, float *k, float *v) {
  if (!c || !c->kslab || layer < 0 || layer >= c->kv_layers) return fail(c, -1, "kv_read_layer");
  const size_t bytes = sizeof(float) * layer_floats(c);
  if (k) HIPCHK(c, hipMemcpyAsync(k, gq_hip_kv_k(c, layer), bytes, hipMemcpyDeviceToHost, c->stream));
  if (v) HIPCHK(c, hipMemcpyAsync(v, gq_hip_kv_v(c, layer), bytes, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_kv_write_layer(gq_ctx *c, int layer, const float *k, const float *v) {
  if (!c || !c->kslab || layer < 0 || layer >= c->kv_layers) return fail(c, -1, "kv_write_layer");
  const size_t bytes = sizeof(float) * layer_floats(c);
  if (k) HIPCHK(c, hipMemcpyAsync(gq_hip_kv_k(c, layer), k, bytes, hipMemcpyHostToDevice, c->stream));
  if (v) HIPCHK(c, hipMemcpyAsync(gq_hip_kv_v(c, layer), v, bytes, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_kv_sync(gq_ctx *c, int layer, int pos, int T, const float *h_k,
                              const float *h_v, int head_stride, int max_seq) {
  if (!c || !c->kslab || !h_k || !h_v || T <= 0) return fail(c, -1, "kv_sync: bad argument");
  if (layer < 0 || layer >= c->kv_layers || max_seq != c->kv_max_seq)
    return fail(c, -1, "kv_sync: layer/max_seq mismatch");
  if (pos < 0 || pos + T > c->kv_max_seq) return fail(c, -5, "kv_sync: rows outside the cache");
  const size_t hd = c->kv_hd, w = sizeof(float) * hd * T;
  const size_t dpitch = sizeof(float) * hd * c->kv_max_seq, spitch = sizeof(float) * head_stride;
  HIPCHK(c, hipMemcpy2DAsync(gq_hip_kv_k(c, layer) + pos * hd, dpitch, h_k + pos * hd, spitch, w,
                             c->kv_heads, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipMemcpy2DAsync(gq_hip_kv_v(c, layer) + pos * hd, dpitch, h_v + pos * hd, spitch, w,
                             c->kv_heads, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_kv_fetch(gq_ctx *c, int layer, int pos, int T, float *h_k, float *h_v, int head_stride,
                               int max_seq) {
  if (!c || !c->kslab || !h_k || !h_v || T <= 0) return fail(c, -1, "kv_fetch: bad argument");
  if (layer < 0 || layer >= c->kv_layers || max_seq != c->kv_max_seq)
    return fail(c, -1, "kv_fetch: layer/max_seq mismatch");
  if (pos < 0 || pos + T > c->kv_max_seq) return fail(c, -5, "kv_fetch: rows outside the cache");
  const size_t hd = c->kv_hd, w = sizeof(float) * hd * T;
  const size_t spitch = sizeof(float) * hd * c->kv_max_seq, dpitch = sizeof(float) * head_stride;
  HIPCHK(c, hipMemcpy2DAsync(h_k + pos * hd, dpitch, gq_hip_kv_k(c, layer) + pos * hd, spitch, w, c->kv_heads,
                             hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipMemcpy2DAsync(h_v + pos * hd, dpitch, gq_hip_kv_v(c, layer) + pos * hd, spitch, w, c->kv_heads,
                             hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_kv_prefill_synth(gq_ctx *c, uint64_t seed_k, uint64_t seed_v, int n_pos) {
  if (!c || !c->kslab) return fail(c, -1, "kv_prefill_synth: no cache");
  if (n_pos < 0 || n_pos > c->kv_max_seq) return fail(c, -5, "kv_prefill_synth: n_pos");
  if (gq_launch_synth_kv(c->kslab, c->kv_layers, c->kv_heads, c->kv_hd, c->kv_max_seq, n_pos, seed_k,
                         c->stream) ||
      gq_launch_synth_kv(c->vslab, c->kv_layers, c->kv_heads, c->kv_hd, c->kv_max_seq, n_pos, seed_v,
                         c->stream))
    return fail(c, -4, "kv_prefill_synth launch");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

/* ------------------------------------------------------------ .lctx */
namespace {
#pragma pack(push, 1)
struct LctxHeader { /* session.c:36-48 */
  uint32_t magic, version;
  int32_t n_layers, n_kv_heads, head_dim, max_seq, current_pos, n_tokens;
  uint8_t reserved[32];
};
#pragma pack(pop)
static_assert(sizeof(LctxHeader) == 64, "lctx header is 64 bytes");
constexpr uint32_t kLctxMagic = 0x5843544Cu, kLctxVersion = 1;
} // namespace

static int check_header(gq_ctx *c, const LctxHeader &h) {
  if (h.magic != kLctxMagic) return fail(c, -1, "lctx: bad magic");
  if (h.version != kLctxVersion) return fail(c, -1, "lctx: unsupported version %u", h.version);
  if (h.n_layers != c->kv_layers || h.n_kv_heads != c->kv_heads || h.head_dim != c->kv_hd)
    return fail(c, -1, "lctx: model geometry mismatch");
  if (h.max_seq != c->kv_max_seq) return fail(c, -1, "lctx: max_seq mismatch");
  if (h.n_tokens < 0) return fail(c, -1, "lctx: negative token count");
  return 0;
}

extern "C" int gq_hip_lctx_save(gq_ctx *c, const char *path, int current_pos, const int32_t *tokens,
                                int n_tokens) {
  if (!c || !c->kslab || !path) return fail(c, -1, "lctx_save: bad argument");
  FILE *f = fopen(path, "wb");
  if (!f) return fail(c, -1, "lctx_save: cannot open %s", path);
  LctxHeader h;
  memset(&h, 0, sizeof h);
  h.magic = kLctxMagic, h.version = kLctxVersion;
  h.n_layers = c->kv_layers, h.n_kv_heads = c->kv_heads, h.head_dim = c->kv_hd;
  h.max_seq = c->kv_max_seq, h.current_pos = current_pos, h.n_tokens = n_tokens;
  const size_t lb = sizeof(float) * layer_floats(c);
  void *buf = gq_hip_host_alloc_pinned(lb);
  int rc = 0;
  if (!buf) rc = fail(c, -4, "lctx_save: pinned buffer");
  if (!rc && fwrite(&h, sizeof h, 1, f) != 1) rc = fail(c, -1, "lctx_save: write");
  if (!rc && n_tokens > 0 && tokens &&
      fwrite(tokens, sizeof(int32_t), (size_t)n_tokens, f) != (size_t)n_tokens)
    rc = fail(c, -1, "lctx_save: write");
  for (int which = 0; which < 2 && !rc; which++)
    for (int l = 0; l < c->kv_layers && !rc; l++) {
      const float *src = which ? gq_hip_kv_v(c, l) : gq_hip_kv_k(c, l);
      if (hipMemcpyAsync(buf, src, lb, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
          hipStreamSynchronize(c->stream) != hipSuccess)
        rc = fail(c, -4, "lctx_save: device gather");
      else if (fwrite(buf, 1, lb, f) != lb)
        rc = fail(c, -1, "lctx_save: write");
    }
  gq_hip_host_free_pinned(buf);
  fclose(f);
  return rc;
}

extern "C" int gq_hip_lctx_load(gq_ctx *c, const char *path, int *current_pos, int32_t **tokens,
                                int *n_tokens) {
  if (!c || !c->kslab || !path) return fail(c, -1, "lctx_load: bad argument");
  FILE *f = fopen(path, "rb");
  if (!f) return fail(c, -1, "lctx_load: cannot open %s", path);
  LctxHeader h;
  int rc = fread(&h, sizeof h, 1, f) == 1 ? check_header(c, h) : fail(c, -1, "lctx_load: short header");
  int32_t *tok = nullptr;
  if (!rc && h.n_tokens > 0) {
    tok = (int32_t *)malloc(sizeof(int32_t) * h.n_tokens);
    if (!tok || fread(tok, sizeof(int32_t), (size_t)h.n_tokens, f) != (size_t)h.n_tokens)
      rc = fail(c, -1, "lctx_load: short token block");
  }
  const size_t lb = sizeof(float) * layer_floats(c);
  void *buf = rc ? nullptr : gq_hip_host_alloc_pinned(lb);
  if (!rc && !buf) rc = fail(c, -4, "lctx_load: pinned buffer");
  for (int which = 0; which < 2 && !rc; which++)
    for (int l = 0; l < c->kv_layers && !rc; l++) {
      float *dst = which ? gq_hip_kv_v(c, l) : gq_hip_kv_k(c, l);
      if (fread(buf, 1, lb, f) != lb)
        rc = fail(c, -1, "lctx_load: short K/V block");
      else if (hipMemcpyAsync(dst, buf, lb, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
               hipStreamSynchronize(c->stream) != hipSuccess)
        rc = fail(c, -4, "lctx_load: device restore");
    }
  gq_hip_host_free_pinned(buf);
  fclose(f);
  if (rc) {
    free(tok);
    return rc;
  }
  if (current_pos) *current_pos = h.current_pos;
  if (n_tokens) *n_tokens = h.n_tokens;
  if (tokens) *tokens = tok;
  else free(tok);
  return 0;
}

/* The frozen-prefix prompt cache (session.c:192-251): the .lctx format with
 * current_pos = prefix_len and no token history, every layer at the full
 * max_seq stride; load is kv_cache_load without the tokens. */
extern "C" int gq_hip_prompt_cache_save(gq_ctx *c, int prefix_len, const char *path) {
  if (!c || !path || prefix_len <= 0) return fail(c, -1, "prompt_cache_save: bad argument");
  return gq_hip_lctx_save(c, path, prefix_len, nullptr, 0);
}

extern "C" int gq_hip_prompt_cache_load(gq_ctx *c, const char *path, int *prefix_len) {
  return gq_hip_lctx_load(c, path, prefix_len, nullptr, nullptr);
}

extern "C" int gq_hip_lctx_restore_image(gq_ctx *c, const void *image, size_t size, int *current_pos,
                                         float *ms) {
  if (!c || !c->kslab || !image || size < sizeof(LctxHeader)) return fail(c, -1, "lctx_restore");
  LctxHeader h;
  memcpy(&h, image, sizeof h);
  int rc = check_header(c, h);
  if (rc) return rc;
  const size_t slab = sizeof(float) * layer_floats(c) * c->kv_layers;
  const size_t off = sizeof h + sizeof(int32_t) * (size_t)h.n_tokens;
  if (size < off + 2 * slab) return fail(c, -1, "lctx_restore: short image");
  /* the image's K and V regions are laid out exactly like the device slabs */
  EventPair ev;
  HIPCHK(c, ev.create());
  HIPCHK(c, hipEventRecord(ev.e0, c->stream));
  HIPCHK(c, hipMemcpyAsync(c->kslab, (const char *)image + off, slab, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(c->vslab, (const char *)image + off + slab, slab, hipMemcpyHostToDevice,
                           c->stream));
  HIPCHK(c, hipEventRecord(ev.e1, c->stream));
  HIPCHK(c, hipEventSynchronize(ev.e1));
  if (ms) *ms = ev.ms();
  if (current_pos) *current_pos = h.current_pos;
  return 0;
}

/* ------------------------------------------------------------ model */
static int check_weight(gq_ctx *c, const gq_weight &w, int rows, int cols, const char *what) {
  int qk;
  if (!w.data || !block_bytes(w.dtype, &qk)) return fail(c, -1, "%s: missing or bad dtype", what);
  if (w.rows != rows || w.cols != cols) return fail(c, -1, "%s: shape %dx%d, expected %dx%d", what, w.rows, w.cols, rows, cols);
  if (cols % qk) return fail(c, -2, "%s: cols %% block", what);
  return 0;
}

static bool mm_tileable(const gq_weight &w) {
  return (w.dtype == GQ_Q4_K || w.dtype == GQ_Q6_K) && w.cols % 256 == 0 && w.rows > 0;
}

/* One tile-interleaved tensor for the weights ws[0..n) (stacked in order,
 * each rows % 16 == 0 when n > 1), or for gate and up together (swiglu);
 * NULL when they do not take the layout or memory runs out. */
static const uint8_t *mm_build(gq_ctx *c, const gq_weight *const *ws, int n, bool swiglu) {
  size_t bytes = 0;
  for (int i = 0; i < n; i++) {
    if (!mm_tileable(*ws[i]) || ws[i]->dtype != ws[0]->dtype || ws[i]->cols != ws[0]->cols) return nullptr;
    if (n > 1 && !swiglu && ws[i]->rows % 16) return nullptr;
  }
  if (swiglu) {
    if (n != 2 || ws[0]->rows != ws[1]->rows) return nullptr;
    bytes = gq_mm_tile_bytes(ws[0]->dtype, ws[0]->rows, ws[0]->cols, true);
  } else {
    for (int i = 0; i < n; i++) bytes += gq_mm_tile_bytes(ws[i]->dtype, ws[i]->rows, ws[i]->cols, false);
  }
  uint8_t *d = (uint8_t *)dev_alloc(c, bytes);
  if (!d) return nullptr;
  if (swiglu) {
    if (gq_launch_mm_tile(d, ws[0]->dtype, ws[0]->data, ws[1]->data, ws[0]->rows, ws[0]->cols, c->stream)) return nullptr;
    return d;
  }
  size_t off = 0;
  for (int i = 0; i < n; i++) {
    if (gq_launch_mm_tile(d + off, ws[i]->dtype, ws[i]->data, nullptr, ws[i]->rows, ws[i]->cols, c->stream))
      return nullptr;
    off += gq_mm_tile_bytes(ws[i]->dtype, ws[i]->rows, ws[i]->cols, false);
  }
  return d;
}

static void mm_free(gq_ctx *c) {
  auto rel = [&](const uint8_t *&p) {
    if (p) gq_hip_free(c, (void *)p);
    p = nullptr;
  };
  for (auto &L : c->mm) {
    if (L.ux[6] == L.dx) L.ux[6] = nullptr; /* one allocation */
    rel(L.gu), rel(L.dx);
    for (auto &p : L.ux) rel(p);
  }
  c->mm.clear();
  rel(c->mm_lm);
}

extern "C" int gq_hip_model_bind(gq_ctx *c, const gq_model *m) {
  if (!c || !m || !m->layers) return fail(c, -1, "model_bind: NULL");
  if (!c->kslab) return fail(c, -1, "model_bind: call gq_hip_kv_init first");
  if (m->n_layers != c->kv_layers || m->n_kv_heads != c->kv_heads || m->head_dim != c->kv_hd)
    return fail(c, -1, "model_bind: model and KV geometry differ");
  if (m->n_heads % m->n_kv_heads || m->hidden != m->n_heads * m->head_dim)
    return fail(c, -1, "model_bind: head geometry");
  {
    const int G = m->n_heads / m->n_kv_heads;
    if ((m->head_dim != 64 && m->head_dim != 128) || (G != 1 && G != 2 && G != 4 && G != 8))
      return fail(c, -1, "model_bind: attention kernels take head_dim 64 or 128 with 1, 2, 4 or 8 query heads per KV head (got %d, %d)",
                  m->head_dim, G);
  }
  if ((m->hidden & 255) || (m->ff & 255))
    return fail(c, -1, "model_bind: hidden and ff must be multiples of 256");
  const int H = m->hidden, F = m->ff, kvd = m->n_kv_heads * m->head_dim;
  /* A layer whose seven projections and norm weights are all NULL stays on
   * the host (the --n-gpu-layers split, or a projection the device kernels
   * do not take); so may the LM head and the embedding (an F32 LM head, for
   * one).  Anything in between is an error. */
  std::vector<char> on(m->n_layers, 0);
  for (int l = 0; l < m->n_layers; l++) {
    const gq_layer &L = m->layers[l];
    const void *ps[9] = {L.wq.data, L.wk.data, L.wv.data, L.wo.data, L.w_gate.data, L.w_up.data, L.w_down.data,
                         L.rms_att, L.rms_ffn};
    int n_set = 0;
    for (const void *p : ps) n_set += p != nullptr;
    if (n_set == 0) continue;
    int rc = check_weight(c, L.wq, H, H, "wq") || check_weight(c, L.wk, kvd, H, "wk") ||
             check_weight(c, L.wv, kvd, H, "wv") || check_weight(c, L.wo, H, H, "wo") ||
             check_weight(c, L.w_gate, F, H, "w_gate") || check_weight(c, L.w_up, F, H, "w_up") ||
             check_weight(c, L.w_down, H, F, "w_down");
    if (rc) return fail(c, -1, "layer %d: %s", l, c->err);
    if (!L.rms_att || !L.rms_ffn) return fail(c, -1, "layer %d: norm weights", l);
    on[l] = 1;
  }
  const bool has_lm = m->lm_head.data != nullptr, has_embed = m->embed.data != nullptr;
  if (has_lm && check_weight(c, m->lm_head, m->vocab, H, "lm_head")) return -1;
  if (has_embed && (m->embed.rows != m->vocab || m->embed.cols != H ||
                    (m->embed.dtype != GQ_F32 && m->embed.dtype != GQ_Q8_0 && m->embed.dtype != GQ_Q4_K)))
    return fail(c, -1, "embed: F32, Q8_0 or Q4_K (vocab x hidden)");
  if (has_lm && !m->rms_final) return fail(c, -1, "rms_final");
  free_graph(c);
  pf_release(c); /* sized for the previous model */
  c->m = *m;
  c->layers.assign(m->layers, m->layers + m->n_layers);
  c->m.layers = c->layers.data();
  c->layer_on = on;
  c->whole = has_lm && has_embed && m->rms_final;
  for (char o : on) c->whole = c->whole && o;
  /* tile-interleaved copies for the matrix-core matvec, for the launches
   * the decode step runs on it (gate/up + SwiGLU, the LM head); ordered on
   * the stream after whatever wrote the weights */
  mm_free(c);
  c->mm.resize(m->n_layers);
  for (int l = 0; l < m->n_layers; l++) {
    if (!on[l]) continue;
    const gq_layer &L = c->layers[l];
    const gq_weight *gu[2] = {&L.w_gate, &L.w_up};
    if (L.w_gate.dtype == L.w_up.dtype) c->mm[l].gu = mm_build(c, gu, 2, true);
    /* the down projection's Q6_K rows re-laid out so 8-row groups fit the
     * vector-ALU kernel's registers (one round of workgroups) */
    if (L.w_down.dtype == GQ_Q6_K && L.w_down.cols % 512 == 0) {
      uint8_t *d = (uint8_t *)dev_alloc(c, gq_q6k_units_bytes(L.w_down.rows, L.w_down.cols));
      if (d && gq_launch_q6k_units(d, L.w_down.data, L.w_down.rows, L.w_down.cols, c->stream) == 0) c->mm[l].dx = d;
      else if (d) gq_hip_free(c, d);
    }
    /* the prefill GEMM reads Q6_K projections whose rows fall on 16-byte
     * boundaries in the same unit layout, where a step's quant bytes are one
     * 16-byte-aligned range: the down projection's copy above, one of their
     * own for the others */
    const gq_weight *pw[7] = {&L.wq, &L.wk, &L.wv, &L.wo, &L.w_gate, &L.w_up, &L.w_down};
    for (int i = 0; i < 7; i++) {
      const gq_weight &g = *pw[i];
      if (g.dtype != GQ_Q6_K || g.cols % 2048 || g.rows % 128) continue;
      if (i == 6) {
        c->mm[l].ux[6] = c->mm[l].dx;
        continue;
      }
      uint8_t *d = (uint8_t *)dev_alloc(c, gq_q6k_units_bytes(g.rows, g.cols));
      if (d && gq_launch_q6k_units(d, g.data, g.rows, g.cols, c->stream) == 0) c->mm[l].ux[i] = d;
      else if (d) gq_hip_free(c, d);
    }
  }
  if (has_lm) {
    const gq_weight *lm[1] = {&m->lm_head};
    c->mm_lm = mm_build(c, lm, 1, false);
  }
  Workspace &w = c->ws;
  w.nch = gq_attn_nch(m->n_kv_heads, c->kv_max_seq);
  w.s_max = gq_attn_smax(c->kv_max_seq, w.nch);
  w.amax_blocks = gq_argmax_blocks(m->vocab);
  auto need = [&](float *&p, size_t n) -> bool {
    if (p) gq_hip_free(c, p);
    p = (float *)dev_alloc(c, sizeof(float) * n);
    return p != nullptr;
  };
  if (!need(w.hidden, H) || !need(w.qkv, H + 2 * kvd) || !need(w.attn, H) || !need(w.act, F) ||
      !need(w.act2, F) || !need(w.logits, m->vocab) ||
      !need(w.part_o, (size_t)m->n_heads * w.nch * m->head_dim) ||
      !need(w.part_ml, (size_t)m->n_heads * w.nch * 2) || !need(w.amax, 2 * (size_t)w.amax_blocks))
    return -4;
  w.part_cap = (size_t)m->n_heads * w.nch * m->head_dim;
  w.part_ml_cap = (size_t)m->n_heads * w.nch * 2;
  if (!w.d_token) {
    w.d_token = (int *)dev_alloc(c, 4 * sizeof(int));
    if (!w.d_token) return -4;
    w.d_pos = w.d_token + 1;
    w.d_step = w.d_token + 2;
  }
  c->bound = true;
  return 0;
}

/* ---- eager-step measurement hooks ---- */
static hipEvent_t next_event(gq_ctx *c) {
  hipEvent_t e;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  c->ev.push_back(e);
  return e;
}

static void mark(gq_ctx *c, int cls, double bytes) {
  if (!c->prof) return;
  hipEvent_t e = next_event(c);
  if (!e) return;
  (void)hipEventRecord(e, c->stream);
  c->ev_class.push_back(cls);
  c->ev_bytes.push_back(bytes);
}

static double mv_bytes(const gq_weight &w, int extra_vectors) {
  int qk;
  const size_t bb = block_bytes(w.dtype, &qk);
  return (double)w.rows * (w.cols / qk) * bb + 4.0 * w.cols + 4.0 * w.rows * (1 + extra_vectors);
}

/* The launches of one decode layer, op by op; positions come from pos_dev
 * when not NULL. */
/* q, k, v: one launch per distinct dtype, RMSNorm fused into the x staging;
 * RoPE of q and k and the K/V cache append fused into the epilogue
 * (engine.c:356-392 in one pass) */
static int op_qkv(gq_ctx *c, int l, int pos, const int *pos_dev, float *hidden) {
  const gq_model &m = c->m;
  const gq_layer &L = c->layers[l];
  const gq_weight *W[3] = {&L.wq, &L.wk, &L.wv};
  float *Y[3] = {c->ws.qkv, gq_hip_kv_k(c, l), gq_hip_kv_v(c, l)};
  const int kind[3] = {SEG_ROPE, SEG_ROPE_KV, SEG_KV};
  bool done[3] = {false, false, false};
  MvArgs g[3];
  int gdt[3], ng = 0;
  double bytes = 4.0 * m.hidden;
  for (int i = 0; i < 3; i++) {
    if (done[i]) continue;
    MvArgs &a = g[ng];
    a = MvArgs{};
    gdt[ng++] = W[i]->dtype;
    a.cols = m.hidden, a.x = hidden, a.norm_w = L.rms_att, a.eps = m.rms_eps;
    a.rope = MvRope{c->rope, pos_dev, pos, m.head_dim, c->kv_max_seq};
    for (int j = i; j < 3; j++)
      if (!done[j] && W[j]->dtype == W[i]->dtype) {
        a.seg[a.nseg++] = MvSeg{(const uint8_t *)W[j]->data, Y[j], nullptr, W[j]->rows, kind[j]};
        bytes += mv_bytes(*W[j], 0) - 4.0 * m.hidden;
        done[j] = true;
      }
  }
  /* Q4_K q, k and Q6_K v (the Q4_K_M mix): one paired launch, v from its
   * unit-layout copy where bind made one */
  if (ng == 2) {
    if (gdt[1] == GQ_Q6_K && g[1].nseg == 1 && g[1].seg[0].w == (const uint8_t *)L.wv.data && (size_t)l < c->mm.size() &&
        !gq_matvec_q6k_ref())
      g[1].dx = c->mm[l].ux[2];
    const int rc = gq_launch_matvec_pair(gdt[0], g[0], gdt[1], g[1], c->stream);
    if (rc <= 0) {
      if (rc == 0) mark(c, PC_QKV, bytes);
      return rc;
    }
  }
  for (int k = 0; k < ng; k++) {
    const int rc = gq_launch_matvec(gdt[k], MV_STORE, g[k], c->stream);
    if (rc) return rc;
  }
  mark(c, PC_QKV, bytes);
  return 0;
}

static int op_attention(gq_ctx *c, int l, int pos, const int *pos_dev) {
  const gq_model &m = c->m;
  Workspace &w = c->ws;
  const int kvd = m.n_kv_heads * m.head_dim;
  AttnArgs aa{};
  aa.q = w.qkv, aa.k = gq_hip_kv_k(c, l), aa.v = gq_hip_kv_v(c, l);
  aa.part_o = w.part_o, aa.part_ml = w.part_ml, aa.out = w.attn;
  aa.pos_dev = pos_dev, aa.pos = pos;
  aa.n_heads = m.n_heads, aa.n_kv = m.n_kv_heads, aa.hd = m.head_dim, aa.max_seq = c->kv_max_seq;
  aa.nch = w.nch, aa.s_max = w.s_max, aa.scale = 1.0f / sqrtf((float)m.head_dim);
  const int rc = gq_launch_attention(aa, c->stream, nullptr);
  if (rc) return rc;
  mark(c, PC_ATTN, 2.0 * 4.0 * kvd * (double)(std::min(pos + 1, c->kv_max_seq)) + 8.0 * m.hidden);
  return 0;
}

/* o-proj + residual (in place on hidden) */
static int op_o(gq_ctx *c, int l, float *hidden) {
  const gq_layer &L = c->layers[l];
  MvArgs a{};
  a.seg[0] = MvSeg{(const uint8_t *)L.wo.data, hidden, hidden, L.wo.rows};
  a.nseg = 1, a.cols = L.wo.cols, a.x = c->ws.attn;
  const int rc = gq_launch_matvec(L.wo.dtype, MV_RESID, a, c->stream);
  if (rc) return rc;
  mark(c, PC_O, mv_bytes(L.wo, 1));
  return 0;
}

/* gate/up + SwiGLU, RMSNorm fused */
static int op_gate_up(gq_ctx *c, int l, float *hidden) {
  const gq_model &m = c->m;
  const gq_layer &L = c->layers[l];
  Workspace &w = c->ws;
  int rc;
  if (L.w_gate.dtype == L.w_up.dtype) {
    MvArgs a{};
    a.seg[0] = MvSeg{(const uint8_t *)L.w_gate.data, w.act, nullptr, L.w_gate.rows};
    a.seg[1] = MvSeg{(const uint8_t *)L.w_up.data, nullptr, nullptr, L.w_up.rows};
    a.nseg = 2, a.cols = m.hidden, a.x = hidden, a.norm_w = L.rms_ffn, a.eps = m.rms_eps;
    a.mm = (size_t)l < c->mm.size() ? c->mm[l].gu : nullptr;
    if ((rc = gq_launch_matvec(L.w_gate.dtype, MV_SWIGLU, a, c->stream))) return rc;
    mark(c, PC_GATE_UP, mv_bytes(L.w_gate, 0) + mv_bytes(L.w_up, 0) - 4.0 * m.hidden - 4.0 * m.ff);
    return 0;
  }
  for (int i = 0; i < 2; i++) {
    const gq_weight &g = i ? L.w_up : L.w_gate;
    MvArgs a{};
    a.seg[0] = MvSeg{(const uint8_t *)g.data, i ? w.act2 : w.act, nullptr, g.rows};
    a.nseg = 1, a.cols = m.hidden, a.x = hidden, a.norm_w = L.rms_ffn, a.eps = m.rms_eps;
    if ((rc = gq_launch_matvec(g.dtype, MV_STORE, a, c->stream))) return rc;
    mark(c, PC_GATE_UP, mv_bytes(g, 0));
  }
  if ((rc = gq_launch_silu_mul(w.act, w.act2, m.ff, c->stream))) return rc;
  mark(c, PC_GATE_UP, 12.0 * m.ff);
  return 0;
}

/* down + residual (in place on hidden) */
static int op_down(gq_ctx *c, int l, float *hidden) {
  const gq_layer &L = c->layers[l];
  MvArgs a{};
  a.seg[0] = MvSeg{(const uint8_t *)L.w_down.data, hidden, hidden, L.w_down.rows};
  a.nseg = 1, a.cols = L.w_down.cols, a.x = c->ws.act;
  a.dx = (size_t)l < c->mm.size() ? c->mm[l].dx : nullptr;
  const int rc = gq_launch_matvec(L.w_down.dtype, MV_RESID, a, c->stream);
  if (rc) return rc;
  mark(c, PC_DOWN, mv_bytes(L.w_down, 1));
  return 0;
}

/* final RMSNorm fused into the LM head */
static int op_lm_head(gq_ctx *c, float *hidden) {
  const gq_model &m = c->m;
  MvArgs a{};
  a.seg[0] = MvSeg{(const uint8_t *)m.lm_head.data, c->ws.logits, nullptr, m.lm_head.rows};
  a.nseg = 1, a.cols = m.hidden, a.x = hidden, a.norm_w = m.rms_final, a.eps = m.rms_eps;
  a.mm = c->mm_lm;
  const int rc = gq_launch_matvec(m.lm_head.dtype, MV_STORE, a, c->stream);
  if (rc) return rc;
  mark(c, PC_LM_HEAD, mv_bytes(m.lm_head, 0));
  return 0;
}

static int run_layer(gq_ctx *c, int l, int pos, const int *pos_dev, float *hidden) {
  int rc;
  if ((rc = op_qkv(c, l, pos, pos_dev, hidden))) return rc;
  if ((rc = op_attention(c, l, pos, pos_dev))) return rc;
  if ((rc = op_o(c, l, hidden))) return rc;
  if ((rc = op_gate_up(c, l, hidden))) return rc;
  return op_down(c, l, hidden);
}

/* embedding -> layers -> final RMSNorm + LM head -> argmax.  Eager form
 * (token/pos host values) or graph form (device token/pos/step).  The graph
 * form starts from the embedding already in w.hidden and leaves the next
 * token's there: its argmax launch writes it, and gq_hip_decode_loop embeds
 * the first token before the first step. */
static int run_step(gq_ctx *c, int token, int pos, bool device_state, float *hidden_per_layer) {
  const gq_model &m = c->m;
  Workspace &w = c->ws;
  int rc;
  const int *pos_dev = device_state ? w.d_pos : nullptr;
  if (!device_state) c->g_valid = false; /* w.hidden and d_token take this step's values */
  if (!device_state) {
    if ((rc = gq_launch_embed(m.embed.dtype, m.embed.data, m.hidden, nullptr, token, w.hidden, c->stream)))
      return rc;
    mark(c, PC_OTHER, 4.0 * m.hidden);
  }
  for (int l = 0; l < m.n_layers; l++) {
    if ((rc = run_layer(c, l, pos, pos_dev, w.hidden))) return rc;
    if (hidden_per_layer)
      HIPCHK(c, hipMemcpyAsync(hidden_per_layer + (size_t)l * m.hidden, w.hidden, sizeof(float) * m.hidden,
                               hipMemcpyDeviceToHost, c->stream));
  }
  if ((rc = op_lm_head(c, w.hidden))) return rc;
  if ((rc = gq_launch_argmax(w.logits, m.vocab, w.amax, w.amax_blocks, w.d_token,
                             device_state ? w.d_tokens : nullptr, device_state ? w.d_step : nullptr,
                             device_state ? w.d_pos : nullptr, c->stream, m.embed.dtype, m.embed.data, m.hidden,
                             device_state ? w.hidden : nullptr)))
    return rc;
  mark(c, PC_OTHER, 4.0 * m.vocab);
  return 0;
}

/* Positions pos .. pos+n-1 of a whole-model entry point (every layer, the
 * embedding and the LM head on the device). */
static int check_pos(gq_ctx *c, int pos, int n) {
  if (!c->bound) return fail(c, -1, "no model bound");
  if (!c->whole)
    return fail(c, -1, "the bound model is not wholly on the device (host layers, LM head or embedding)");
  if (pos < 0 || pos + n > c->kv_max_seq)
    return fail(c, -5, "positions %d..%d outside the KV cache (max_seq %d)", pos, pos + n - 1, c->kv_max_seq);
  return 0;
}

/* One bound layer at one position (the per-layer hook). */
static int check_layer_pos(gq_ctx *c, int layer, int pos) {
  if (!c->bound) return fail(c, -1, "no model bound");
  if (layer < 0 || layer >= c->m.n_layers) return fail(c, -1, "bad layer %d", layer);
  if (!c->layer_on[layer]) return fail(c, -1, "layer %d is not on the device", layer);
  if (pos < 0 || pos >= c->kv_max_seq)
    return fail(c, -5, "position %d outside the KV cache (max_seq %d)", pos, c->kv_max_seq);
  return 0;
}

extern "C" int gq_hip_decode_layer_dev(gq_ctx *c, int layer, int pos, float *hidden) {
  if (!c || !hidden) return -1;
  int rc = check_layer_pos(c, layer, pos);
  if (rc) return rc;
  rc = run_layer(c, layer, pos, nullptr, hidden);
  return rc ? fail(c, rc, "decode_layer launch failed") : 0;
}

extern "C" int gq_hip_transformer_layer(gq_ctx *c, int layer, int pos, float *h_hidden, float *h_k,
                                        float *h_v, int head_stride) {
  if (!c || !h_hidden) return -1;
  int rc = check_layer_pos(c, layer, pos);
  if (rc) return rc;
  const int H = c->m.hidden;
  c->g_valid = false;
  HIPCHK(c, hipMemcpyAsync(c->ws.hidden, h_hidden, sizeof(float) * H, hipMemcpyHostToDevice, c->stream));
  if ((rc = run_layer(c, layer, pos, nullptr, c->ws.hidden))) return fail(c, rc, "layer launch failed");
  HIPCHK(c, hipMemcpyAsync(h_hidden, c->ws.hidden, sizeof(float) * H, hipMemcpyDeviceToHost, c->stream));
  if (h_k && h_v) { /* keep the host cache coherent for kv_cache_save */
    const size_t hd = c->kv_hd, row = sizeof(float) * hd;
    const size_t spitch = row * c->kv_max_seq, dpitch = sizeof(float) * head_stride;
    HIPCHK(c, hipMemcpy2DAsync(h_k + pos * hd, dpitch, gq_hip_kv_k(c, layer) + pos * hd, spitch, row,
                               c->kv_heads, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpy2DAsync(h_v + pos * hd, dpitch, gq_hip_kv_v(c, layer) + pos * hd, spitch, row,
                               c->kv_heads, hipMemcpyDeviceToHost, c->stream));
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

static int ensure_tokens(gq_ctx *c, int n);
static int ensure_graph(gq_ctx *c);

/* One decode step of a host-driven loop (the generate and chat loops call
 * forward_token / forward_sample once per token) as a replay of the
 * captured step graph.  The graph expects the token's embedding in w.hidden
 * and token, position and step on the device, and leaves the argmax
 * token's embedding and the next position there.  When the caller's
 * (token, pos) is what the previous replay left (a greedy loop), only the
 * step counter is reset; otherwise the token is embedded first. */
static int graph_step(gq_ctx *c, int token, int pos) {
  Workspace &w = c->ws;
  int rc;
  if ((rc = ensure_tokens(c, 1)) || (rc = ensure_graph(c))) return rc;
  if (!c->st_pinned && hipHostMalloc((void **)&c->st_pinned, 4 * sizeof(int)) != hipSuccess) {
    c->st_pinned = nullptr;
    return fail(c, -4, "pinned step state");
  }
  const bool same = c->g_valid && c->g_token == token && c->g_pos == pos;
  c->st_pinned[0] = token, c->st_pinned[1] = pos, c->st_pinned[2] = 0;
  HIPCHK(c, hipMemcpyAsync(w.d_token, c->st_pinned, 3 * sizeof(int), hipMemcpyHostToDevice, c->stream));
  if (!same && (rc = gq_launch_embed(c->m.embed.dtype, c->m.embed.data, c->m.hidden, w.d_token, token, w.hidden,
                                     c->stream)))
    return fail(c, rc, "embed launch failed");
  c->g_valid = false;
  HIPCHK(c, hipGraphLaunch(c->gexec, c->stream));
  return 0;
}

/* After graph_step: the argmax token to the host; the device state is then
 * (next, pos + 1). */
static int graph_step_token(gq_ctx *c, int pos, float *logits) {
  HIPCHK(c, hipMemcpyAsync(c->st_pinned + 3, c->ws.d_token, sizeof(int), hipMemcpyDeviceToHost, c->stream));
  if (logits)
    HIPCHK(c, hipMemcpyAsync(logits, c->ws.logits, sizeof(float) * c->m.vocab, hipMemcpyDeviceToHost,
                             c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  const int next = c->st_pinned[3];
  c->g_valid = true, c->g_token = next, c->g_pos = pos + 1;
  return next;
}

extern "C" int gq_hip_forward_token(gq_ctx *c, int token, int pos, float *logits, float *hidden_per_layer) {
  if (!c) return -1;
  int rc = check_pos(c, pos, 1);
  if (rc) return rc;
  if (token < 0 || token >= c->m.vocab) return fail(c, -1, "token %d out of range", token);
  if (!hidden_per_layer) { /* no per-layer copies: the captured step */
    if ((rc = graph_step(c, token, pos))) return rc;
    return graph_step_token(c, pos, logits);
  }
  if ((rc = run_step(c, token, pos, false, hidden_per_layer))) return fail(c, rc, "step launch failed");
  int next = -1;
  HIPCHK(c, hipMemcpyAsync(&next, c->ws.d_token, sizeof(int), hipMemcpyDeviceToHost, c->stream));
  if (logits)
    HIPCHK(c, hipMemcpyAsync(logits, c->ws.logits, sizeof(float) * c->m.vocab, hipMemcpyDeviceToHost,
                             c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return next;
}

static int ensure_tokens(gq_ctx *c, int n) {
  Workspace &w = c->ws;
  if (w.tokens_cap >= n) return 0;
  if (w.d_tokens) gq_hip_free(c, w.d_tokens);
  w.d_tokens = (int *)dev_alloc(c, sizeof(int) * n);
  if (!w.d_tokens) return -4;
  w.tokens_cap = n;
  free_graph(c); /* the graph captured the old pointer */
  return 0;
}

/* The decode step captured once into a HIP graph (run_step's device-state
 * form: token, position and step read on the device). */
static int ensure_graph(gq_ctx *c) {
  if (c->gexec) return 0;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  const int rc = run_step(c, 0, 0, true, nullptr);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(c->stream, &g);
  if (rc || e != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return fail(c, rc ? rc : -4, "graph capture failed");
  }
  c->graph = g;
  if (hipGraphInstantiate(&c->gexec, g, nullptr, nullptr, 0) != hipSuccess) {
    free_graph(c);
    return fail(c, -4, "graph instantiate failed");
  }
  return 0;
}

extern "C" int gq_hip_decode_loop(gq_ctx *c, int token, int pos, int n_steps, int use_graph,
                                  int32_t *tokens_out, float *ms) {
  if (!c || n_steps <= 0 || !tokens_out) return fail(c, -1, "decode_loop: bad argument");
  int rc = check_pos(c, pos, n_steps);
  if (rc) return rc;
  if (token < 0 || token >= c->m.vocab) return fail(c, -1, "token out of range");
  if ((rc = ensure_tokens(c, n_steps))) return rc;
  Workspace &w = c->ws;
  int st[3] = {token, pos, 0};
  HIPCHK(c, hipMemcpyAsync(w.d_token, st, sizeof st, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (use_graph && (rc = ensure_graph(c))) return rc;
  c->g_valid = false;
  EventPair ev;
  HIPCHK(c, ev.create());
  HIPCHK(c, hipEventRecord(ev.e0, c->stream));
  /* the first step's input; each step's argmax embeds the next token */
  if ((rc = gq_launch_embed(c->m.embed.dtype, c->m.embed.data, c->m.hidden, w.d_token, token, w.hidden, c->stream)))
    return fail(c, rc, "embed launch failed");
  for (int i = 0; i < n_steps; i++) {
    if (use_graph) {
      HIPCHK(c, hipGraphLaunch(c->gexec, c->stream));
    } else if ((rc = run_step(c, 0, 0, true, nullptr))) {
      return fail(c, rc, "step launch failed");
    }
  }
  HIPCHK(c, hipEventRecord(ev.e1, c->stream));
  HIPCHK(c, hipMemcpyAsync(tokens_out, w.d_tokens, sizeof(int32_t) * n_steps, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (ms) *ms = ev.ms();
  return 0;
}

/* ------------------------------------------------------------ prefill
 * forward(model, kv, scr, tokens, n, pos) for n > 1 (engine.c:559-595 with
 * transformer_layer's T-token path, engine.c:352-509): chunks of up to 512
 * tokens; per layer and chunk one GEMM launch per projection on the matrix
 * cores, RoPE + append of every token of the chunk, then causal attention
 * (token t sees positions 0 .. pos + t). */
template <class T>
static int pf_ensure(gq_ctx *c, T *&p, size_t &cap, size_t n) {
  if (cap >= n && p) return 0;
  if (p) gq_hip_free(c, p);
  p = (T *)dev_alloc(c, sizeof(T) * n);
  if (!p) return -4;
  cap = n;
  return 0;
}

/* Release the prefill activations (a model of another shape is bound, or
 * the cache was re-made). */
static void pf_release(gq_ctx *c) {
  PrefillWs &w = c->pf;
  void *bufs[8] = {w.x, w.q, w.k, w.v, w.xn, w.att, w.act, w.tok};
  for (void *p : bufs)
    if (p) gq_hip_free(c, p);
  w.x = w.q = w.k = w.v = nullptr;
  w.xn = w.att = w.act = nullptr;
  w.tok = nullptr;
  w.cap = w.H = w.F = w.kvd = 0;
}

static int pf_alloc(gq_ctx *c) {
  PrefillWs &w = c->pf;
  const gq_model &m = c->m;
  const int kvd_m = m.n_kv_heads * m.head_dim;
  if (w.cap && w.H == m.hidden && w.F == m.ff && w.kvd == kvd_m) return 0;
  pf_release(c);
  const size_t T = kPrefillChunk, H = m.hidden, F = m.ff, kvd = (size_t)kvd_m;
  float **f32[4] = {&w.x, &w.q, &w.k, &w.v};
  const size_t nf[4] = {T * H, T * H, T * kvd, T * kvd};
  for (int i = 0; i < 4; i++)
    if (!(*f32[i] = (float *)dev_alloc(c, sizeof(float) * nf[i]))) return -4;
  __bf16 **b16[3] = {&w.xn, &w.att, &w.act};
  const size_t nb[3] = {T * H, T * H, T * F};
  for (int i = 0; i < 3; i++)
    if (!(*b16[i] = (__bf16 *)dev_alloc(c, sizeof(__bf16) * nb[i]))) return -4;
  if (!(w.tok = (int *)dev_alloc(c, sizeof(int) * T))) return -4;
  w.cap = kPrefillChunk;
  w.H = m.hidden, w.F = m.ff, w.kvd = kvd_m;
  return 0;
}

/* The GEMM takes Q4_K and Q8_0 rows in multiples of 128 and Q6_K rows
 * likewise with cols % 512 == 0; a model with any other projection
 * prefills token by token through the decode step instead. */
static bool pf_gemm_ok(const gq_weight &w) {
  return (w.dtype == GQ_Q4_K || w.dtype == GQ_Q8_0 || (w.dtype == GQ_Q6_K && w.cols % 512 == 0)) &&
         w.rows % 128 == 0 && w.cols % 256 == 0;
}

static bool pf_model_ok(const gq_ctx *c) {
  if (c->prefill_mode != 0) return false;
  for (const gq_layer &L : c->layers)
    if (!pf_gemm_ok(L.wq) || !pf_gemm_ok(L.wk) || !pf_gemm_ok(L.wv) || !pf_gemm_ok(L.wo) || !pf_gemm_ok(L.w_gate) ||
        !pf_gemm_ok(L.w_up) || !pf_gemm_ok(L.w_down) || L.w_gate.dtype != L.w_up.dtype)
      return false;
  return true;
}

/* weight i (wq, wk, wv, wo, gate, up, down) of layer l as a GEMM segment:
 * its unit-layout copy where model bind made one */
static PgSeg pg_seg(const gq_ctx *c, int l, int i, const gq_weight &w, float *y) {
  const uint8_t *ux = (size_t)l < c->mm.size() && !gq_matvec_q6k_ref() ? c->mm[l].ux[i] : nullptr;
  return ux ? PgSeg{ux, y, w.rows, GQ_Q6_KX} : PgSeg{(const uint8_t *)w.data, y, w.rows, w.dtype};
}

/* RoPE + append of T tokens at pos..pos+T-1 (q: T x n_heads*hd in place,
 * k/v: T x n_kv*hd), then causal attention of the T tokens into out (fp32)
 * or out16 (bf16), T x n_heads*hd */
static int pf_attention(gq_ctx *c, int layer, int pos, int T, int n_heads, float *q, const float *k, const float *v,
                        float *out, __bf16 *out16, int kparts = 1) {
  const int hd = c->kv_hd, kvd = c->kv_heads * hd, qd = n_heads * hd;
  RopeArgs ra{q, k, v, gq_hip_kv_k(c, layer), gq_hip_kv_v(c, layer), c->rope, nullptr, pos,
              n_heads, c->kv_heads, hd, c->kv_max_seq, T, qd, kvd, kvd};
  if (kparts > 1) /* q, k, v are still the q/k/v GEMM's K parts */
    ra.parts = c->pf.part, ra.kparts = kparts, ra.prow = qd + 2 * kvd, ra.pstride = (size_t)T * (qd + 2 * kvd);
  int rc = gq_launch_rope_append(ra, c->stream);
  if (rc) return rc;
  AttnArgs aa{};
  aa.q = q, aa.q_stride = qd, aa.k = gq_hip_kv_k(c, layer), aa.v = gq_hip_kv_v(c, layer);
  aa.out = out, aa.out16 = out16, aa.out_stride = qd, aa.pos = pos, aa.ntok = T;
  aa.n_heads = n_heads, aa.n_kv = c->kv_heads, aa.hd = hd, aa.max_seq = c->kv_max_seq;
  aa.scale = 1.0f / sqrtf((float)hd);
  return gq_launch_flash_prefill(aa, c->stream);
}

/* one layer over the chunk (engine.c:352-554 with T tokens): 7 launches of
 * the GEMM (q/k/v together, gate/up together with SwiGLU), RMSNorms writing
 * bf16, RoPE + append + attention writing bf16 */
/* the K-part workspace for a launch of T x (its segments' rows) */
static void pf_parts(gq_ctx *c, PgArgs &a) {
  PrefillWs &w = c->pf;
  size_t rows = 0;
  for (int i = 0; i < a.nseg; i++) rows += a.seg[i].rows;
  const size_t n = (size_t)kPgKParts * a.T * rows;
  if (pf_ensure(c, w.part, w.part_cap, n) == 0) a.part = w.part, a.part_cap = w.part_cap;
}

/* pending: K parts of the previous layer's down launch still to be added
 * into the residual x (1: none); this layer's first RMSNorm adds them, and
 * this layer leaves its own down's parts the same way unless it is the
 * last */
static int pf_layer(gq_ctx *c, int l, int pos, int T, int &pending) {
  const gq_model &m = c->m;
  const gq_layer &L = c->layers[l];
  PrefillWs &w = c->pf;
  int rc;
  PgArgs qkv{}, o{}, gu{}, dn{};
  qkv.T = o.T = gu.T = dn.T = T;
  qkv.x = w.xn, qkv.K = m.hidden, qkv.nseg = 3;
  qkv.seg[0] = pg_seg(c, l, 0, L.wq, w.q), qkv.seg[1] = pg_seg(c, l, 1, L.wk, w.k);
  qkv.seg[2] = pg_seg(c, l, 2, L.wv, w.v);
  o.x = w.att, o.K = m.hidden, o.nseg = 1, o.seg[0] = pg_seg(c, l, 3, L.wo, w.x);
  gu.x = w.xn, gu.K = m.hidden, gu.nseg = 2, gu.act = w.act;
  gu.seg[0] = pg_seg(c, l, 4, L.w_gate, nullptr), gu.seg[1] = pg_seg(c, l, 5, L.w_up, nullptr);
  dn.x = w.act, dn.K = m.ff, dn.nseg = 1, dn.seg[0] = pg_seg(c, l, 6, L.w_down, w.x);
  pf_parts(c, qkv), pf_parts(c, o), pf_parts(c, dn);
  /* the q/k/v launch leaves its K parts' sum to the RoPE + append kernel,
   * o and down theirs to the next RMSNorm (the last layer's down sums its
   * own: the LM head reads x) */
  int kq = 1, ko = 1, kd = 1;
  qkv.kparts_out = &kq;
  o.kparts_out = &ko;
  if (l + 1 < m.n_layers) dn.kparts_out = &kd;
  auto norm = [&](const float *nw, int k) {
    return gq_launch_rmsnorm_rows(w.x, nw, nullptr, m.hidden, T, m.rms_eps, c->stream, w.xn,
                                  k > 1 ? w.part : nullptr, k, w.x);
  };
  if ((rc = norm(L.rms_att, pending)) || (rc = gq_launch_pgemm(MV_STORE, qkv, c->stream)) ||
      (rc = pf_attention(c, l, pos, T, m.n_heads, w.q, w.k, w.v, nullptr, w.att, kq)) ||
      (rc = gq_launch_pgemm(MV_RESID, o, c->stream)) || (rc = norm(L.rms_ffn, ko)) ||
      (rc = gq_launch_pgemm(MV_SWIGLU, gu, c->stream)) || (rc = gq_launch_pgemm(MV_RESID, dn, c->stream)))
    return rc;
  pending = kd;
  return 0;
}

extern "C" int gq_hip_prefill(gq_ctx *c, const int32_t *tokens, int n_tokens, int pos, float *logits,
                              float *hidden_last, float *ms) {
  if (!c || !tokens || n_tokens <= 0) return fail(c, -1, "prefill: bad argument");
  int rc = check_pos(c, pos, n_tokens);
  if (rc) return rc;
  const gq_model &m = c->m;
  for (int i = 0; i < n_tokens; i++)
    if (tokens[i] < 0 || tokens[i] >= m.vocab) return fail(c, -1, "prefill: token %d out of range", tokens[i]);
  const bool gemm = pf_model_ok(c);
  if (gemm && (rc = pf_alloc(c))) return rc;
  c->g_valid = false;
  PrefillWs &w = c->pf;
  Workspace &ws = c->ws;
  EventPair ev;
  if (ms) {
    HIPCHK(c, ev.create());
    HIPCHK(c, hipEventRecord(ev.e0, c->stream));
  }
  int T = 0;
  if (!gemm) { /* token by token through the decode step */
    for (int t = 0; t < n_tokens; t++)
      if ((rc = run_step(c, tokens[t], pos + t, false, nullptr))) return fail(c, rc, "prefill: step launch failed");
  } else {
    for (int t0 = 0; t0 < n_tokens; t0 += T) {
      T = std::min(kPrefillChunk, n_tokens - t0);
      HIPCHK(c, hipMemcpyAsync(w.tok, tokens + t0, sizeof(int) * T, hipMemcpyHostToDevice, c->stream));
      if ((rc = gq_launch_embed_rows(m.embed.dtype, m.embed.data, m.hidden, w.tok, T, w.x, c->stream)))
        return fail(c, rc, "prefill: embed");
      int pending = 1;
      for (int l = 0; l < m.n_layers; l++)
        if ((rc = pf_layer(c, l, pos + t0, T, pending))) return fail(c, rc, "prefill: layer %d launch failed", l);
    }
    /* last token: final RMSNorm + LM head + argmax as in a decode step */
    HIPCHK(c, hipMemcpyAsync(ws.hidden, w.x + (size_t)(T - 1) * m.hidden, sizeof(float) * m.hidden,
                             hipMemcpyDeviceToDevice, c->stream));
    if ((rc = op_lm_head(c, ws.hidden)) ||
        (rc = gq_launch_argmax(ws.logits, m.vocab, ws.amax, ws.amax_blocks, ws.d_token, nullptr, nullptr, nullptr,
                               c->stream)))
      return fail(c, rc, "prefill: lm head");
  }
  if (ms) HIPCHK(c, hipEventRecord(ev.e1, c->stream));
  int next = -1;
  HIPCHK(c, hipMemcpyAsync(&next, ws.d_token, sizeof(int), hipMemcpyDeviceToHost, c->stream));
  if (logits)
    HIPCHK(c, hipMemcpyAsync(logits, ws.logits, sizeof(float) * m.vocab, hipMemcpyDeviceToHost, c->stream));
  if (hidden_last)
    HIPCHK(c, hipMemcpyAsync(hidden_last, ws.hidden, sizeof(float) * m.hidden, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (ms) *ms = ev.ms();
  return next;
}

extern "C" int gq_hip_bound_layers(gq_ctx *c, int *whole) {
  if (!c) return -1;
  int n = 0;
  if (c->bound)
    for (char o : c->layer_on) n += o;
  if (whole) *whole = c->bound && c->whole;
  return n;
}

extern "C" int gq_hip_set_prefill_mode(gq_ctx *c, int mode) {
  if (!c || (mode != 0 && mode != 1)) return -1;
  const int prev = c->prefill_mode;
  c->prefill_mode = mode;
  return prev;
}

/* ------------------------------------------------------------ measurement */
extern "C" int gq_hip_profile_step(gq_ctx *c, int token, int pos, double ms[GQ_NCLASS],
                                   int launches[GQ_NCLASS], double bytes[GQ_NCLASS]) {
  if (!c) return -1;
  int rc = check_pos(c, pos, 1);
  if (rc) return rc;
  for (hipEvent_t e : c->ev) (void)hipEventDestroy(e);
  c->ev.clear(), c->ev_class.clear(), c->ev_bytes.clear();
  HIPCHK(c, hipStreamSynchronize(c->stream));
  c->prof = true;
  hipEvent_t e0 = next_event(c);
  (void)hipEventRecord(e0, c->stream);
  rc = run_step(c, token, pos, false, nullptr);
  c->prof = false;
  if (rc) return fail(c, rc, "profile step failed");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  for (int k = 0; k < GQ_NCLASS; k++) ms[k] = 0, launches[k] = 0, bytes[k] = 0;
  for (size_t i = 0; i < c->ev_class.size(); i++) {
    float t = 0.f;
    (void)hipEventElapsedTime(&t, c->ev[i], c->ev[i + 1]);
    const int k = c->ev_class[i];
    ms[k] += t;
    launches[k] += 1;
    bytes[k] += c->ev_bytes[i];
  }
  return 0;
}

extern "C" float gq_hip_time_op(gq_ctx *c, int op, int pos, int n_iter) {
  if (!c || n_iter <= 0 || op < 0 || op > PC_LM_HEAD) return -1.f;
  if (check_pos(c, pos, 1)) return -1.f;
  EventPair ev;
  if (ev.create() != hipSuccess) return -1.f;
  float *h = c->ws.hidden;
  c->g_valid = false;
  int rc = 0;
  (void)hipEventRecord(ev.e0, c->stream);
  for (int i = 0; i < n_iter && !rc; i++) {
    const int l = i % c->m.n_layers; /* every layer's weights: no cache reuse */
    switch (op) {
    case PC_QKV: rc = op_qkv(c, l, pos, nullptr, h); break;
    case PC_ATTN: rc = op_attention(c, l, pos, nullptr); break;
    case PC_O: rc = op_o(c, l, h); break;
    case PC_GATE_UP: rc = op_gate_up(c, l, h); break;
    case PC_DOWN: rc = op_down(c, l, h); break;
    default: rc = op_lm_head(c, h); break;
    }
  }
  (void)hipEventRecord(ev.e1, c->stream);
  (void)hipEventSynchronize(ev.e1);
  if (rc) return fail(c, rc, "time_op launch failed"), -1.f;
  return ev.ms() / n_iter;
}

extern "C" float gq_hip_time_matvec(gq_ctx *c, int dtype, const void *const *w_devs, int n_w, int rows,
                                    int cols, const float *x, float *y, int n_iter) {
  if (!c || !w_devs || n_w <= 0 || n_iter <= 0) return -1.f;
  if (check_mv(c, dtype, w_devs[0], rows, cols, 0, x, y)) return -1.f;
  /* tiled copies, made before the timed region, when the matrix-core
   * kernel is selected */
  std::vector<const uint8_t *> mm(n_w, nullptr);
  for (int i = 0; i < n_w; i++) mm[i] = op_tile(c, dtype, w_devs[i], rows, cols);
  EventPair ev;
  int rc = ev.create() == hipSuccess ? 0 : -4;
  if (!rc) (void)hipEventRecord(ev.e0, c->stream);
  for (int i = 0; i < n_iter && !rc; i++)
    rc = launch_one_mv(c, dtype, w_devs[i % n_w], rows, cols, x, y + (size_t)(i % n_w) * rows, mm[i % n_w]);
  float t = 0.f;
  if (!rc) {
    (void)hipEventRecord(ev.e1, c->stream);
    (void)hipEventSynchronize(ev.e1);
    t = ev.ms();
  }
  for (const uint8_t *p : mm)
    if (p) gq_hip_free(c, (void *)p);
  return rc ? -1.f : t / n_iter;
}

extern "C" float gq_hip_time_attention(gq_ctx *c, int layer, int pos, const float *q, float *out,
                                       int n_iter) {
  if (!c || !c->kslab || !q || !out || n_iter <= 0 || pos < 0 || pos >= c->kv_max_seq) return -1.f;
  const int n_heads = c->bound ? c->m.n_heads : -1;
  if (n_heads <= 0) return -1.f;
  EventPair ev;
  if (ev.create() != hipSuccess) return -1.f;
  AttnArgs aa{};
  aa.q = q, aa.part_o = c->ws.part_o, aa.part_ml = c->ws.part_ml, aa.out = out;
  aa.pos = pos, aa.n_heads = n_heads, aa.n_kv = c->kv_heads, aa.hd = c->kv_hd;
  aa.max_seq = c->kv_max_seq, aa.nch = c->ws.nch, aa.s_max = c->ws.s_max;
  aa.scale = 1.0f / sqrtf((float)c->kv_hd);
  (void)hipEventRecord(ev.e0, c->stream);
  for (int i = 0; i < n_iter; i++) {
    const int l = (layer + i) % c->kv_layers;
    aa.k = gq_hip_kv_k(c, l), aa.v = gq_hip_kv_v(c, l);
    if (gq_launch_attention(aa, c->stream, nullptr)) return -1.f;
  }
  (void)hipEventRecord(ev.e1, c->stream);
  (void)hipEventSynchronize(ev.e1);
  return ev.ms() / n_iter;
}

/* ------------------------------------------------------------ op-level */
extern "C" int gq_hip_qkv_rope_dev(gq_ctx *c, int layer, int pos, const float *hidden, float *q_out,
                                   int fused) {
  if (!c || !hidden || !q_out) return -1;
  int rc = check_layer_pos(c, layer, pos);
  if (rc) return rc;
  const gq_model &m = c->m;
  const gq_layer &L = c->layers[layer];
  Workspace &w = c->ws;
  const int H = m.hidden, kvd = m.n_kv_heads * m.head_dim;
  float *k = w.qkv + H, *v = w.qkv + H + kvd;
  const gq_weight *W[3] = {&L.wq, &L.wk, &L.wv};
  float *Y[3] = {q_out, fused ? gq_hip_kv_k(c, layer) : k, fused ? gq_hip_kv_v(c, layer) : v};
  const int kind[3] = {SEG_ROPE, SEG_ROPE_KV, SEG_KV};
  for (int i = 0; i < 3; i++) {
    MvArgs a{};
    a.cols = H, a.x = hidden, a.norm_w = L.rms_att, a.eps = m.rms_eps;
    a.rope = MvRope{c->rope, nullptr, pos, m.head_dim, c->kv_max_seq};
    a.seg[0] = MvSeg{(const uint8_t *)W[i]->data, Y[i], nullptr, W[i]->rows, fused ? kind[i] : SEG_PLAIN};
    a.nseg = 1;
    if ((rc = gq_launch_matvec(W[i]->dtype, MV_STORE, a, c->stream))) return fail(c, rc, "qkv launch");
  }
  if (!fused) {
    RopeArgs ra{q_out, k, v, gq_hip_kv_k(c, layer), gq_hip_kv_v(c, layer), c->rope, nullptr, pos,
                m.n_heads, m.n_kv_heads, m.head_dim, c->kv_max_seq};
    if ((rc = gq_launch_rope_append(ra, c->stream))) return fail(c, rc, "rope_append launch");
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return 0;
}

extern "C" int gq_hip_rmsnorm_dev(gq_ctx *c, const float *x, const float *w, float *out, int dim, float eps) {
  if (!c || !x || !out || dim <= 0) return -1;
  return gq_launch_rmsnorm(x, w, out, dim, eps, c->stream) ? fail(c, -4, "rmsnorm launch") : 0;
}

extern "C" int gq_hip_rope_append_dev(gq_ctx *c, int layer, int pos, int n_heads, float *q,
                                      const float *k, const float *v) {
  if (!c || !c->kslab || !q || !k || !v || layer < 0 || layer >= c->kv_layers) return fail(c, -1, "rope_append: bad argument");
  if (pos < 0 || pos >= c->kv_max_seq) return fail(c, -5, "rope_append: position outside the cache");
  RopeArgs ra{q, k, v, gq_hip_kv_k(c, layer), gq_hip_kv_v(c, layer), c->rope, nullptr, pos,
              n_heads, c->kv_heads, c->kv_hd, c->kv_max_seq};
  return gq_launch_rope_append(ra, c->stream) ? fail(c, -4, "rope_append launch") : 0;
}

static int attention_check(gq_ctx *c, int layer, int pos, int n_heads, const float *q, const float *out) {
  if (!c || !c->kslab || !q || !out || layer < 0 || layer >= c->kv_layers || n_heads <= 0 ||
      n_heads % c->kv_heads)
    return fail(c, -1, "attention: bad argument");
  if (pos < 0 || pos >= c->kv_max_seq) return fail(c, -5, "attention: position outside the cache");
  if (c->bound && n_heads != c->m.n_heads) return fail(c, -1, "attention: n_heads differs from the bound model");
  return 0;
}

static int attention_launch(gq_ctx *c, int layer, int pos, int n_heads, const float *q, float *out, float *part_o,
                            float *part_ml, int nch) {
  AttnArgs aa{};
  aa.q = q, aa.k = gq_hip_kv_k(c, layer), aa.v = gq_hip_kv_v(c, layer);
  aa.part_o = part_o, aa.part_ml = part_ml, aa.out = out, aa.pos = pos;
  aa.n_heads = n_heads, aa.n_kv = c->kv_heads, aa.hd = c->kv_hd, aa.max_seq = c->kv_max_seq;
  aa.nch = nch, aa.s_max = gq_attn_smax(c->kv_max_seq, nch), aa.scale = 1.0f / sqrtf((float)c->kv_hd);
  return gq_launch_attention(aa, c->stream, nullptr) ? fail(c, -1, "attention launch (unsupported head_dim/group?)") : 0;
}

extern "C" int gq_hip_attention_dev(gq_ctx *c, int layer, int pos, int n_heads, const float *q, float *out) {
  if (int rc = attention_check(c, layer, pos, n_heads, q, out)) return rc;
  Workspace &w = c->ws;
  const int nch = gq_attn_nch(c->kv_heads, c->kv_max_seq);
  const size_t need_o = (size_t)n_heads * nch * c->kv_hd, need_ml = (size_t)n_heads * nch * 2;
  if (!c->bound) { /* op-level use without a bound model: private partials */
    if (w.part_cap < need_o || w.part_ml_cap < need_ml || !w.part_o) {
      if (w.part_o) gq_hip_free(c, w.part_o);
      if (w.part_ml) gq_hip_free(c, w.part_ml);
      w.part_o = (float *)dev_alloc(c, sizeof(float) * need_o);
      w.part_ml = (float *)dev_alloc(c, sizeof(float) * need_ml);
      if (!w.part_o || !w.part_ml) return -4;
      w.part_cap = need_o;
      w.part_ml_cap = need_ml;
    }
    w.nch = nch;
    w.s_max = gq_attn_smax(c->kv_max_seq, nch);
  }
  return attention_launch(c, layer, pos, n_heads, q, out, w.part_o, w.part_ml, w.nch);
}

extern "C" int gq_hip_attention_dev_noalloc(gq_ctx *c, int layer, int pos, int n_heads, const float *q, float *out) {
  if (int rc = attention_check(c, layer, pos, n_heads, q, out)) return rc;
  if (!c->scratch) return fail(c, -4, "attention_noalloc: no scratch address on device %d", c->dev);
  const int nch = gq_attn_nch(c->kv_heads, c->kv_max_seq);
  const size_t need_o = (size_t)n_heads * nch * c->kv_hd, need_ml = (size_t)n_heads * nch * 2;
  const size_t off_ml = (need_o + 63) & ~(size_t)63; /* 256-byte aligned (m, l) pairs */
  if (off_ml + need_ml > kScratchFloats)
    return fail(c, -1, "attention_noalloc: %d heads x %d chunks x (head_dim %d + 2) floats exceed the %zu-float scratch",
                n_heads, nch, c->kv_hd, kScratchFloats);
  /* nothing in the partials needs to start at zero: the merge reads only
   * the chunks this launch writes */
  return attention_launch(c, layer, pos, n_heads, q, out, c->scratch, c->scratch + off_ml, nch);
}

extern "C" int gq_hip_prefill_attention_dev(gq_ctx *c, int layer, int pos, int T, int n_heads, float *q,
                                            const float *k, const float *v, float *out) {
  if (!c || !c->kslab || !q || !k || !v || !out || layer < 0 || layer >= c->kv_layers || T <= 0 ||
      n_heads <= 0 || n_heads % c->kv_heads)
    return fail(c, -1, "prefill attention: bad argument");
  if (pos < 0 || pos + T > c->kv_max_seq) return fail(c, -5, "prefill attention: positions outside the cache");
  const int rc = pf_attention(c, layer, pos, T, n_heads, q, k, v, out, nullptr);
  return rc ? fail(c, rc, "prefill attention launch (unsupported head_dim/group?)") : 0;
}

extern "C" int gq_hip_embed_dev(gq_ctx *c, int dtype, const void *table, int hidden, int token, float *out) {
  if (!c || !table || !out || hidden <= 0 || token < 0) return -1;
  return gq_launch_embed(dtype, table, hidden, nullptr, token, out, c->stream) ? fail(c, -1, "embed") : 0;
}

extern "C" int gq_hip_argmax_dev(gq_ctx *c, const float *x, int n, int *out_index_dev) {
  if (!c || !x || n <= 0 || !out_index_dev) return -1;
  const int nblk = gq_argmax_blocks(n);
  float *scratch = (float *)dev_alloc(c, sizeof(float) * 2 * nblk);
  if (!scratch) return -4;
  int rc = gq_launch_argmax(x, n, scratch, nblk, out_index_dev, nullptr, nullptr, nullptr, c->stream);
  (void)hipStreamSynchronize(c->stream);
  gq_hip_free(c, scratch);
  return rc ? fail(c, rc, "argmax") : 0;
}

/* ---- on-device sampling (tokenizer.c:175-333, generate.c:302-311) ---- */
static int sample_ensure(gq_ctx *c, int vocab, bool big) {
  SampleWs &w = c->sw;
  if (!c->d_sample && !(c->d_sample = (int *)dev_alloc(c, sizeof(int)))) return -4;
  if (!big || w.cap >= vocab) return 0;
  const size_t sort_bytes = gq_sample_ws_bytes(vocab);
  float *keys = (float *)dev_alloc(c, sizeof(float) * vocab);
  int *ids_in = (int *)dev_alloc(c, sizeof(int) * vocab), *ids = (int *)dev_alloc(c, sizeof(int) * vocab);
  void *tmp = dev_alloc(c, sort_bytes);
  if (!keys || !ids_in || !ids || !tmp) return -4;
  if (w.keys) gq_hip_free(c, w.keys), gq_hip_free(c, w.ids_in), gq_hip_free(c, w.ids), gq_hip_free(c, w.sort_tmp);
  w.keys = keys, w.ids_in = ids_in, w.ids = ids, w.sort_tmp = tmp, w.sort_bytes = sort_bytes, w.cap = vocab;
  return 0;
}

/* The next token from device logits as the reference's generate loop picks
 * it; greedy falls back to the argmax.  Returns the token or < 0. */
static int sample_on_device(gq_ctx *c, const float *logits, int vocab, float temperature, int top_k, float top_p,
                            int rnd) {
  /* top-p and plain temperature sampling use the vocabulary-sized buffers */
  const bool big = temperature > 0.0f && !(top_k > 0 && top_k < vocab) && top_p > 0.0f;
  int rc = sample_ensure(c, vocab, big);
  if (rc) return rc;
  rc = gq_launch_sample(logits, vocab, temperature, top_k, top_p, rnd, c->sw, c->d_sample, c->stream);
  if (rc == 1) { /* greedy */
    const int nblk = gq_argmax_blocks(vocab);
    float *scratch = c->ws.amax && c->ws.amax_blocks >= nblk ? c->ws.amax
                                                             : (float *)dev_alloc(c, sizeof(float) * 2 * nblk);
    if (!scratch) return -4;
    rc = gq_launch_argmax(logits, vocab, scratch, nblk, c->d_sample, nullptr, nullptr, nullptr, c->stream);
    if (scratch != c->ws.amax) {
      (void)hipStreamSynchronize(c->stream);
      gq_hip_free(c, scratch);
    }
  }
  if (rc == -2) return fail(c, -2, "top_k %d above the device limit %d", top_k, kMaxTopK);
  if (rc) return fail(c, rc, "sampling launch failed");
  int tok = -1;
  HIPCHK(c, hipMemcpyAsync(&tok, c->d_sample, sizeof(int), hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return tok;
}

extern "C" int gq_hip_sample_dev(gq_ctx *c, const float *logits, int vocab, float temperature, int top_k,
                                 float top_p, int rnd) {
  if (!c || !logits || vocab <= 0) return -1;
  return sample_on_device(c, logits, vocab, temperature, top_k, top_p, rnd);
}

extern "C" int gq_hip_forward_sample(gq_ctx *c, int token, int pos, float temperature, int top_k, float top_p,
                                     int rnd) {
  if (!c) return -1;
  int rc = check_pos(c, pos, 1);
  if (rc) return rc;
  if (token < 0 || token >= c->m.vocab) return fail(c, -1, "token %d out of range", token);
  if (temperature <= 0.0f) { /* greedy: the step's own argmax */
    if ((rc = graph_step(c, token, pos))) return rc;
    return graph_step_token(c, pos, nullptr);
  }
  if ((rc = graph_step(c, token, pos))) return rc;
  /* the sampled token generally differs from the argmax the replay embedded */
  const int next = sample_on_device(c, c->ws.logits, c->m.vocab, temperature, top_k, top_p, rnd);
  c->g_valid = false; /* the replay embedded its argmax, not the sampled token */
  return next;
}

/* One turn of the chat REPL (chat_repl, chat.c:157-263) on the device: the
 * caller's tokens (BOS first only when the conversation starts, as chat.c
 * tokenizes, :157-163) through the prefill at *current_pos, then the reply
 * sampled one token at a time (greedy when temperature <= 0, else the
 * device sampler with rnd[i] as the i-th rand() value) until max_tokens,
 * kChatMaxReply tokens or eos.  *current_pos advances by the prompt and by
 * the reply tokens as chat.c counts them: the last sampled token (eos
 * included) is counted but not fed, so its position stays unwritten. */
constexpr int kChatMaxReply = 512; /* CHAT_MAX_OUTPUT_TOKENS, chat.c:14 */

extern "C" int gq_hip_chat_turn(gq_ctx *c, const int32_t *tokens, int n_tokens, int *current_pos, int max_tokens,
                                int eos_token, float temperature, int top_k, float top_p, const int *rnd,
                                int32_t *reply) {
  if (!c || !c->whole || !tokens || n_tokens <= 0 || !current_pos || max_tokens <= 0 || !reply ||
      (temperature > 0.0f && !rnd))
    return fail(c, -1, "chat_turn: bad argument or no whole model on the device");
  const int p0 = *current_pos;
  if (p0 < 0 || p0 + n_tokens >= c->kv_max_seq - 1) /* chat.c:169 */
    return fail(c, -6, "chat_turn: %d tokens at %d do not fit the %d-position context", n_tokens, p0,
                c->kv_max_seq);
  int next = gq_hip_prefill(c, tokens, n_tokens, p0, nullptr, nullptr, nullptr);
  if (next < 0) return next;
  int used = 0;
  if (temperature > 0.0f && (next = sample_on_device(c, c->ws.logits, c->m.vocab, temperature, top_k, top_p,
                                                     rnd[used++])) < 0)
    return next;
  const int cur = p0 + n_tokens;
  int n = 0;
  reply[n++] = next;
  for (int i = 1; i < max_tokens && n < kChatMaxReply; i++) {
    const int pos = cur + i - 1;
    next = temperature > 0.0f ? gq_hip_forward_sample(c, next, pos, temperature, top_k, top_p, rnd[used++])
                              : gq_hip_forward_token(c, next, pos, nullptr, nullptr);
    if (next < 0) return next;
    reply[n++] = next;
    if (next == eos_token) break;
  }
  *current_pos = cur + n;
  return n;
}

/* Q6_K weights the prefill GEMM can read in the unit layout (cols % 2048):
 * a copy for the call, as a bound model keeps from gq_hip_model_bind;
 * matvec path 3 keeps the reference layout.  Freed by the caller. */
static const uint8_t *op_units(gq_ctx *c, int dtype, const void *w, int rows, int cols) {
  if (dtype != GQ_Q6_K || cols % 2048 || gq_matvec_q6k_ref()) return nullptr;
  uint8_t *d = (uint8_t *)dev_alloc(c, gq_q6k_units_bytes(rows, cols));
  if (d && gq_launch_q6k_units(d, w, rows, cols, c->stream)) {
    gq_hip_free(c, d);
    return nullptr;
  }
  return d;
}

static PgSeg op_seg(const uint8_t *ps, const void *w, float *y, int n, int dtype) {
  return ps ? PgSeg{ps, y, n, GQ_Q6_KX} : PgSeg{(const uint8_t *)w, y, n, dtype};
}

/* fp32 x -> the bf16 copy the GEMM reads */
static const __bf16 *pf_x16(gq_ctx *c, const float *x, size_t n) {
  PrefillWs &w = c->pf;
  if (pf_ensure(c, w.xb, w.xb_cap, n) || gq_launch_to_bf16(x, w.xb, n, c->stream)) return nullptr;
  return w.xb;
}

extern "C" int gq_hip_prefill_gemm_dev(gq_ctx *c, int dtype, int mode, const void *w, int n, int k,
                                       const float *x, int t, float *y, const float *r) {
  if (!c || !w || !x || !y || t <= 0 || n <= 0 || k <= 0 || (mode == 1 && !r) || (mode != 0 && mode != 1))
    return fail(c, -1, "prefill GEMM: bad argument");
  if (dtype != GQ_Q4_K && dtype != GQ_Q6_K && dtype != GQ_Q8_0)
    return fail(c, -1, "prefill GEMM: Q4_K, Q6_K or Q8_0 weights only");
  if (k % 256 || (dtype == GQ_Q6_K && k % 512)) return fail(c, -2, "prefill GEMM: cols %% 256 (Q6_K: %% 512)");
  if (n % 128) return fail(c, -1, "prefill GEMM: rows must be a multiple of 128");
  PgArgs a{};
  if (!(a.x = pf_x16(c, x, (size_t)t * k))) return fail(c, -4, "prefill GEMM: x conversion");
  const uint8_t *ps = op_units(c, dtype, w, n, k);
  a.T = t, a.K = k, a.nseg = 1, a.seg[0] = op_seg(ps, w, y, n, dtype);
  pf_parts(c, a);
  if (mode == 1 && r != y)
    HIPCHK(c, hipMemcpyAsync(y, r, sizeof(float) * (size_t)t * n, hipMemcpyDeviceToDevice, c->stream));
  const int rc = gq_launch_pgemm(mode == 1 ? MV_RESID : MV_STORE, a, c->stream);
  if (ps) gq_hip_free(c, (void *)ps);
  return rc ? fail(c, rc, "prefill GEMM launch") : 0;
}

extern "C" float gq_hip_time_prefill_gemm(gq_ctx *c, int dtype, const void *w, int n, int k, const float *x, int t,
                                         float *y, int n_iter) {
  if (!c || !w || !x || !y || t <= 0 || n <= 0 || k <= 0 || n_iter <= 0) return fail(c, -1, "time GEMM: bad argument"), -1.f;
  if (dtype != GQ_Q4_K && dtype != GQ_Q6_K && dtype != GQ_Q8_0)
    return fail(c, -1, "time GEMM: Q4_K, Q6_K or Q8_0 weights only"), -1.f;
  if (k % 256 || (dtype == GQ_Q6_K && k % 512) || n % 128) return fail(c, -2, "time GEMM: shape"), -1.f;
  PgArgs a{};
  if (!(a.x = pf_x16(c, x, (size_t)t * k))) return fail(c, -4, "time GEMM: x conversion"), -1.f;
  const uint8_t *ps = op_units(c, dtype, w, n, k);
  a.T = t, a.K = k, a.nseg = 1, a.seg[0] = op_seg(ps, w, y, n, dtype);
  pf_parts(c, a);
  EventPair ev;
  int rc = ev.create() == hipSuccess ? 0 : -4;
  if (!rc) rc = gq_launch_pgemm(MV_STORE, a, c->stream); /* untimed first launch */
  if (!rc) (void)hipEventRecord(ev.e0, c->stream);
  for (int i = 0; i < n_iter && !rc; i++) rc = gq_launch_pgemm(MV_STORE, a, c->stream);
  float ms = 0.f;
  if (!rc) {
    (void)hipEventRecord(ev.e1, c->stream);
    (void)hipEventSynchronize(ev.e1);
    ms = ev.ms();
  }
  if (ps) gq_hip_free(c, (void *)ps);
  if (rc) return fail(c, rc, "time GEMM launch"), -1.f;
  return ms / n_iter;
}

extern "C" int gq_hip_prefill_gate_up_dev(gq_ctx *c, int dtype, const void *w_gate, const void *w_up, int n, int k,
                                          const float *x, int t, uint16_t *act) {
  if (!c || !w_gate || !w_up || !x || !act || t <= 0 || n <= 0 || k <= 0)
    return fail(c, -1, "prefill gate/up: bad argument");
  if (dtype != GQ_Q4_K && dtype != GQ_Q6_K && dtype != GQ_Q8_0)
    return fail(c, -1, "prefill gate/up: Q4_K, Q6_K or Q8_0 weights only");
  if (k % 256 || (dtype == GQ_Q6_K && k % 512)) return fail(c, -2, "prefill gate/up: cols %% 256 (Q6_K: %% 512)");
  if (n % 64) return fail(c, -1, "prefill gate/up: rows must be a multiple of 64");
  PgArgs a{};
  if (!(a.x = pf_x16(c, x, (size_t)t * k))) return fail(c, -4, "prefill gate/up: x conversion");
  const uint8_t *pg = op_units(c, dtype, w_gate, n, k), *pu = pg ? op_units(c, dtype, w_up, n, k) : nullptr;
  if (pg && !pu) gq_hip_free(c, (void *)pg), pg = nullptr;
  a.T = t, a.K = k, a.nseg = 2, a.act = (__bf16 *)act;
  a.seg[0] = op_seg(pg, w_gate, nullptr, n, dtype);
  a.seg[1] = op_seg(pu, w_up, nullptr, n, dtype);
  const int rc = gq_launch_pgemm(MV_SWIGLU, a, c->stream);
  if (pg) gq_hip_free(c, (void *)pg), gq_hip_free(c, (void *)pu);
  return rc ? fail(c, rc, "prefill gate/up launch") : 0;
}

extern "C" float gq_hip_time_read(gq_ctx *c, const void *src, size_t bytes, size_t stride, int n_buf, int n_iter) {
  if (!c || !src || !bytes || n_buf <= 0 || n_iter <= 0 || (bytes & 15) || (stride & 15) ||
      (n_buf > 1 && stride < bytes))
    return fail(c, -1, "time read: bad argument"), -1.f;
  constexpr size_t kSink = 4096;
  uint32_t *sink = (uint32_t *)dev_alloc(c, sizeof(uint32_t) * kSink);
  if (!sink) return fail(c, -4, "time read: sink"), -1.f;
  const uint8_t *base = (const uint8_t *)src;
  EventPair ev;
  int rc = ev.create() == hipSuccess ? 0 : -4;
  if (!rc) rc = gq_launch_stream_read(base, bytes, sink, kSink, c->stream); /* untimed first launch */
  if (!rc) (void)hipEventRecord(ev.e0, c->stream);
  for (int i = 0; i < n_iter && !rc; i++)
    rc = gq_launch_stream_read(base + (size_t)((i + 1) % n_buf) * stride, bytes, sink, kSink, c->stream);
  float ms = 0.f;
  if (!rc) {
    (void)hipEventRecord(ev.e1, c->stream);
    (void)hipEventSynchronize(ev.e1);
    ms = ev.ms();
  }
  gq_hip_free(c, sink);
  if (rc) return fail(c, rc, "time read launch"), -1.f;
  return ms / n_iter;
}

extern "C" int gq_hip_copy_dev(gq_ctx *c, void *dst, const void *src, size_t bytes) {
  if (!c || !dst || !src) return -1;
  const int rc = gq_launch_copy(dst, src, bytes, c->n_cu, c->stream);
  return rc ? fail(c, rc, "copy: sizes and pointers must be multiples of 16 bytes") : 0;
}

extern "C" int gq_hip_silu_mul_dev(gq_ctx *c, float *gate, const float *up, int n) {
  if (!c || !gate || !up || n <= 0) return -1;
  return gq_launch_silu_mul(gate, up, n, c->stream) ? fail(c, -4, "silu_mul") : 0;
}
