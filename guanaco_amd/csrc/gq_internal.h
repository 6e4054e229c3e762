/*
 * gq_internal.h — launchers shared between the translation units of
 * libgq_hip.so (not part of the C ABI).
 */
#ifndef GQ_INTERNAL_H
#define GQ_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gq_hip.h"

/* ---- quantised matvec ----------------------------------------------------
 * One launch computes up to three row segments of the same dtype and shared
 * input x (e.g. the q and k projections), with optional fused prologue and
 * epilogue:
 *   prologue: x <- RMSNorm(x) * norm_w (when norm_w != NULL)
 *   MV_STORE:  y = W x
 *   MV_RESID:  y = r + W x            (r may alias y)
 *   MV_SWIGLU: seg[0] = gate, seg[1] = up (same rows);
 *              seg[0].y = silu(W_g x) * (W_u x)
 */
enum { MV_STORE = 0, MV_RESID = 1, MV_SWIGLU = 2 };

/* Per-segment output kind of MV_STORE launches (the fused q/k/v epilogue):
 *   SEG_PLAIN  y[r] = (W x)[r]
 *   SEG_ROPE   rows (2i, 2i+1) of each head rotated by the RoPE table row of
 *              pos, stored to y (the query)
 *   SEG_ROPE_KV rotated, stored into the K cache slab at pos
 *   SEG_KV     stored into the V cache slab at pos
 * Cache row r = h*head_dim + d lands at ((h*max_seq + pos)*head_dim + d). */
enum { SEG_PLAIN = 0, SEG_ROPE = 1, SEG_ROPE_KV = 2, SEG_KV = 3 };

/* Q6_K in the vector-ALU matvec's unit layout: an internal weight type,
 * never seen at the C ABI; the prefill GEMM reads it too (cols % 2048) */
#define GQ_Q6_KX 65

struct MvSeg {
  const uint8_t *w;
  float *y;
  const float *r;
  int rows;
  int kind;
};

struct MvRope {
  const float2 *cs; /* [max_seq][head_dim/2] (cos, sin) */
  const int *pos_dev;
  int pos;
  int head_dim, max_seq;
};

struct MvArgs {
  MvSeg seg[3];
  int nseg;
  int cols;
  const float *x;
  const float *norm_w;
  float eps;
  MvRope rope;
  /* the same weights tile-interleaved for the matrix-core kernel
   * (gq_launch_mm_tile), segments in order (MV_SWIGLU: gate and up in one
   * tensor); NULL: that kernel is not used */
  const uint8_t *mm;
  /* a Q6_K segment 0 in the vector-ALU kernel's unit layout
   * (gq_launch_q6k_units), used for one-segment store and residual launches
   * instead of seg[0].w; NULL: the reference layout */
  const uint8_t *dx;
};

/* silu(g) * u as the reference computes it: silu(g) = g * (1 / (1 + expf(-g)))
 * (kernels_cpu.c:322-336), then the product (elemwise_mul, :367-389) */
__device__ __forceinline__ float gq_silu_mul(float g, float u) {
  const float sig = 1.0f / (1.0f + expf(0.0f - g));
  return (g * sig) * u;
}

/* The segments of a launch as plain values, read from the kernel
 * arguments once with constant indices and pinned in scalar registers: a
 * runtime index into the argument struct (or a select between its fields,
 * which the compiler may turn into a load through a selected address)
 * compiles to a copy of the struct in scratch memory or a global load with a
 * full vmcnt(0) wait. */
struct MvSegs {
  const uint8_t *w0, *w1, *w2;
  float *y0, *y1, *y2;
  const float *r0, *r1, *r2;
  int n0, n1, n2;
  int k0, k1, k2;
  int nseg;
};

template <class T>
__device__ __forceinline__ T gq_pin(T v) {
  asm volatile("" : "+s"(v));
  return v;
}

__device__ __forceinline__ MvSegs gq_mv_segs(const MvArgs &a) {
  MvSegs s;
  s.w0 = gq_pin(a.seg[0].w), s.w1 = gq_pin(a.seg[1].w), s.w2 = gq_pin(a.seg[2].w);
  s.y0 = gq_pin(a.seg[0].y), s.y1 = gq_pin(a.seg[1].y), s.y2 = gq_pin(a.seg[2].y);
  s.r0 = gq_pin(a.seg[0].r), s.r1 = gq_pin(a.seg[1].r), s.r2 = gq_pin(a.seg[2].r);
  s.n0 = gq_pin(a.seg[0].rows), s.n1 = gq_pin(a.seg[1].rows), s.n2 = gq_pin(a.seg[2].rows);
  s.k0 = gq_pin(a.seg[0].kind), s.k1 = gq_pin(a.seg[1].kind), s.k2 = gq_pin(a.seg[2].kind);
  s.nseg = gq_pin(a.nseg);
  return s;
}

/* segment and local row of output row gr of a launch */
__device__ __forceinline__ void gq_mv_locate(const MvSegs &v, int gr, int &s, int &lr) {
  s = 0;
  lr = gr;
  if (v.nseg > 1 && lr >= v.n0) {
    lr -= v.n0, s = 1;
    if (v.nseg > 2 && lr >= v.n1) lr -= v.n1, s = 2;
  }
}
/* A field of segment s.  The three values are pinned in registers before
 * the select: a select between fields of the struct would otherwise be
 * folded into a load at a computed offset, which keeps the struct in
 * scratch memory for the whole launch. */
template <class T>
__device__ __forceinline__ T gq_mv_sel(T a, T b, T c, int s) {
  a = gq_pin(a), b = gq_pin(b), c = gq_pin(c);
  return s == 0 ? a : s == 1 ? b : c;
}
__device__ __forceinline__ const uint8_t *gq_mv_w(const MvSegs &v, int s) { return gq_mv_sel(v.w0, v.w1, v.w2, s); }
__device__ __forceinline__ float *gq_mv_y(const MvSegs &v, int s) { return gq_mv_sel(v.y0, v.y1, v.y2, s); }
__device__ __forceinline__ const float *gq_mv_r(const MvSegs &v, int s) { return gq_mv_sel(v.r0, v.r1, v.r2, s); }
__device__ __forceinline__ int gq_mv_rows(const MvSegs &v, int s) { return gq_mv_sel(v.n0, v.n1, v.n2, s); }
__device__ __forceinline__ int gq_mv_kind(const MvSegs &v, int s) { return gq_mv_sel(v.k0, v.k1, v.k2, s); }

/* Any dtype and shape the reference's matvec takes (cols % 256, Q8_0
 * cols % 32): the matrix-core kernel where the path setting picks it and
 * a.mm is set, else the vector-ALU kernel (gq_mvx.hip).  0, -1 bad
 * arguments, -2 cols, -4 launch error. */
int gq_launch_matvec(int dtype, int mode, const MvArgs &a, hipStream_t s);
/* The matrix-core kernel alone (a.mm required); 1 when the shape does not
 * fit it. */
int gq_launch_mm(int dtype, int mode, const MvArgs &a, hipStream_t s);
/* Two MV_STORE matvecs of different dtypes (Q4_K, then Q6_K) over the same
 * x in one launch; 1 when the pair is not supported (launch them apart). */
int gq_launch_matvec_pair(int dt0, const MvArgs &a0, int dt1, const MvArgs &a1, hipStream_t s);
/* compute units of the device (sizes the matrix-core kernel's grid) */
void gq_matvec_set_cus(int n_cu);

/* Tile-interleaved copy of a Q4_K or Q6_K weight for the matrix-core matvec.
 * For each 16-row tile T and block b, the 16 rows' block bytes are stored
 * together (16 * block bytes), as 16-byte units ordered (chunk, row): byte o
 * of row n's block at (o / 16) * 256 + 16 n + o % 16, and Q6_K's last two
 * bytes (d) at 13 * 256 + 2 n.  Tile T covers rows 16T .. 16T+15 of w0 (rows
 * past `rows` zero), or with w1 (MV_SWIGLU) rows 8T .. 8T+7 of w0 then the
 * same rows of w1.  Bytes: gq_mm_tile_bytes. */
size_t gq_mm_tile_bytes(int dtype, int rows, int cols, bool swiglu);
int gq_launch_mm_tile(void *dst, int dtype, const void *w0, const void *w1, int rows, int cols, hipStream_t s);
/* Q6_K weights (rows x cols, cols a multiple of 512) re-laid out for the
 * vector-ALU matvec and the prefill GEMM: each 32-column unit's quants, high
 * bits, scales and d at naturally aligned offsets, the same bytes
 * (gq_q6k_units_bytes). */
size_t gq_q6k_units_bytes(int rows, int cols);
int gq_launch_q6k_units(void *dst, const void *src, int rows, int cols, hipStream_t s);
/* whether the matrix-core kernel is selected for every launch it fits
 * (gq_hip_set_matvec_path(2)): the op-level entry points then tile their
 * weights per call */
bool gq_matvec_mm_forced();
/* matvec path 3: every Q6_K launch on the reference layout (no re-laid copies) */
bool gq_matvec_q6k_ref();

/* ---- attention -------------------------------------------------------- */
struct AttnArgs {
  const float *q;   /* n_heads x hd (already rotated) */
  const float *k;   /* layer K slab [n_kv][max_seq][hd] */
  const float *v;
  float *part_o;    /* [n_heads][nch][hd] */
  float *part_ml;   /* [n_heads][nch][2] */
  float *out;       /* n_heads x hd */
  const int *pos_dev; /* position read on the device when not NULL */
  int pos;
  int n_heads, n_kv, hd, max_seq, nch, s_max;
  float scale;
  /* the prefill form (gq_launch_flash_prefill): ntok query tokens at
   * positions pos .. pos + ntok - 1, token t attending to 0 .. pos + t;
   * per-token strides in elements; out16 != NULL writes bf16 there instead
   * of fp32 to out.  Decode launches leave these zero. */
  int ntok, q_stride, out_stride;
  __bf16 *out16;
};
int gq_attn_nch(int n_kv, int max_seq);
int gq_attn_smax(int max_seq, int nch);
int gq_launch_attention(const AttnArgs &a, hipStream_t s, hipEvent_t mid);
/* Causal attention of a prefill chunk (a.ntok tokens at a.pos, their keys
 * already appended) by the fp32-MFMA flash kernel: q, q_stride, k, v, out
 * or out16, out_stride, pos, ntok, n_heads, n_kv, hd (64 or 128), max_seq
 * and scale are used. */
int gq_launch_flash_prefill(const AttnArgs &a, hipStream_t s);

struct RopeArgs {
  float *q;
  const float *k, *v;
  float *kc, *vc;      /* layer slabs */
  const float2 *cs;    /* rope table [max_seq][hd/2] (cos, sin) */
  const int *pos_dev;
  int pos;
  int n_heads, n_kv, hd, max_seq;
  /* ntok tokens at pos .. pos + ntok - 1 (0 or 1: one); per-token strides in
   * floats of q, k, v */
  int ntok, q_stride, k_stride, v_stride;
  /* parts != NULL: q, k and v of token t are the sums of a K-split GEMM's
   * kparts parts (PgArgs.kparts_out), q | k | v of token t at parts +
   * t * prow, part p at + p * pstride; the rotated q still goes to q */
  const float *parts;
  int kparts, prow;
  size_t pstride;
};
int gq_launch_rope_append(const RopeArgs &a, hipStream_t s);

/* ---- misc -------------------------------------------------------------- */
int gq_launch_rmsnorm(const float *x, const float *w, float *out, int dim, float eps,
                      hipStream_t s);
int gq_launch_embed(int dtype, const void *table, int hidden, const int *token_dev, int token,
                    float *out, hipStream_t s);
/* argmax of x[n] (ties -> lowest index) -> *out_index; when step_dev != NULL
 * also stores the index at tokens[*step_dev], then ++*step_dev and
 * ++*pos_dev (the decode-loop bookkeeping of one graph replay). */
/* emb_out != NULL: the winner's embedding row (emb_dtype, emb_table,
 * hidden) is also written to emb_out, by the same launch */
int gq_launch_argmax(const float *x, int n, float *scratch, int nblk, int *out_index,
                     int *tokens, int *step_dev, int *pos_dev, hipStream_t s, int emb_dtype = 0,
                     const void *emb_table = nullptr, int hidden = 0, float *emb_out = nullptr);
int gq_argmax_blocks(int n);

/* On-device sampling (gq_sample.hip).  top-k handles k <= kMaxTopK. */
constexpr int kMaxTopK = 1024;
struct SampleWs {
  float *keys = nullptr;           /* sorted logits (top-p) or probabilities (temperature) */
  int *ids_in = nullptr, *ids = nullptr;
  void *sort_tmp = nullptr;        /* radix-sort temporary storage */
  size_t sort_bytes = 0;
  int cap = 0;                     /* vocabulary the buffers hold */
};
/* radix-sort temporary bytes for a vocabulary */
size_t gq_sample_ws_bytes(int vocab);
/* The reference's sampler choice (generate.c:302-311) for rnd = its rand()
 * draw: 0 launched (token -> *out on the device), 1 greedy (use the argmax),
 * -1 bad argument or workspace, -2 top_k above kMaxTopK, -4 launch error. */
int gq_launch_sample(const float *logits, int vocab, float temperature, int top_k, float top_p, int rnd,
                     const SampleWs &ws, int *out, hipStream_t s);
int gq_launch_silu_mul(float *gate, const float *up, int n, hipStream_t s);
int gq_launch_copy(void *dst, const void *src, size_t bytes, int n_cu, hipStream_t s);
/* Read bytes (a multiple of 16, 16-byte aligned) from src and store nothing:
 * at most sink_n workgroups of eight 16-byte loads per thread per pass
 * (sink: sink_n words the kernel only writes in a case that does not occur
 * in practice). */
int gq_launch_stream_read(const void *src, size_t bytes, uint32_t *sink, size_t sink_n, hipStream_t s);

/* ---- prefill chunk ---------------------------------------------------
 * Y[T][rows] = X[T][K] . W^T on the bf16 matrix cores for up to three weight
 * segments in one launch (each rows % 128 == 0, Q4_K, Q8_0, Q6_K with
 * K % 512 == 0, or Q6_K in the unit layout, GQ_Q6_KX, with K % 2048 == 0;
 * K % 256 == 0), X bf16 row-major.  MV_STORE writes y, MV_RESID adds into
 * y; MV_SWIGLU takes gate (seg 0) and up (seg 1) of equal rows
 * (rows % 64 == 0) and writes act[T][rows] = bf16(silu(gate) * up). */
struct PgSeg {
  const uint8_t *w;
  float *y;
  int rows, dtype;
};
struct PgArgs {
  const __bf16 *x;
  __bf16 *act;
  PgSeg seg[3];
  int nseg, T, K;
  /* optional workspace of part_cap floats: a STORE or RESID launch whose
   * grid is too small for 128-token tiles then splits K over workgroups,
   * each part writing its sums there (T x all segments' rows per part), and
   * a second kernel adds the parts (and the residual) in a fixed order and
   * scatters them to the segments' outputs */
  float *part;
  size_t part_cap;
  int kparts, rows_total; /* set by the launcher */
  /* a launch with kparts_out set leaves the parts' sum (and for RESID the
   * residual add) to its caller when it splits, writing the number of parts
   * there (1: not split, y is final) */
  int *kparts_out;
};
int gq_launch_pgemm(int mode, const PgArgs &a, hipStream_t s);
/* at most this many K parts in a split launch: PgArgs.part needs
 * kPgKParts * T * (all segments' rows) floats */
constexpr int kPgKParts = 4;
int gq_launch_to_bf16(const float *x, __bf16 *y, size_t n, hipStream_t s);
/* RMSNorm of `rows` consecutive rows of dim floats, one workgroup per row;
 * out16 != NULL writes bf16 there instead of fp32 to out.  parts != NULL
 * (kparts of rows x dim each, a K-split GEMM's sums left to this launch by
 * PgArgs.kparts_out): each row is first x plus the sum of its parts, which
 * is also stored to xnew (may be x). */
int gq_launch_rmsnorm_rows(const float *x, const float *w, float *out, int dim, int rows, float eps,
                           hipStream_t s, __bf16 *out16 = nullptr, const float *parts = nullptr, int kparts = 0,
                           float *xnew = nullptr);
/* embedding rows of tokens[0..n) (device array) into out (n x hidden) */
int gq_launch_embed_rows(int dtype, const void *table, int hidden, const int *tokens_dev, int n, float *out,
                         hipStream_t s);
int gq_launch_synth_quant(void *dev, int dtype, int rows, int cols, uint64_t seed, hipStream_t s);
int gq_launch_synth_normal(float *dev, size_t n, uint64_t seed, int norm_weight, hipStream_t s);
int gq_launch_synth_kv(float *slab, int n_layers, int n_kv, int hd, int max_seq, int n_pos,
                       uint64_t seed, hipStream_t s);

#endif
