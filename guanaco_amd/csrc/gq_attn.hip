/*
 * gq_attn.hip — fused RoPE + KV append and split-K single-query GQA
 * attention over the device KV cache (gfx950).
 *
 * KV layout is the reference's: [layer][kv_head][max_seq][head_dim] fp32, K
 * and V in separate slabs (kv_cache.c:25-32, :90-93).
 *
 * rope_append: one workgroup rotates every Q head and the new K row with the
 * (cos, sin) table row of `pos` (precomputed on the host with the reference's
 * fp32 expressions, kernels_cpu.c:409-413; rotation products and differences
 * rounded separately, :415-429) and writes K and V at pos % max_seq
 * (kv_cache.c:101-125).  Appended rows are bit copies of the reference's.
 *
 * attention: flash-decoding split over the sequence.  Workgroup (g, c)
 * streams chunk c of KV head g once for all G = n_heads/n_kv query heads
 * that share it (the reference re-reads K/V per Q head, engine.c:458-509):
 *   phase 1  scores s[h][j] = (q_h . K_j) * 1/sqrt(hd); 16 lanes per
 *            position (hd 128), 8 dims per lane, DPP row reduction;
 *   phase 2  per head chunk max m, p = expf(s - m), l = sum p;
 *   phase 3  o[h][:] = sum_j p[h][j] V_j, V read as coalesced 512-byte rows.
 * A merge kernel combines the chunks: M = max m_c, out = sum o_c e^(m_c-M) /
 * sum l_c e^(m_c-M).  The position count is read on the device, so the same
 * launch serves every step of a captured decode graph.
 */
#include "gq_device.h"
#include "gq_internal.h"

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void rope_append_kernel(RopeArgs a) {
#pragma clang fp contract(off)
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  /* the host rejects positions outside the cache; this keeps a stray
   * device-side position from indexing past the table or the slab */
  if (pos < 0 || pos >= a.max_seq) return;
  const int half = a.hd >> 1;
  const int p = pos;
  const float2 *cs = a.cs + (size_t)pos * half;
  const int nq = a.n_heads * half, nk = a.n_kv * half;
  for (int t = threadIdx.x; t < nq + nk; t += kThreads) {
    const bool isq = t < nq;
    const int u = isq ? t : t - nq;
    const int h = u / half, i = u - h * half;
    const float2 c = cs[i];
    const float *src = isq ? a.q + (size_t)h * a.hd : a.k + (size_t)h * a.hd;
    const float x0 = src[2 * i], x1 = src[2 * i + 1];
    const float y0 = x0 * c.x - x1 * c.y;
    const float y1 = x0 * c.y + x1 * c.x;
    if (isq) {
      a.q[(size_t)h * a.hd + 2 * i] = y0;
      a.q[(size_t)h * a.hd + 2 * i + 1] = y1;
    } else {
      float *dst = a.kc + ((size_t)h * a.max_seq + p) * a.hd;
      dst[2 * i] = y0;
      dst[2 * i + 1] = y1;
    }
  }
  for (int t = threadIdx.x; t < a.n_kv * a.hd; t += kThreads) {
    const int h = t / a.hd, d = t - h * a.hd;
    a.vc[((size_t)h * a.max_seq + p) * a.hd + d] = a.v[t];
  }
}

/* Chunk c of [0, L): length S = ceil(L/nch) rounded up to 16. */
__device__ __forceinline__ void chunk_range(int L, int nch, int c, int &c0, int &c1) {
  int S = (L + nch - 1) / nch;
  S = (S + 15) & ~15;
  c0 = c * S;
  c1 = min(L, c0 + S);
}

template <int HD, int G>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(AttnArgs a) {
  constexpr int LPP = HD / 8;         /* lanes per position in phase 1 */
  constexpr int PPW = GQ_WAVE / LPP;  /* positions per wave step */
  constexpr int DG = HD / 4;          /* float4 dim groups in phase 3 */
  constexpr int NPG = kThreads / DG;  /* position groups in phase 3 */
  extern __shared__ float sm[];
  float *sq = sm;                     /* [G][HD] */
  float *ss = sq + G * HD;            /* [G][s_max] scores / probabilities */
  float *sr = ss + G * a.s_max;       /* [NPG][G][HD] phase-3 partials */

  const int g = blockIdx.x, c = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  const int L = min(pos + 1, a.max_seq);
  int c0, c1;
  chunk_range(L, a.nch, c, c0, c1);
  const int h0 = g * G;
  const size_t obase = ((size_t)h0 * a.nch + c);

  if (c0 >= c1) { /* empty chunk: neutral element of the merge */
    for (int t = tid; t < G * HD; t += kThreads) {
      const int h = t / HD, d = t - h * HD;
      a.part_o[(obase + (size_t)h * a.nch) * HD + d] = 0.f;
    }
    if (tid < G) {
      a.part_ml[(obase + (size_t)tid * a.nch) * 2] = -INFINITY;
      a.part_ml[(obase + (size_t)tid * a.nch) * 2 + 1] = 0.f;
    }
    return;
  }

  for (int t = tid; t < G * HD; t += kThreads) sq[t] = a.q[(size_t)h0 * HD + t];
  __syncthreads();

  const float *K = a.k + (size_t)g * a.max_seq * HD;
  const float *V = a.v + (size_t)g * a.max_seq * HD;

  /* ---- phase 1: scores ---- */
  {
    const int sub = lane % LPP, pw = lane / LPP;
    const int d0 = 4 * sub, d1 = HD / 2 + 4 * sub;
    float q0[G][4], q1[G][4];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
      for (int e = 0; e < 4; e++) q0[h][e] = sq[h * HD + d0 + e], q1[h][e] = sq[h * HD + d1 + e];
    for (int j0 = c0 + wave * PPW; j0 < c1; j0 += 4 * PPW) {
      const int j = j0 + pw;
      const bool ok = j < c1;
      const float *kr = K + (size_t)(ok ? j : c0) * HD;
      const float4 ka = *(const float4 *)(kr + d0), kb = *(const float4 *)(kr + d1);
#pragma unroll
      for (int h = 0; h < G; h++) {
        float s = q0[h][0] * ka.x;
        s = __builtin_fmaf(q0[h][1], ka.y, s);
        s = __builtin_fmaf(q0[h][2], ka.z, s);
        s = __builtin_fmaf(q0[h][3], ka.w, s);
        s = __builtin_fmaf(q1[h][0], kb.x, s);
        s = __builtin_fmaf(q1[h][1], kb.y, s);
        s = __builtin_fmaf(q1[h][2], kb.z, s);
        s = __builtin_fmaf(q1[h][3], kb.w, s);
        s = LPP == 16 ? gq_row16_sum(s) : gq_row8_sum(s);
        if (ok && sub == 0) ss[h * a.s_max + (j - c0)] = s * a.scale;
      }
    }
  }
  __syncthreads();

  /* ---- phase 2: chunk softmax statistics per head ---- */
  const int n = c1 - c0;
  for (int h = wave; h < G; h += kThreads / GQ_WAVE) {
    float *row = ss + h * a.s_max;
    float m = -INFINITY;
    for (int j = lane; j < n; j += GQ_WAVE) m = fmaxf(m, row[j]);
    m = gq_wave_max(m);
    float l = 0.f;
    for (int j = lane; j < n; j += GQ_WAVE) {
      const float e = expf(row[j] - m);
      row[j] = e;
      l += e;
    }
    l = gq_wave_sum(l);
    if (lane == 0) {
      a.part_ml[(obase + (size_t)h * a.nch) * 2] = m;
      a.part_ml[(obase + (size_t)h * a.nch) * 2 + 1] = l;
    }
  }
  __syncthreads();

  /* ---- phase 3: o = P V over the chunk ---- */
  {
    const int dg = tid % DG, pg = tid / DG;
    float acc[G][4];
#pragma unroll
    for (int h = 0; h < G; h++) acc[h][0] = acc[h][1] = acc[h][2] = acc[h][3] = 0.f;
    for (int j = c0 + pg; j < c1; j += NPG) {
      const float4 v = *(const float4 *)(V + (size_t)j * HD + 4 * dg);
#pragma unroll
      for (int h = 0; h < G; h++) {
        const float p = ss[h * a.s_max + (j - c0)];
        acc[h][0] = __builtin_fmaf(p, v.x, acc[h][0]);
        acc[h][1] = __builtin_fmaf(p, v.y, acc[h][1]);
        acc[h][2] = __builtin_fmaf(p, v.z, acc[h][2]);
        acc[h][3] = __builtin_fmaf(p, v.w, acc[h][3]);
      }
    }
#pragma unroll
    for (int h = 0; h < G; h++)
      *(float4 *)(sr + ((size_t)pg * G + h) * HD + 4 * dg) =
          make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
  }
  __syncthreads();
  for (int t = tid; t < G * HD; t += kThreads) {
    float o = 0.f;
#pragma unroll 4
    for (int pg = 0; pg < NPG; pg++) o += sr[(size_t)pg * G * HD + t];
    const int h = t / HD, d = t - h * HD;
    a.part_o[(obase + (size_t)h * a.nch) * HD + d] = o;
  }
}

__global__ void attn_merge_kernel(AttnArgs a) {
  const int h = blockIdx.x, d = threadIdx.x;
  const float *ml = a.part_ml + (size_t)h * a.nch * 2;
  float M = -INFINITY;
  for (int c = 0; c < a.nch; c++) M = fmaxf(M, ml[2 * c]);
  float o = 0.f, l = 0.f;
  for (int c = 0; c < a.nch; c++) {
    const float m = ml[2 * c];
    if (m == -INFINITY) continue;
    const float w = expf(m - M);
    l = __builtin_fmaf(ml[2 * c + 1], w, l);
    o = __builtin_fmaf(a.part_o[((size_t)h * a.nch + c) * a.hd + d], w, o);
  }
  a.out[(size_t)h * a.hd + d] = o / l;
}

template <int HD, int G>
int launch_partial(const AttnArgs &a, hipStream_t s) {
  constexpr int NPG = kThreads / (HD / 4);
  const size_t lds = sizeof(float) * ((size_t)G * HD + (size_t)G * a.s_max + (size_t)NPG * G * HD);
  if (lds > 65536) return -1;
  hipLaunchKernelGGL((attn_partial_kernel<HD, G>), dim3(a.n_kv, a.nch), dim3(kThreads), lds, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

} // namespace

int gq_attn_nch(int n_kv, int max_seq) {
  /* about 512 workgroups (2 per CU) for long contexts, at least 64
   * positions per chunk */
  int nch = (512 + n_kv - 1) / n_kv;
  const int by_len = (max_seq + 63) / 64;
  if (nch > by_len) nch = by_len;
  return nch < 1 ? 1 : nch;
}

int gq_attn_smax(int max_seq, int nch) {
  int S = (max_seq + nch - 1) / nch;
  return (S + 15) & ~15;
}

int gq_launch_attention(const AttnArgs &a, hipStream_t s, hipEvent_t mid) {
  if (a.n_kv <= 0 || a.n_heads % a.n_kv) return -1;
  const int G = a.n_heads / a.n_kv;
  int rc = -1;
  if (a.hd == 128 && G == 4) rc = launch_partial<128, 4>(a, s);
  else if (a.hd == 128 && G == 8) rc = launch_partial<128, 8>(a, s);
  else if (a.hd == 128 && G == 1) rc = launch_partial<128, 1>(a, s);
  else if (a.hd == 64 && G == 4) rc = launch_partial<64, 4>(a, s);
  else if (a.hd == 64 && G == 8) rc = launch_partial<64, 8>(a, s);
  else if (a.hd == 64 && G == 1) rc = launch_partial<64, 1>(a, s);
  if (rc) return rc;
  if (mid) (void)hipEventRecord(mid, s);
  hipLaunchKernelGGL(attn_merge_kernel, dim3(a.n_heads), dim3(a.hd), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_rope_append(const RopeArgs &a, hipStream_t s) {
  if ((a.hd & 1) || a.n_kv <= 0) return -1;
  hipLaunchKernelGGL(rope_append_kernel, dim3(1), dim3(kThreads), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
