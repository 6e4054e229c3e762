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
#include <algorithm>

#include "gq_device.h"
#include "gq_internal.h"

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void rope_append_kernel(RopeArgs a) {
#pragma clang fp contract(off)
  /* token blockIdx.x of a chunk (0 for one token) */
  const int tz = blockIdx.x;
  const int pos = (a.pos_dev ? *a.pos_dev : a.pos) + tz;
  /* the host rejects positions outside the cache; this keeps a stray
   * device-side position from indexing past the table or the slab */
  if (pos < 0 || pos >= a.max_seq) return;
  const int half = a.hd >> 1;
  const int p = pos;
  const float2 *cs = a.cs + (size_t)pos * half;
  float *q = a.q + (size_t)tz * a.q_stride;
  const float *kin = a.k + (size_t)tz * a.k_stride, *vin = a.v + (size_t)tz * a.v_stride;
  const int nq = a.n_heads * half, nk = a.n_kv * half;
  for (int t = threadIdx.x; t < nq + nk; t += kThreads) {
    const bool isq = t < nq;
    const int u = isq ? t : t - nq;
    const int h = u / half, i = u - h * half;
    const float2 c = cs[i];
    const float *src = isq ? q + (size_t)h * a.hd : kin + (size_t)h * a.hd;
    const float x0 = src[2 * i], x1 = src[2 * i + 1];
    const float y0 = x0 * c.x - x1 * c.y;
    const float y1 = x0 * c.y + x1 * c.x;
    if (isq) {
      q[(size_t)h * a.hd + 2 * i] = y0;
      q[(size_t)h * a.hd + 2 * i + 1] = y1;
    } else {
      float *dst = a.kc + ((size_t)h * a.max_seq + p) * a.hd;
      dst[2 * i] = y0;
      dst[2 * i + 1] = y1;
    }
  }
  for (int t = threadIdx.x; t < a.n_kv * a.hd; t += kThreads) {
    const int h = t / a.hd, d = t - h * a.hd;
    a.vc[((size_t)h * a.max_seq + p) * a.hd + d] = vin[t];
  }
}

/* Positions per split-K chunk (one workgroup). */
constexpr int kChunk = 128;

/* Workgroup (g, c) handles positions [128c, 128c + 128) of KV head g for the
 * G query heads sharing it.  Every K and V load of the chunk is issued before
 * any arithmetic (64 + 64 VGPRs per thread at head_dim 128), so a workgroup
 * costs one memory round trip plus its FMAs. */
template <int HD, int G>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(AttnArgs a) {
  constexpr int S = kChunk;
  constexpr int LPP = HD / 8;          /* lanes per position, phase 1 */
  constexpr int PPI = kThreads / LPP;  /* positions per pass, phase 1 */
  constexpr int KIT = S / PPI;
  constexpr int DG = HD / 4;           /* float4 columns of a V row */
  constexpr int NPG = kThreads / DG;   /* position groups, phase 3 */
  constexpr int VIT = S / NPG;
  __shared__ float ss[G][S];
  __shared__ float4 sr[NPG][G][DG];

  const int g = blockIdx.x, c = blockIdx.y, tz = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  /* token tz of a chunk (0 for one token): its query, partials, position */
  const int pos = (a.pos_dev ? gld<int>(a.pos_dev) : a.pos) + tz;
  const float *aq = a.q + (size_t)tz * a.q_stride;
  float *part_o = a.part_o + (size_t)tz * a.po_stride, *part_ml = a.part_ml + (size_t)tz * a.pml_stride;
  const int L = min(pos + 1, a.max_seq);
  const int c0 = c * S;
  const int n = min(S, L - c0);
  if (n <= 0) return; /* past the sequence: the merge reads chunks < ceil(L/S) */
  const int h0 = g * G;
  const float *K = a.k + ((size_t)g * a.max_seq + c0) * HD;
  const float *V = a.v + ((size_t)g * a.max_seq + c0) * HD;

  /* V rows of phase 3 first: they do not depend on the scores */
  const int dg = tid % DG, pg = tid / DG;
  float4 vr[VIT];
#pragma unroll
  for (int k = 0; k < VIT; k++) vr[k] = gld<float4>(V + (size_t)min(pg + NPG * k, n - 1) * HD + 4 * dg);
  /* query slices and K rows of phase 1 */
  const int sub = tid % LPP, pw = tid / LPP;
  const int d0 = 4 * sub, d1 = HD / 2 + 4 * sub;
  float4 qa[G], qb[G];
#pragma unroll
  for (int h = 0; h < G; h++) {
    qa[h] = gld<float4>(aq + (size_t)(h0 + h) * HD + d0);
    qb[h] = gld<float4>(aq + (size_t)(h0 + h) * HD + d1);
  }
  float4 ka[KIT], kb[KIT];
#pragma unroll
  for (int k = 0; k < KIT; k++) {
    const float *kr = K + (size_t)min(pw + PPI * k, n - 1) * HD;
    ka[k] = gld<float4>(kr + d0);
    kb[k] = gld<float4>(kr + d1);
  }

  /* phase 1: scores (q . k) * 1/sqrt(hd) */
#pragma unroll
  for (int k = 0; k < KIT; k++) {
    const int j = pw + PPI * k;
#pragma unroll
    for (int h = 0; h < G; h++) {
      float s = qa[h].x * ka[k].x;
      s = __builtin_fmaf(qa[h].y, ka[k].y, s);
      s = __builtin_fmaf(qa[h].z, ka[k].z, s);
      s = __builtin_fmaf(qa[h].w, ka[k].w, s);
      s = __builtin_fmaf(qb[h].x, kb[k].x, s);
      s = __builtin_fmaf(qb[h].y, kb[k].y, s);
      s = __builtin_fmaf(qb[h].z, kb[k].z, s);
      s = __builtin_fmaf(qb[h].w, kb[k].w, s);
      s = LPP == 16 ? gq_row16_sum(s) : gq_row8_sum(s);
      if (sub == 0 && j < n) ss[h][j] = s * a.scale;
    }
  }
  __syncthreads();

  /* phase 2: chunk max, exponentials and their sum per head */
  const size_t ml = (size_t)a.nch * 2;
  for (int h = wave; h < G; h += kThreads / GQ_WAVE) {
    float m = -INFINITY;
    for (int j = lane; j < n; j += GQ_WAVE) m = fmaxf(m, ss[h][j]);
    m = gq_wave_max(m);
    float l = 0.f;
    for (int j = lane; j < n; j += GQ_WAVE) {
      const float e = expf(ss[h][j] - m);
      ss[h][j] = e;
      l += e;
    }
    l = gq_wave_sum(l);
    if (lane == 0) {
      gst<float>(part_ml + (size_t)(h0 + h) * ml + 2 * c, m);
      gst<float>(part_ml + (size_t)(h0 + h) * ml + 2 * c + 1, l);
    }
  }
  __syncthreads();

  /* phase 3: o = sum_j p_j V_j over the chunk */
  float4 acc[G];
#pragma unroll
  for (int h = 0; h < G; h++) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < VIT; k++) {
    const int j = pg + NPG * k;
    if (j < n) {
#pragma unroll
      for (int h = 0; h < G; h++) {
        const float p = ss[h][j];
        acc[h].x = __builtin_fmaf(p, vr[k].x, acc[h].x);
        acc[h].y = __builtin_fmaf(p, vr[k].y, acc[h].y);
        acc[h].z = __builtin_fmaf(p, vr[k].z, acc[h].z);
        acc[h].w = __builtin_fmaf(p, vr[k].w, acc[h].w);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) sr[pg][h][dg] = acc[h];
  __syncthreads();
  for (int t = tid; t < G * DG; t += kThreads) {
    const int h = t / DG, q = t - h * DG;
    float4 o = sr[0][h][q];
#pragma unroll
    for (int p = 1; p < NPG; p++) {
      const float4 u = sr[p][h][q];
      o.x += u.x, o.y += u.y, o.z += u.z, o.w += u.w;
    }
    gst<float4>(part_o + ((size_t)(h0 + h) * a.nch + c) * HD + 4 * q, o);
  }
}

/* Merge the chunks of one query head for 32 of its dimensions:
 * out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M). */
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(AttnArgs a) {
  extern __shared__ float sw[]; /* [nch] weights e^(m_c - M), then l_c */
  __shared__ float red[kThreads / GQ_WAVE];
  __shared__ float sacc[kThreads / 32][32];
  const int h = blockIdx.x, tz = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pos = (a.pos_dev ? gld<int>(a.pos_dev) : a.pos) + tz;
  const int L = min(pos + 1, a.max_seq);
  const int nc = (L + kChunk - 1) / kChunk;
  const float *ml = a.part_ml + (size_t)tz * a.pml_stride + (size_t)h * a.nch * 2;
  float *sl = sw + a.nch;
  float m = -INFINITY;
  for (int c = tid; c < nc; c += kThreads) {
    const float mc = gld<float>(ml + 2 * c);
    sw[c] = mc;
    sl[c] = gld<float>(ml + 2 * c + 1);
    m = fmaxf(m, mc);
  }
  m = gq_wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float l = 0.f;
  for (int c = tid; c < nc; c += kThreads) {
    const float w = expf(sw[c] - M);
    sw[c] = w;
    l = __builtin_fmaf(sl[c], w, l);
  }
  l = gq_wave_sum(l);
  __syncthreads();
  if (lane == 0) red[wave] = l;
  __syncthreads();
  const float Ls = (red[0] + red[1]) + (red[2] + red[3]);
  const int d = blockIdx.y * 32 + (tid & 31), cg = tid >> 5;
  const float *o = a.part_o + (size_t)tz * a.po_stride + (size_t)h * a.nch * a.hd + d;
  float acc = 0.f;
#pragma unroll 8
  for (int c = cg; c < nc; c += kThreads / 32) acc = __builtin_fmaf(gld<float>(o + (size_t)c * a.hd), sw[c], acc);
  sacc[cg][tid & 31] = acc;
  __syncthreads();
  if (tid < 32) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < kThreads / 32; k++) t += sacc[k][tid];
    const size_t o = (size_t)tz * a.out_stride + (size_t)h * a.hd + d;
    if (a.out16)
      gst<unsigned short>(a.out16 + o, __builtin_bit_cast(unsigned short, (__bf16)(t / Ls)));
    else
      gst<float>(a.out + o, t / Ls);
  }
}

template <int HD, int G>
int launch_partial(const AttnArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((attn_partial_kernel<HD, G>), dim3(a.n_kv, a.nch, std::max(a.ntok, 1)), dim3(kThreads), 0, s,
                     a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_partial_any(const AttnArgs &a, hipStream_t s) {
  const int G = a.n_heads / a.n_kv;
  if (a.hd == 128 && G == 4) return launch_partial<128, 4>(a, s);
  if (a.hd == 128 && G == 8) return launch_partial<128, 8>(a, s);
  if (a.hd == 128 && G == 1) return launch_partial<128, 1>(a, s);
  if (a.hd == 64 && G == 4) return launch_partial<64, 4>(a, s);
  if (a.hd == 64 && G == 8) return launch_partial<64, 8>(a, s);
  if (a.hd == 64 && G == 1) return launch_partial<64, 1>(a, s);
  return -1;
}

} // namespace

int gq_attn_nch(int n_kv, int max_seq) {
  (void)n_kv;
  return (max_seq + kChunk - 1) / kChunk;
}

int gq_attn_smax(int max_seq, int nch) {
  (void)max_seq;
  (void)nch;
  return kChunk;
}

int gq_launch_attention(const AttnArgs &a, hipStream_t s, hipEvent_t mid) {
  if (a.n_kv <= 0 || a.n_heads % a.n_kv || a.nch != gq_attn_nch(a.n_kv, a.max_seq)) return -1;
  if (a.hd % 32 || (size_t)a.nch * 2 * sizeof(float) > 32768 || a.ntok > 1) return -1;
  const int rc = launch_partial_any(a, s);
  if (rc) return rc;
  if (mid) (void)hipEventRecord(mid, s);
  hipLaunchKernelGGL(attn_merge_kernel, dim3(a.n_heads, a.hd / 32), dim3(kThreads),
                     (size_t)a.nch * 2 * sizeof(float), s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_attention_chunk(const AttnArgs &a, hipStream_t s) {
  if (a.n_kv <= 0 || a.n_heads % a.n_kv || a.ntok < 1 || a.hd % 32 || a.pos < 0) return -1;
  if (a.pos + a.ntok > a.max_seq || a.nch != (a.pos + a.ntok + kChunk - 1) / kChunk) return -1;
  if ((size_t)a.nch * 2 * sizeof(float) > 32768 || a.po_stride < (size_t)a.n_heads * a.nch * a.hd ||
      a.pml_stride < (size_t)a.n_heads * a.nch * 2)
    return -1;
  const int rc = launch_partial_any(a, s);
  if (rc) return rc;
  hipLaunchKernelGGL(attn_merge_kernel, dim3(a.n_heads, a.hd / 32, a.ntok), dim3(kThreads),
                     (size_t)a.nch * 2 * sizeof(float), s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_rope_append(const RopeArgs &a, hipStream_t s) {
  if ((a.hd & 1) || a.n_kv <= 0 || a.ntok < 0) return -1;
  hipLaunchKernelGGL(rope_append_kernel, dim3(std::max(a.ntok, 1)), dim3(kThreads), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
