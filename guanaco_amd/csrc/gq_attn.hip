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
 * rounded separately, :415-429) and writes K and V at row pos of the slab
 * (kv_cache.c:101-125 with pos < max_seq; the device cache does not wrap,
 * the host rejects pos >= max_seq with -5 and the kernel returns for such a
 * position).  Appended rows are bit copies of the reference's.
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
 *
 * flash_prefill: causal attention of a prefill chunk (many query tokens) on
 * the fp32 matrix cores; see the kernel.
 */
#include <algorithm>

#include "gq_device.h"
#include "gq_internal.h"

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void rope_append_kernel(RopeArgs a) {
#pragma clang fp contract(off)
  /* token blockIdx.x / n_kv of a chunk (0 for one token), KV head
   * g = blockIdx.x % n_kv and its G query heads: workgroup L runs on XCD
   * L mod 8, so head g's K/V rows are written where the flash kernel, which
   * takes head g on those workgroups, reads them */
  const int tz = (int)blockIdx.x / a.n_kv, g = (int)blockIdx.x % a.n_kv, G = a.n_heads / a.n_kv;
  const int pos = (a.pos_dev ? *a.pos_dev : a.pos) + tz;
  /* the host rejects positions outside the cache; this keeps a stray
   * device-side position from indexing past the table or the slab */
  if (pos < 0 || pos >= a.max_seq) return;
  const int half = a.hd >> 1;
  const int p = pos;
  const float2 *cs = a.cs + (size_t)pos * half;
  float *q = a.q + (size_t)tz * a.q_stride;
  const float *kin = a.k + (size_t)tz * a.k_stride, *vin = a.v + (size_t)tz * a.v_stride;
  /* element o of this token's q | k | v from the GEMM's parts, summed in
   * pg_parts_kernel's order */
  const int qd = a.n_heads * a.hd, kvd = a.n_kv * a.hd;
  const float *prow = a.parts ? a.parts + (size_t)tz * a.prow : nullptr;
  /* element pairs (2i, 2i + 1) move as one 8-byte access when every address
   * of this token allows it (always, from the runtime's own buffers: hd and
   * the strides are even); op-level callers' 4-byte-aligned buffers take
   * two scalar accesses.  The values and their order are the same. */
  const bool v2 = ((uintptr_t)q & 7) == 0 && (((uintptr_t)a.kc | (uintptr_t)a.vc) & 7) == 0 &&
                  (prow ? ((uintptr_t)prow & 7) == 0 && (a.pstride & 1) == 0
                        : (((uintptr_t)kin | (uintptr_t)vin) & 7) == 0);
  auto ld2 = [&](const float *s) {
    return v2 ? gld<float2>(s) : make_float2(s[0], s[1]);
  };
  auto st2 = [&](float *d, float2 y) {
    if (v2) gst<float2>(d, y);
    else d[0] = y.x, d[1] = y.y;
  };
  auto part2 = [&](int o) {
    float2 v = ld2(prow + o);
    for (int k = 1; k < a.kparts; k++) {
      const float2 u = ld2(prow + (size_t)k * a.pstride + o);
      v.x += u.x, v.y += u.y;
    }
    return v;
  };
  for (int t = threadIdx.x; t < (G + 1) * half; t += kThreads) {
    const bool isq = t < G * half;
    const int u = isq ? t : t - G * half;
    const int hl = u / half, i = u - hl * half;
    const int h = isq ? g * G + hl : g;
    const float2 c = cs[i];
    const float2 x = prow ? part2((isq ? 0 : qd) + h * a.hd + 2 * i)
                          : ld2((isq ? (const float *)q : kin) + (size_t)h * a.hd + 2 * i);
    const float2 y = make_float2(x.x * c.x - x.y * c.y, x.x * c.y + x.y * c.x);
    st2(isq ? q + (size_t)h * a.hd + 2 * i : a.kc + ((size_t)h * a.max_seq + p) * a.hd + 2 * i, y);
  }
  for (int d = 2 * threadIdx.x; d < a.hd; d += 2 * kThreads) {
    const int t = g * a.hd + d;
    st2(a.vc + ((size_t)g * a.max_seq + p) * a.hd + d, prow ? part2(qd + kvd + t) : ld2(vin + t));
  }
}

/* Positions per split-K chunk (one workgroup), chosen by the cache
 * capacity.  32 gives 2080 workgroups at the 8B shape and ctx 8192 (79
 * VGPRs, six waves per SIMD): measured in the graph-replayed decode step
 * 0.9% faster than 64 (four workgroups per CU), although the attention op
 * alone, launched back to back, is 0.4 us slower; 64 had in turn measured
 * 1.3% faster per step than 128.  Past 12288 positions the merge, which
 * reads every chunk's partials, grows enough that 128 wins (16384: 32.7 vs
 * 34.7 us per layer with 64; 32768: 57.0 vs 61.9). */
int chunk_for(int max_seq) { return max_seq > 12288 ? 128 : 32; }

/* Workgroup (g, c) handles positions [Sc, Sc + S) of KV head g for the G
 * query heads sharing it.  Every K and V load of the chunk is issued before
 * any arithmetic (S/2 + S/2 VGPRs per thread at head_dim 128), so a
 * workgroup costs one memory round trip plus its FMAs. */
template <int HD, int G, int S>
__device__ __forceinline__ void attn_partial_body(const AttnArgs &a) {
  constexpr int LPP = HD / 8;          /* lanes per position, phase 1 */
  constexpr int PPI = kThreads / LPP;  /* positions per pass, phase 1 */
  constexpr int KIT = S / PPI;
  constexpr int DG = HD / 4;           /* float4 columns of a V row */
  constexpr int NPG = kThreads / DG;   /* position groups, phase 3 */
  constexpr int VIT = S / NPG;
  __shared__ float ss[G][S];
  __shared__ float4 sr[NPG][G][DG];

  const int g = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int pos = a.pos_dev ? gld<int>(a.pos_dev) : a.pos;
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
  for (int k = 0; k < VIT; k++) vr[k] = gld_nt<float4>(V + (size_t)min(pg + NPG * k, n - 1) * HD + 4 * dg);
  /* query slices and K rows of phase 1 */
  const int sub = tid % LPP, pw = tid / LPP;
  const int d0 = 4 * sub, d1 = HD / 2 + 4 * sub;
  float4 qa[G], qb[G];
#pragma unroll
  for (int h = 0; h < G; h++) {
    qa[h] = gld<float4>(a.q + (size_t)(h0 + h) * HD + d0);
    qb[h] = gld<float4>(a.q + (size_t)(h0 + h) * HD + d1);
  }
  float4 ka[KIT], kb[KIT];
#pragma unroll
  for (int k = 0; k < KIT; k++) {
    const float *kr = K + (size_t)min(pw + PPI * k, n - 1) * HD;
    ka[k] = gld_nt<float4>(kr + d0);
    kb[k] = gld_nt<float4>(kr + d1);
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
      gst<float>(a.part_ml + (size_t)(h0 + h) * ml + 2 * c, m);
      gst<float>(a.part_ml + (size_t)(h0 + h) * ml + 2 * c + 1, l);
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
    gst<float4>(a.part_o + ((size_t)(h0 + h) * a.nch + c) * HD + 4 * q, o);
  }
}

template <int HD, int G, int S>
__global__ __launch_bounds__(kThreads) void attn_partial_kernel(AttnArgs a) {
  attn_partial_body<HD, G, S>(a);
}

/* 32-position chunks at 7 waves per SIMD: 72 VGPRs, no spill (the free
 * allocation took 79, six waves).  The 2,056 workgroups of ctx 8193 then
 * take ~1.15 rounds instead of ~1.35: 18.9 against 19.1 us per layer, decode
 * +0.4%.  Eight waves (64 VGPRs) spilled and ran at 29.7 us. */
template <int HD, int G>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(7, 8))) void attn_partial32_kernel(AttnArgs a) {
  attn_partial_body<HD, G, 32>(a);
}

/* Dimensions of one query head per merge workgroup.  16 (256 workgroups at
 * 32 heads x 128) measured faster in the graph-replayed decode than 32:
 * each thread's chain of chunk loads is half as long. */
constexpr int kMergeDims = 16;

/* Merge the chunks of one query head for kMergeDims of its dimensions:
 * out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M). */
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(AttnArgs a) {
  constexpr int NG = kThreads / kMergeDims; /* chunk groups */
  extern __shared__ float sw[]; /* [nch] weights e^(m_c - M), then l_c */
  __shared__ float red[kThreads / GQ_WAVE];
  __shared__ float sacc[NG][kMergeDims];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pos = a.pos_dev ? gld<int>(a.pos_dev) : a.pos;
  const int L = min(pos + 1, a.max_seq);
  const int nc = (L + a.s_max - 1) / a.s_max;
  const float *ml = a.part_ml + (size_t)h * a.nch * 2;
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
  const int d = blockIdx.y * kMergeDims + tid % kMergeDims, cg = tid / kMergeDims;
  const float *o = a.part_o + (size_t)h * a.nch * a.hd + d;
  float acc = 0.f;
  /* unrolled so a thread's ~16 chunk loads (260 chunks at ctx 8192 over 16
   * chunk groups) go out in one batch: decode +0.4% against unroll 8 */
#pragma unroll 16
  for (int c = cg; c < nc; c += NG) acc = __builtin_fmaf(gld<float>(o + (size_t)c * a.hd), sw[c], acc);
  sacc[cg][tid % kMergeDims] = acc;
  __syncthreads();
  if (tid < kMergeDims) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < NG; k++) t += sacc[k][tid];
    gst<float>(a.out + (size_t)h * a.hd + d, t / Ls);
  }
}

template <int HD, int G>
int launch_partial(const AttnArgs &a, hipStream_t s) {
  if (a.s_max == 128)
    hipLaunchKernelGGL((attn_partial_kernel<HD, G, 128>), dim3(a.n_kv, a.nch), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((attn_partial32_kernel<HD, G>), dim3(a.n_kv, a.nch), dim3(kThreads), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

} // namespace

int gq_attn_nch(int n_kv, int max_seq) {
  (void)n_kv;
  const int s = chunk_for(max_seq);
  return (max_seq + s - 1) / s;
}

int gq_attn_smax(int max_seq, int nch) {
  (void)nch;
  return chunk_for(max_seq);
}

int gq_launch_attention(const AttnArgs &a, hipStream_t s, hipEvent_t mid) {
  if (a.n_kv <= 0 || a.n_heads % a.n_kv || a.nch != gq_attn_nch(a.n_kv, a.max_seq) ||
      a.s_max != chunk_for(a.max_seq))
    return -1;
  if (a.hd % 32 || (size_t)a.nch * 2 * sizeof(float) > 32768) return -1;
  const int G = a.n_heads / a.n_kv;
  int rc = -1;
  if (a.hd == 128 && G == 4) rc = launch_partial<128, 4>(a, s);
  else if (a.hd == 128 && G == 8) rc = launch_partial<128, 8>(a, s);
  else if (a.hd == 128 && G == 1) rc = launch_partial<128, 1>(a, s);
  else if (a.hd == 128 && G == 2) rc = launch_partial<128, 2>(a, s);
  else if (a.hd == 64 && G == 4) rc = launch_partial<64, 4>(a, s);
  else if (a.hd == 64 && G == 8) rc = launch_partial<64, 8>(a, s);
  else if (a.hd == 64 && G == 1) rc = launch_partial<64, 1>(a, s);
  else if (a.hd == 64 && G == 2) rc = launch_partial<64, 2>(a, s);
  if (rc) return rc;
  if (mid) (void)hipEventRecord(mid, s);
  hipLaunchKernelGGL(attn_merge_kernel, dim3(a.n_heads, a.hd / kMergeDims), dim3(kThreads),
                     (size_t)a.nch * 2 * sizeof(float), s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

namespace {

typedef float gq_f32x4 __attribute__((ext_vector_type(4)));
typedef float gq_f2a __attribute__((ext_vector_type(2)));
typedef __bf16 gq_bf2a __attribute__((ext_vector_type(2)));

/* Causal attention of a prefill chunk on the fp32 matrix cores
 * (v_mfma_f32_16x16x4_f32), flash-attention style: one wave per 16 query
 * rows = 16 / G tokens x the G query heads of KV head g (the heads that
 * share K/V), streaming the keys 0 .. (last token's position) in blocks of
 * 16 with an online softmax.  Per block:
 *   S^T = K Q^T   D[key][row]: lane (c, j) = (lane % 16, lane / 16) holds
 *                 row c, keys 4 j + i (i < 4); the head dimension is split
 *                 into 4 lane groups (dims HD/4 j ..) so every MFMA step
 *                 reads one K and one Q float per lane;
 *   scale, mask keys past each row's position, running max / sum across
 *   the 4 lanes of a row;
 *   O += P V      A = P straight from the S^T layout (step i takes keys
 *                 4 j + i), B = V rows; output tile d holds dims ND c + d,
 *                 so a lane reads ND consecutive floats of each V row and
 *                 holds ND consecutive output dims of rows 4 j + i.
 * Four waves per workgroup take every fourth key block each and combine
 * their (max, sum, O) through LDS at the end, so the longest causal rows
 * finish in a quarter of the time.  One register buffer per wave: the next
 * block's K loads once the scores have read K, its V once P V has read V,
 * which keeps the kernel at 208 VGPRs, two waves per SIMD (two buffers
 * needed 312, one wave per SIMD, and ran 1.25-1.4x slower).  Same mathematics as the reference (engine.c:476-501:
 * scores * 1/sqrt(hd), -inf past the query position, softmax, P V) in fp32
 * throughout; only the summation order differs. */
template <int HD, int G>
__global__ __launch_bounds__(256) void flash_prefill_kernel(AttnArgs a) {
  constexpr int TPT = 16 / G; /* tokens per tile */
  constexpr int NS = HD / 4;  /* QK^T MFMA steps */
  constexpr int ND = HD / 16; /* output tiles over the head dimension */
  __shared__ float xm[3][64], xl[3][64], xo[3][ND * 4][64];
  const int lane = threadIdx.x & 63, c = lane & 15, j = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  /* One linear grid: workgroup L runs on XCD L mod 8, and takes KV head
   * L mod n_kv, so a head's K/V stays in one XCD's L2 (n_kv = 8: one head
   * per XCD; with tile-major ids every XCD read every head's K/V, 4 MB at
   * 512 tokens: 49.3 -> 38.6 us per layer).  Heavy (late) tiles first. */
  const int ntile = gridDim.x / a.n_kv;
  const int g = blockIdx.x % a.n_kv, tile = ntile - 1 - blockIdx.x / a.n_kv;
  const int t0 = tile * TPT;
  const int last = min(t0 + TPT, a.ntok) - 1;
  const int pmax = a.pos + last; /* last key any row of the tile needs */
  /* B operand of S^T: row c's query, dims NS j .. NS j + NS - 1 */
  const int qt = min(t0 + c / G, a.ntok - 1), qh = g * G + c % G;
  float qv[NS];
  {
    const float *qp = a.q + (size_t)qt * a.q_stride + (size_t)qh * HD + NS * j;
#pragma unroll
    for (int s4 = 0; s4 < NS / 4; s4++) {
      const float4 v = gld<float4>(qp + 4 * s4);
      qv[4 * s4] = v.x, qv[4 * s4 + 1] = v.y, qv[4 * s4 + 2] = v.z, qv[4 * s4 + 3] = v.w;
    }
  }
  const int cpos = a.pos + t0 + c / G; /* row c's position (S^T layout) */
  const float *K = a.k + (size_t)g * a.max_seq * HD;
  const float *V = a.v + (size_t)g * a.max_seq * HD;
  float m = -INFINITY, l = 0.f;
  gq_f32x4 o[ND];
#pragma unroll
  for (int d = 0; d < ND; d++) o[d] = gq_f32x4{0.f, 0.f, 0.f, 0.f};
  const int nblk = pmax / 16 + 1;
  /* K row key0 + c, dims NS j ..; V rows key0 + 4 j + i, dims ND c ..
   * (rows past pmax are never weighted: zeroed so stale cache contents
   * cannot leak in as 0 * inf). */
  float kv[NS], vv[4][ND];
  auto loadk = [&](int key0, float (&kq)[NS]) {
    const float *kp = K + (size_t)min(key0 + c, a.max_seq - 1) * HD + NS * j;
#pragma unroll
    for (int s4 = 0; s4 < NS / 4; s4++) {
      const float4 v = gld<float4>(kp + 4 * s4);
      kq[4 * s4] = v.x, kq[4 * s4 + 1] = v.y, kq[4 * s4 + 2] = v.z, kq[4 * s4 + 3] = v.w;
    }
  };
  auto loadv = [&](int key0, float (&vq)[4][ND]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int key = key0 + 4 * j + i;
      const float *vp = V + (size_t)min(key, a.max_seq - 1) * HD + ND * c;
#pragma unroll
      for (int d4 = 0; d4 < ND / 4; d4++) {
        float4 v = gld<float4>(vp + 4 * d4);
        if (key > pmax) v = make_float4(0.f, 0.f, 0.f, 0.f);
        vq[i][4 * d4] = v.x, vq[i][4 * d4 + 1] = v.y, vq[i][4 * d4 + 2] = v.z, vq[i][4 * d4 + 3] = v.w;
      }
    }
  };
  /* one key block: S^T (four independent MFMA chains), mask, online
   * softmax, rescale, O += P V */
  auto stepS = [&](int key0, const float (&kq)[NS], float (&p)[4]) {
    gq_f32x4 sp[4];
#pragma unroll
    for (int u = 0; u < 4; u++) sp[u] = gq_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; s++) sp[s & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(kq[s], qv[s], sp[s & 3], 0, 0, 0);
    const gq_f32x4 st = (sp[0] + sp[1]) + (sp[2] + sp[3]);
    /* st[i] = q(row c) . k(key0 + 4 j + i) */
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sv[i] = key0 + 4 * j + i <= cpos ? st[i] * a.scale : -INFINITY;
    float mb = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
    mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
    /* a wave's rows may not see any key of its first blocks (the second
     * wave starts at block 1): keep m = -inf and weigh those blocks 0 */
    const float mn = fmaxf(m, mb);
    const float ms = mn == -INFINITY ? 0.f : mn;
    const float alpha = __expf(m - ms);
    float lb = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      p[i] = __expf(sv[i] - ms);
      lb += p[i];
    }
    lb += __shfl_xor(lb, 16, 64);
    lb += __shfl_xor(lb, 32, 64);
    l = __builtin_fmaf(l, alpha, lb);
    m = mn;
    /* O rows 4 j + i take the rescale of row 4 j + i (held by lane 4 j + i) */
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float al = __shfl(alpha, 4 * j + i, 64);
#pragma unroll
      for (int d = 0; d < ND; d++) o[d][i] *= al;
    }
  };
  auto stepPV = [&](const float (&p)[4], const float (&vq)[4][ND]) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int d = 0; d < ND; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[i], vq[i][d], o[d], 0, 0, 0);
  };
  /* wave wv takes blocks wv, wv + 4, ...; the wave's next block loads into
   * the registers as the current one frees them */
  if (wv < nblk) loadk(16 * wv, kv), loadv(16 * wv, vv);
  for (int b = wv; b < nblk; b += 4) {
    float p[4];
    stepS(16 * b, kv, p);
    if (b + 4 < nblk) loadk(16 * (b + 4), kv);
    stepPV(p, vv);
    if (b + 4 < nblk) loadv(16 * (b + 4), vv);
  }
  /* combine: waves 1-3 hand (m, l, O) to wave 0 (wave 0 holds block 0, so
   * its m is finite; a wave that had no block has m = -inf and weighs 0) */
  if (wv > 0) {
    xm[wv - 1][lane] = m, xl[wv - 1][lane] = l;
#pragma unroll
    for (int d = 0; d < ND; d++)
#pragma unroll
      for (int i = 0; i < 4; i++) xo[wv - 1][4 * d + i][lane] = o[d][i];
  }
  __syncthreads();
  if (wv > 0) return;
#pragma unroll
  for (int w = 0; w < 3; w++) {
    const float m1 = xm[w][lane], mt = fmaxf(m, m1);
    const float s0 = __expf(m - mt), s1 = __expf(m1 - mt);
    l = l * s0 + xl[w][lane] * s1;
    m = mt;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float a0 = __shfl(s0, 4 * j + i, 64), a1 = __shfl(s1, 4 * j + i, 64);
#pragma unroll
      for (int d = 0; d < ND; d++) o[d][i] = o[d][i] * a0 + xo[w][4 * d + i][lane] * a1;
    }
  }
  /* out[row] = O[row] / l[row]; row 4 j + i -> token t0 + row / G, head
   * g G + row % G */
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = 4 * j + i, t = t0 + row / G, h = g * G + row % G;
    const float inv = 1.0f / __shfl(l, row, 64);
    if (t < a.ntok) {
      const size_t base = (size_t)t * a.out_stride + (size_t)h * HD + ND * c;
#pragma unroll
      for (int d4 = 0; d4 < ND / 4; d4++) {
        const float4 v = make_float4(o[4 * d4][i] * inv, o[4 * d4 + 1][i] * inv, o[4 * d4 + 2][i] * inv,
                                     o[4 * d4 + 3][i] * inv);
        if (a.out16) {
          uint2 u;
          u.x = __builtin_bit_cast(uint32_t, __builtin_convertvector((gq_f2a){v.x, v.y}, gq_bf2a));
          u.y = __builtin_bit_cast(uint32_t, __builtin_convertvector((gq_f2a){v.z, v.w}, gq_bf2a));
          gst<uint2>(a.out16 + base + 4 * d4, u);
        } else {
          gst<float4>(a.out + base + 4 * d4, v);
        }
      }
    }
  }
}

template <int HD, int G>
int launch_flash(const AttnArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((flash_prefill_kernel<HD, G>), dim3((a.ntok + 16 / G - 1) / (16 / G) * a.n_kv), dim3(256), 0, s,
                     a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

} // namespace

int gq_launch_flash_prefill(const AttnArgs &a, hipStream_t s) {
  if (a.n_kv <= 0 || a.n_heads % a.n_kv || a.ntok < 1 || a.pos < 0 || a.pos + a.ntok > a.max_seq) return -1;
  const int G = a.n_heads / a.n_kv;
  if (a.hd == 128 && G == 4) return launch_flash<128, 4>(a, s);
  if (a.hd == 128 && G == 8) return launch_flash<128, 8>(a, s);
  if (a.hd == 128 && G == 1) return launch_flash<128, 1>(a, s);
  if (a.hd == 128 && G == 2) return launch_flash<128, 2>(a, s);
  if (a.hd == 64 && G == 4) return launch_flash<64, 4>(a, s);
  if (a.hd == 64 && G == 8) return launch_flash<64, 8>(a, s);
  if (a.hd == 64 && G == 1) return launch_flash<64, 1>(a, s);
  if (a.hd == 64 && G == 2) return launch_flash<64, 2>(a, s);
  return -1;
}

int gq_launch_rope_append(const RopeArgs &a, hipStream_t s) {
  if ((a.hd & 1) || a.n_kv <= 0 || a.n_heads % a.n_kv || a.ntok < 0 || (a.parts && a.kparts < 1)) return -1;
  hipLaunchKernelGGL(rope_append_kernel, dim3(std::max(a.ntok, 1) * a.n_kv), dim3(kThreads), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
