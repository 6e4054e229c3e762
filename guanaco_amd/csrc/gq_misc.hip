/*
 * gq_misc.hip — small decode-step kernels: RMSNorm, embedding-row dequant,
 * greedy argmax (with the decode loop's device-side bookkeeping), SiLU*up,
 * and the device fills of the synthetic-input generator (gq_synth.h).
 */
#include <algorithm>

#include "gq_device.h"
#include "gq_internal.h"
#include "gq_synth.h"

namespace {

constexpr int kThreads = 256;

/* out = w * (x * 1/sqrt(mean(x^2) + eps)) (kernels_cpu.c:199-265); one
 * workgroup per row (blockIdx.x), sum of squares in a fixed tree order.  A
 * row of up to kNormVec * 4 * kThreads floats is read once into registers
 * (float4 per thread and pass) when dim % 4 == 0 and rows are 16-byte
 * aligned; other shapes take the scalar two-pass loop. */
constexpr int kNormVec = 16;

/* parts != NULL: the row is first x + ((part 0 + part 1) + ...), the sum of
 * a K-split GEMM's parts added to the residual as pg_parts_kernel does
 * (part p of the row at parts + p * pstride), and is stored to xnew */
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *x, const float *w, float *out,
                                                          int dim, float eps, __bf16 *out16, const float *parts,
                                                          int kparts, size_t pstride, float *xnew) {
  __shared__ float red[kThreads / GQ_WAVE];
  const int tid = threadIdx.x;
  x += (size_t)blockIdx.x * dim;
  out += (size_t)blockIdx.x * dim;
  if (out16) out16 += (size_t)blockIdx.x * dim;
  if (parts) parts += (size_t)blockIdx.x * dim, xnew += (size_t)blockIdx.x * dim;
  const bool vec = (dim & 3) == 0 && dim <= kNormVec * 4 * kThreads && (((uintptr_t)x | (uintptr_t)out) & 15) == 0 &&
                   (!w || ((uintptr_t)w & 15) == 0) && (!out16 || ((uintptr_t)out16 & 7) == 0) &&
                   (!parts || (((uintptr_t)parts | (uintptr_t)xnew | pstride) & 3) == 0);
  float4 xv[kNormVec];
  float ss = 0.f;
  if (vec) {
#pragma unroll
    for (int k = 0; k < kNormVec; k++) {
      const int e = 4 * (tid + k * kThreads);
      if (e < dim) {
        xv[k] = gld<float4>(x + e);
        if (parts) {
          float4 s = gld<float4>(parts + e);
          for (int p = 1; p < kparts; p++) {
            const float4 u = gld<float4>(parts + p * pstride + e);
            s.x += u.x, s.y += u.y, s.z += u.z, s.w += u.w;
          }
          xv[k] = make_float4(xv[k].x + s.x, xv[k].y + s.y, xv[k].z + s.z, xv[k].w + s.w);
          gst<float4>(xnew + e, xv[k]);
        }
        ss = __builtin_fmaf(xv[k].x, xv[k].x, ss), ss = __builtin_fmaf(xv[k].y, xv[k].y, ss);
        ss = __builtin_fmaf(xv[k].z, xv[k].z, ss), ss = __builtin_fmaf(xv[k].w, xv[k].w, ss);
      }
    }
  } else {
    for (int i = tid; i < dim; i += kThreads) {
      float xi = x[i];
      if (parts) {
        float s = parts[i];
        for (int p = 1; p < kparts; p++) s += parts[p * pstride + i];
        xi = xi + s;
        xnew[i] = xi;
      }
      ss = __builtin_fmaf(xi, xi, ss);
    }
    if (parts) x = xnew; /* this thread's own elements, read back below */
  }
  ss = gq_wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = (red[0] + red[1]) + (red[2] + red[3]);
  tot = tot / (float)dim;
  tot = tot + eps;
  const float r = 1.0f / sqrtf(tot);
  if (vec) {
#pragma unroll
    for (int k = 0; k < kNormVec; k++) {
      const int e = 4 * (tid + k * kThreads);
      if (e < dim) {
        const float4 wv = w ? gld<float4>(w + e) : make_float4(1.f, 1.f, 1.f, 1.f);
        const float4 v = make_float4(wv.x * (xv[k].x * r), wv.y * (xv[k].y * r), wv.z * (xv[k].z * r),
                                     wv.w * (xv[k].w * r));
        if (out16) {
          uint2 u;
          u.x = (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)v.x) |
                ((uint32_t)__builtin_bit_cast(unsigned short, (__bf16)v.y) << 16);
          u.y = (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)v.z) |
                ((uint32_t)__builtin_bit_cast(unsigned short, (__bf16)v.w) << 16);
          gst<uint2>(out16 + e, u);
        } else {
          gst<float4>(out + e, v);
        }
      }
    }
    return;
  }
  for (int i = tid; i < dim; i += kThreads) {
    const float v = (w ? w[i] : 1.0f) * (x[i] * r);
    if (out16)
      out16[i] = (__bf16)v;
    else
      out[i] = v;
  }
}

/* Element e of embedding row `tok` (engine.c:214-283): F32 copy, Q8_0
 * q*scale, Q4_K (d*sc)*q - dmin*m with separate roundings. */
__device__ __forceinline__ float embed_value(int dtype, const uint8_t *table, int hidden, int tok, int e) {
#pragma clang fp contract(off)
  if (dtype == GQ_F32) return ((const float *)table)[(size_t)tok * hidden + e];
  if (dtype == GQ_Q8_0) {
    const uint8_t *blk = table + ((size_t)tok * (hidden / 32) + e / 32) * 34;
    return (float)(int8_t)blk[2 + (e & 31)] * gq_h2f(blk[0] | (blk[1] << 8));
  }
  const uint8_t *blk = table + ((size_t)tok * (hidden / 256) + e / 256) * 144;
  const int u = e & 255, cc = u >> 6, o = u & 63;
  const int j = 2 * cc + (o >= 32);
  const uint8_t *s = blk + 4;
  int sc, m;
  if (j < 4) {
    sc = s[j] & 63, m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
  const uint8_t qb = blk[16 + 32 * cc + (o & 31)];
  const int q = o < 32 ? (qb & 15) : (qb >> 4);
  const float d = gq_h2f(blk[0] | (blk[1] << 8)), dm = gq_h2f(blk[2] | (blk[3] << 8));
  const float d1 = d * (float)sc, m1 = dm * (float)m;
  return d1 * (float)q - m1;
}

/* Embedding row of `token`.  With tokens != NULL, row blockIdx.y holds
 * tokens[blockIdx.y] (out + blockIdx.y * hidden); blockIdx.x covers
 * 256-element slices of the row. */
__global__ __launch_bounds__(kThreads) void embed_kernel(int dtype, const uint8_t *table, int hidden,
                                                        const int *token_dev, int token, const int *tokens,
                                                        float *out) {
  const int tok = tokens ? tokens[blockIdx.y] : token_dev ? *token_dev : token;
  out += (size_t)blockIdx.y * hidden;
  for (int e = blockIdx.x * kThreads + threadIdx.x; e < hidden; e += gridDim.x * kThreads)
    out[e] = embed_value(dtype, table, hidden, tok, e);
}

/* (value, index) reduction, ties to the lower index (tokenizer.c:175-185). */
__device__ __forceinline__ void better(float &v, int &i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) v = v2, i = i2;
}

__device__ __forceinline__ void block_argmax(float &v, int &i) {
  __shared__ float sv[kThreads / GQ_WAVE];
  __shared__ int si[kThreads / GQ_WAVE];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const int i2 = __shfl_xor(i, o, 64);
    better(v, i, v2, i2);
  }
  const int tid = threadIdx.x;
  if ((tid & 63) == 0) sv[tid >> 6] = v, si[tid >> 6] = i;
  __syncthreads();
  v = sv[0], i = si[0];
  for (int w = 1; w < kThreads / GQ_WAVE; w++) better(v, i, sv[w], si[w]);
}

constexpr int kArgmaxPerBlock = 1024; /* 126 workgroups for a 128256-entry vocabulary */

__global__ __launch_bounds__(kThreads) void argmax_stage1(const float *x, int n, float *scratch) {
  const int base = blockIdx.x * kArgmaxPerBlock;
  const int end = min(n, base + kArgmaxPerBlock);
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int e = base + threadIdx.x; e < end; e += kThreads) {
    float xe = x[e];
    /* sample_greedy starts from logits[0] and only a strictly greater value
     * replaces it, so a NaN there is never replaced: index 0 wins.  As +inf
     * it does, since ties go to the lowest index.  A NaN elsewhere never
     * compares greater and is skipped, as better() skips it. */
    if (e == 0 && xe != xe) xe = INFINITY;
    better(v, i, xe, e);
  }
  block_argmax(v, i);
  if (threadIdx.x == 0) {
    scratch[2 * blockIdx.x] = v;
    scratch[2 * blockIdx.x + 1] = __int_as_float(i);
  }
}

/* The winner of stage 1's block results.  With eout != NULL it also writes
 * the winner's embedding row (the next decode step's input) to eout: each
 * workgroup of the grid reduces the same block results to the same winner
 * and writes its 256-element slices of the row, and workgroup 0 alone
 * writes the token, the step and the position (one launch fewer than a
 * separate embedding after the argmax). */
__global__ __launch_bounds__(kThreads) void argmax_stage2(const float *scratch, int nblk, int *out,
                                                         int *tokens, int *step_dev, int *pos_dev, int edt,
                                                         const uint8_t *etab, int hidden, float *eout) {
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int b = threadIdx.x; b < nblk; b += kThreads)
    better(v, i, scratch[2 * b], __float_as_int(scratch[2 * b + 1]));
  block_argmax(v, i);
  if (i == 0x7fffffff) i = 0; /* all NaN: the reference keeps index 0 */
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *out = i;
    if (step_dev) {
      tokens[*step_dev] = i;
      *step_dev += 1;
      *pos_dev += 1;
    }
  }
  if (eout)
    for (int e = blockIdx.x * kThreads + threadIdx.x; e < hidden; e += gridDim.x * kThreads)
      eout[e] = embed_value(edt, etab, hidden, i, e);
}

__global__ void silu_mul_kernel(float *gate, const float *up, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float g = gate[i];
    const float sig = 1.0f / (1.0f + expf(0.0f - g));
    gate[i] = (g * sig) * up[i];
  }
}

/* Plain 16-byte-per-thread grid-stride copy: the reference workload for
 * scaling the HBM byte counters (n16 = bytes / 16). */
__global__ __launch_bounds__(kThreads) void copy_kernel(const uint4 *src, uint4 *dst, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += (size_t)gridDim.x * kThreads)
    gst<uint4>(dst + i, gld<uint4>(src + i));
}

/* Read-only streaming: every thread issues eight 16-byte loads spaced a
 * grid apart before it uses any, folds them into an XOR, and writes only in
 * the (data-dependent, practically never taken) case that the XOR equals a
 * marker, so the loads cannot be dropped and the kernel stores nothing.  The
 * grid covers the bytes in one pass at every size (a grid capped at 4096
 * workgroups, looping, read 431 MB at 4.9 TB/s against 5.9 in one pass).
 * The floor a launch of this many bytes can reach: what the decode kernels'
 * durations are set beside. */
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const uint4 *src, size_t n16, uint32_t *sink,
                                                               unsigned sink_n) {
  const size_t stride = (size_t)gridDim.x * kThreads;
  uint32_t acc = 0;
  /* every pass issues all eight loads (those past the end masked off)
   * before folding any */
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += 8 * stride) {
    uint4 v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = i + k * stride < n16 ? gld<uint4>(src + i + k * stride) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int k = 0; k < 8; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  if (acc == 0x9E3779B9u) gst<uint32_t>(sink + blockIdx.x % sink_n, acc);
}

/* ---- synthetic fills: one thread per 4 output bytes / one float ---- */
__global__ void synth_quant_kernel(uint8_t *out, int dtype, size_t nbytes, int bb, uint64_t seed) {
  const size_t i4 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i4 >= nbytes) return;
  uint32_t word = 0;
  for (int k = 0; k < 4 && i4 + k < nbytes; k++) {
    const size_t i = i4 + k;
    const uint64_t b = i / (size_t)bb;
    const uint32_t o = (uint32_t)(i - b * bb);
    const uint8_t v = dtype == GQ_Q4_K                             ? gq_q4k_byte(seed, b, o)
                      : dtype == (GQ_Q4_K | GQ_SYNTH_Q4K_ZERO_MEAN) ? gq_q4k_zm_byte(seed, b, o)
                      : dtype == GQ_Q6_K                             ? gq_q6k_byte(seed, b, o)
                                                                     : gq_q8_0_byte(seed, b, o);
    word |= (uint32_t)v << (8 * k);
  }
  if (i4 + 4 <= nbytes) {
    *(uint32_t *)(out + i4) = word;
  } else {
    for (int k = 0; i4 + k < nbytes; k++) out[i4 + k] = (uint8_t)(word >> (8 * k));
  }
}

__global__ void synth_normal_kernel(float *out, size_t n, uint64_t seed, int norm_weight) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = norm_weight ? gq_norm_weight(seed, i) : gq_normal(seed, i);
}

__global__ void synth_kv_kernel(float *slab, int n_kv, int hd, int max_seq, int n_pos, uint64_t seed) {
  /* blockIdx.y = layer * n_kv + head; x covers n_pos * hd elements */
  const int lh = blockIdx.y;
  const int layer = lh / n_kv, h = lh - layer * n_kv;
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (size_t)n_pos * hd) return;
  const int p = (int)(e / hd), d = (int)(e - (size_t)p * hd);
  slab[((size_t)lh * max_seq + p) * hd + d] = gq_normal(seed, gq_kv_index(layer, n_kv, h, p, hd, d));
}

} // namespace

int gq_launch_rmsnorm(const float *x, const float *w, float *out, int dim, float eps, hipStream_t s) {
  return gq_launch_rmsnorm_rows(x, w, out, dim, 1, eps, s);
}

int gq_launch_rmsnorm_rows(const float *x, const float *w, float *out, int dim, int rows, float eps,
                           hipStream_t s, __bf16 *out16, const float *parts, int kparts, float *xnew) {
  if (rows <= 0 || dim <= 0 || (parts && (kparts < 1 || !xnew))) return -1;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, s, x, w, out, dim, eps, out16,
                     parts, kparts, (size_t)rows * dim, xnew);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_embed(int dtype, const void *table, int hidden, const int *token_dev, int token,
                    float *out, hipStream_t s) {
  if (dtype != GQ_F32 && dtype != GQ_Q8_0 && dtype != GQ_Q4_K) return -1;
  hipLaunchKernelGGL(embed_kernel, dim3((hidden + kThreads - 1) / kThreads), dim3(kThreads), 0, s, dtype,
                     (const uint8_t *)table, hidden, token_dev, token, (const int *)nullptr, out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_embed_rows(int dtype, const void *table, int hidden, const int *tokens_dev, int n, float *out,
                         hipStream_t s) {
  if ((dtype != GQ_F32 && dtype != GQ_Q8_0 && dtype != GQ_Q4_K) || !tokens_dev || n <= 0) return -1;
  hipLaunchKernelGGL(embed_kernel, dim3((hidden + kThreads - 1) / kThreads, n), dim3(kThreads), 0, s, dtype,
                     (const uint8_t *)table, hidden, (const int *)nullptr, 0, tokens_dev, out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_argmax_blocks(int n) { return (n + kArgmaxPerBlock - 1) / kArgmaxPerBlock; }

int gq_launch_argmax(const float *x, int n, float *scratch, int nblk, int *out_index, int *tokens,
                     int *step_dev, int *pos_dev, hipStream_t s, int emb_dtype, const void *emb_table, int hidden,
                     float *emb_out) {
  if (n <= 0 || nblk != gq_argmax_blocks(n)) return -1;
  if (emb_out && ((emb_dtype != GQ_F32 && emb_dtype != GQ_Q8_0 && emb_dtype != GQ_Q4_K) || !emb_table ||
                  hidden <= 0))
    return -1;
  hipLaunchKernelGGL(argmax_stage1, dim3(nblk), dim3(kThreads), 0, s, x, n, scratch);
  hipLaunchKernelGGL(argmax_stage2, dim3(emb_out ? (hidden + kThreads - 1) / kThreads : 1), dim3(kThreads), 0, s,
                     scratch, nblk, out_index, tokens, step_dev, pos_dev, emb_dtype, (const uint8_t *)emb_table,
                     hidden, emb_out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_silu_mul(float *gate, const float *up, int n, hipStream_t s) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, s, gate, up, n);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_copy(void *dst, const void *src, size_t bytes, int n_cu, hipStream_t s) {
  if ((bytes & 15) || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15)) return -1;
  const size_t n16 = bytes / 16;
  const size_t blocks = std::min((n16 + kThreads - 1) / kThreads, (size_t)n_cu * 8);
  if (!blocks) return 0;
  hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, (const uint4 *)src, (uint4 *)dst,
                     n16);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_stream_read(const void *src, size_t bytes, uint32_t *sink, size_t sink_n, hipStream_t s) {
  if ((bytes & 15) || ((uintptr_t)src & 15) || !sink) return -1;
  const size_t n16 = bytes / 16;
  /* eight loads per thread, one pass */
  const size_t blocks = (n16 + 8 * kThreads - 1) / (8 * kThreads);
  if (!blocks || !sink_n || blocks > 0x7fffffffu) return blocks ? -1 : 0;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, (const uint4 *)src, n16, sink,
                     (unsigned)std::min<size_t>(sink_n, 0xffffffffu));
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_synth_quant(void *dev, int dtype, int rows, int cols, uint64_t seed, hipStream_t s) {
  int qk, bb;
  if (dtype == GQ_Q4_K || dtype == (GQ_Q4_K | GQ_SYNTH_Q4K_ZERO_MEAN)) qk = 256, bb = 144;
  else if (dtype == GQ_Q6_K) qk = 256, bb = 210;
  else if (dtype == GQ_Q8_0) qk = 32, bb = 34;
  else return -1;
  if (cols % qk) return -2;
  const size_t nbytes = (size_t)rows * (cols / qk) * bb;
  const size_t threads = (nbytes + 3) / 4;
  hipLaunchKernelGGL(synth_quant_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                     (uint8_t *)dev, dtype, nbytes, bb, seed);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_synth_normal(float *dev, size_t n, uint64_t seed, int norm_weight, hipStream_t s) {
  hipLaunchKernelGGL(synth_normal_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dev, n,
                     seed, norm_weight);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int gq_launch_synth_kv(float *slab, int n_layers, int n_kv, int hd, int max_seq, int n_pos,
                       uint64_t seed, hipStream_t s) {
  if (n_pos <= 0) return 0;
  const size_t per = (size_t)n_pos * hd;
  hipLaunchKernelGGL(synth_kv_kernel, dim3((unsigned)((per + 255) / 256), n_layers * n_kv), dim3(256),
                     0, s, slab, n_kv, hd, max_seq, n_pos, seed);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
