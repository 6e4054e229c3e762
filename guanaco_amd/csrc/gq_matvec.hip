/*
 * gq_matvec.hip — K-quant dequant-matvec for gfx950 (wave64, no MFMA).
 *
 * y = W x with W in the reference's block layouts (Q4_K 144 B, Q6_K 210 B,
 * Q8_0 34 B per block; quant_matvec_q4_k.c:9-16, quant_matvec_q6_k.c:5-12,
 * quant_matvec_q8_0.c:5-10), rows = out_features, x fp32.  Batch-1 matvec
 * is HBM-bound, so the design minimises bytes and instructions per byte:
 *
 *  - A 256-thread workgroup stages x (RMS-normalised on the fly when the
 *    launch fuses the preceding RMSNorm) into LDS once, then its 4 waves each
 *    stream R rows.
 *  - Inside a wave, LPB lanes share one super-block: lane `part` owns a fixed
 *    32-weight slice of every block it visits, so each lane keeps its 32 x
 *    values in registers for all R rows and issues one 16-byte load of quants
 *    (plus one 16-byte header load for Q4_K) per row per block.  Consecutive
 *    lanes read consecutive bytes: a wave reads 8 whole blocks per row.
 *  - Scales/mins are decoded in registers; the dot product is factored as
 *    d*sc*sum(q*x) - dmin*m*sum(x) so each weight costs one byte-to-float
 *    convert and one FMA; the per-slice sum(x) is computed once per tile.
 *  - The per-row partial sums are reduced across the wave with DPP row
 *    operations.  Epilogues fuse the residual add (o-proj, down-proj) and
 *    SwiGLU (gate/up pairs).
 *
 * The arithmetic is the reference's formula (w = d*sc*q - dmin*m for Q4_K,
 * d*sc*(q-32) for Q6_K, d*q for Q8_0) with a different summation order; the
 * parity tests hold it to a relative-L2 tolerance against the CPU order.
 */
#include "gq_device.h"
#include "gq_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / GQ_WAVE;

template <int DT>
struct Tr;

/* ---------------------------------------------------------------- Q4_K
 * Lane part p (0..7) of a block reads qs[16p .. 16p+15]: chunk cc = p/2 of
 * 64 weights, half (p&1).  Low nibbles are weights 64cc + 16(p&1) + i of
 * sub-block 2cc, high nibbles weights 64cc + 32 + 16(p&1) + i of sub-block
 * 2cc+1 (quant_matvec_q4_k.c:93-132). */
template <>
struct Tr<GQ_Q4_K> {
  static constexpr int QK = 256, BB = 144, LPB = 8;
  struct Frag {
    uint4 h, q;
  };
  struct X {
    float lo[16], hi[16];
    float slo, shi;
  };
  __device__ static void load_x(X &x, const float *xs, int b, int p) {
    const float *base = xs + 256 * b + 64 * (p >> 1) + 16 * (p & 1);
    const float4 *a = (const float4 *)base, *c = (const float4 *)(base + 32);
    float sl = 0.f, sh = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float4 u = a[k], v = c[k];
      x.lo[4 * k] = u.x, x.lo[4 * k + 1] = u.y, x.lo[4 * k + 2] = u.z, x.lo[4 * k + 3] = u.w;
      x.hi[4 * k] = v.x, x.hi[4 * k + 1] = v.y, x.hi[4 * k + 2] = v.z, x.hi[4 * k + 3] = v.w;
      sl += (u.x + u.y) + (u.z + u.w);
      sh += (v.x + v.y) + (v.z + v.w);
    }
    x.slo = sl;
    x.shi = sh;
  }
  __device__ static void load(Frag &f, const uint8_t *row, int b, int p) {
    const uint8_t *blk = row + (size_t)b * BB;
    f.h = *(const uint4 *)blk;
    f.q = *(const uint4 *)(blk + 16 + 16 * p);
  }
  __device__ static float dot(const Frag &f, const X &x, int p) {
    const float d = gq_h2f(f.h.x), dm = gq_h2f(f.h.x >> 16);
    /* 6-bit (scale, min) of sub-blocks j = 2cc, 2cc+1 (quant_matvec_q4_k.c:47-56) */
    const int cc = p >> 1;
    const int sh = 16 * (cc & 1);
    const uint32_t y = f.h.y >> sh, z = f.h.z >> sh, w = f.h.w >> sh;
    uint32_t s0, m0, s1, m1;
    if (cc < 2) {
      s0 = y & 63u, m0 = z & 63u;
      s1 = (y >> 8) & 63u, m1 = (z >> 8) & 63u;
    } else {
      s0 = (w & 15u) | (((y >> 6) & 3u) << 4), m0 = ((w >> 4) & 15u) | (((z >> 6) & 3u) << 4);
      s1 = ((w >> 8) & 15u) | (((y >> 14) & 3u) << 4);
      m1 = ((w >> 12) & 15u) | (((z >> 14) & 3u) << 4);
    }
    const uint32_t qw[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
    float al = 0.f, ah = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t lo = qw[k] & 0x0f0f0f0fu, hi = (qw[k] >> 4) & 0x0f0f0f0fu;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        al = __builtin_fmaf((float)gq_byte(lo, j), x.lo[4 * k + j], al);
        ah = __builtin_fmaf((float)gq_byte(hi, j), x.hi[4 * k + j], ah);
      }
    }
    float r = (d * (float)s0) * al;
    r = __builtin_fmaf(-(dm * (float)m0), x.slo, r);
    r = __builtin_fmaf(d * (float)s1, ah, r);
    r = __builtin_fmaf(-(dm * (float)m1), x.shi, r);
    return r;
  }
};

/* Eight bytes at a 2-byte-aligned address inside a block, read through a
 * dword window that starts 2 or 4 bytes early (never past addr + 10). */
__device__ __forceinline__ uint2 load8_back(const uint8_t *p) {
  const uintptr_t a = (uintptr_t)p;
  const uintptr_t base = (a - 2) & ~(uintptr_t)3;
  const gq_u32x3 w = *(const gq_u32x3 *)base;
  uint2 r;
  if (a - base == 4) {
    r.x = w.y, r.y = w.z;
  } else {
    r.x = __builtin_amdgcn_alignbyte(w.y, w.x, 2);
    r.y = __builtin_amdgcn_alignbyte(w.z, w.y, 2);
  }
  return r;
}

/* ---------------------------------------------------------------- Q6_K
 * Lane part p (0..7): half h = p/4 of the block, l in [8(p&3), 8(p&3)+8).
 * Runs of 8 weights at 128h + {0,32,64,96} + l use ql[l], ql[l+32] low and
 * high nibbles and the four 2-bit fields of qh[l], with scales
 * sc[8h + s + {0,2,4,6}], s = (p&3)/2 (quant_matvec_q6_k.c:75-92). */
template <>
struct Tr<GQ_Q6_K> {
  static constexpr int QK = 256, BB = 210, LPB = 8;
  struct Frag {
    uint2 a, b, h, s;
    uint32_t d;
  };
  struct X {
    float v[4][8];
    float s[4];
  };
  __device__ static void load_x(X &x, const float *xs, int b, int p) {
    const float *base = xs + 256 * b + 128 * (p >> 2) + 8 * (p & 3);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float4 u = *(const float4 *)(base + 32 * r), v = *(const float4 *)(base + 32 * r + 4);
      x.v[r][0] = u.x, x.v[r][1] = u.y, x.v[r][2] = u.z, x.v[r][3] = u.w;
      x.v[r][4] = v.x, x.v[r][5] = v.y, x.v[r][6] = v.z, x.v[r][7] = v.w;
      x.s[r] = ((u.x + u.y) + (u.z + u.w)) + ((v.x + v.y) + (v.z + v.w));
    }
  }
  __device__ static void load(Frag &f, const uint8_t *row, int b, int p) {
    const uint8_t *blk = row + (size_t)b * BB;
    const int h = p >> 2, l0 = 8 * (p & 3);
    f.a = gq_load8_a2(blk + 64 * h + l0);
    f.b = gq_load8_a2(blk + 64 * h + 32 + l0);
    f.h = gq_load8_a2(blk + 128 + 32 * h + l0);
    f.s = load8_back(blk + 192 + 8 * h);
    f.d = *(const uint16_t *)(blk + 208);
  }
  __device__ static float dot(const Frag &f, const X &x, int p) {
    const int s = (p & 3) >> 1;
    const float sc0 = (float)(int8_t)(f.s.x >> (8 * s));
    const float sc1 = (float)(int8_t)(f.s.x >> (8 * s + 16));
    const float sc2 = (float)(int8_t)(f.s.y >> (8 * s));
    const float sc3 = (float)(int8_t)(f.s.y >> (8 * s + 16));
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const uint32_t A[2] = {f.a.x, f.a.y}, B[2] = {f.b.x, f.b.y}, H[2] = {f.h.x, f.h.y};
#pragma unroll
    for (int k = 0; k < 2; k++) {
      uint32_t u[4];
      u[0] = (A[k] & 0x0f0f0f0fu) | ((H[k] & 0x03030303u) << 4);
      u[1] = (B[k] & 0x0f0f0f0fu) | (((H[k] >> 2) & 0x03030303u) << 4);
      u[2] = ((A[k] >> 4) & 0x0f0f0f0fu) | (((H[k] >> 4) & 0x03030303u) << 4);
      u[3] = ((B[k] >> 4) & 0x0f0f0f0fu) | (((H[k] >> 6) & 0x03030303u) << 4);
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[r] = __builtin_fmaf((float)gq_byte(u[r], j), x.v[r][4 * k + j], acc[r]);
    }
    /* sum (u - 32) x = sum u x - 32 sum x */
    float t = sc0 * __builtin_fmaf(-32.f, x.s[0], acc[0]);
    t = __builtin_fmaf(sc1, __builtin_fmaf(-32.f, x.s[1], acc[1]), t);
    t = __builtin_fmaf(sc2, __builtin_fmaf(-32.f, x.s[2], acc[2]), t);
    t = __builtin_fmaf(sc3, __builtin_fmaf(-32.f, x.s[3], acc[3]), t);
    return gq_h2f(f.d) * t;
  }
};

/* ---------------------------------------------------------------- Q8_0
 * One lane per 34-byte block (32 int8 weights, fp16 scale). */
template <>
struct Tr<GQ_Q8_0> {
  static constexpr int QK = 32, BB = 34, LPB = 1;
  struct Frag {
    uint32_t q[8];
    uint32_t d;
  };
  struct X {
    float v[32];
  };
  __device__ static void load_x(X &x, const float *xs, int b, int p) {
    (void)p;
    const float4 *base = (const float4 *)(xs + 32 * b);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float4 u = base[k];
      x.v[4 * k] = u.x, x.v[4 * k + 1] = u.y, x.v[4 * k + 2] = u.z, x.v[4 * k + 3] = u.w;
    }
  }
  __device__ static void load(Frag &f, const uint8_t *row, int b, int p) {
    (void)p;
    const uint8_t *blk = row + (size_t)b * BB;
    f.d = *(const uint16_t *)blk;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint2 v = gq_load8_a2(blk + 2 + 8 * k);
      f.q[2 * k] = v.x, f.q[2 * k + 1] = v.y;
    }
  }
  __device__ static float dot(const Frag &f, const X &x, int p) {
    (void)p;
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc = __builtin_fmaf((float)(int8_t)(f.q[k] >> (8 * j)), x.v[4 * k + j], acc);
    return acc * gq_h2f(f.d);
  }
};

/* Stage x (optionally RMS-normalised: w * (x * 1/sqrt(mean(x^2) + eps)),
 * kernels_cpu.c:242-253) into LDS. */
__device__ __forceinline__ void stage_x(const MvArgs &a, float *xs) {
  __shared__ float red[kWaves];
  const int tid = threadIdx.x, n4 = a.cols >> 2;
  const float4 *x4 = (const float4 *)a.x;
  float4 *s4 = (float4 *)xs;
  if (a.norm_w) {
    float ss = 0.f;
    for (int i = tid; i < n4; i += kThreads) {
      const float4 v = x4[i];
      ss = __builtin_fmaf(v.x, v.x, ss);
      ss = __builtin_fmaf(v.y, v.y, ss);
      ss = __builtin_fmaf(v.z, v.z, ss);
      ss = __builtin_fmaf(v.w, v.w, ss);
    }
    ss = gq_wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = (red[0] + red[1]) + (red[2] + red[3]);
    tot = tot / (float)a.cols;
    tot = tot + a.eps;
    const float r = 1.0f / sqrtf(tot);
    const float4 *w4 = (const float4 *)a.norm_w;
    for (int i = tid; i < n4; i += kThreads) {
      const float4 v = x4[i], w = w4[i];
      s4[i] = make_float4(w.x * (v.x * r), w.y * (v.y * r), w.z * (v.z * r), w.w * (v.w * r));
    }
  } else {
    for (int i = tid; i < n4; i += kThreads) s4[i] = x4[i];
  }
  __syncthreads();
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  /* silu(g) * u with silu(g) = g * (1 / (1 + expf(-g))) (kernels_cpu.c:322-336) */
  const float sig = 1.0f / (1.0f + expf(0.0f - g));
  return (g * sig) * u;
}

template <int DT, int R, int MODE>
__global__ __launch_bounds__(kThreads) void mv_kernel(MvArgs a) {
  using T = Tr<DT>;
  extern __shared__ float xs[];
  stage_x(a, xs);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb = a.cols / T::QK;
  const size_t rowbytes = (size_t)nb * T::BB;
  constexpr int BPT = GQ_WAVE / T::LPB;
  const int ntile = (nb + BPT - 1) / BPT;
  const int part = lane % T::LPB, bt = lane / T::LPB;

  /* rows handled by this wave */
  const uint8_t *rp[R];
  float *yp[R];
  const float *rr[R];
  bool ok[R];
  if (MODE == MV_SWIGLU) {
    constexpr int P = R / 2;
    const int p0 = (blockIdx.x * kWaves + wave) * P;
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int pr = p0 + i;
      ok[i] = ok[P + i] = pr < a.seg[0].rows;
      const int rr0 = ok[i] ? pr : 0;
      rp[i] = a.seg[0].w + rr0 * rowbytes;
      rp[P + i] = a.seg[1].w + rr0 * rowbytes;
      yp[i] = a.seg[0].y + rr0;
      yp[P + i] = nullptr;
      rr[i] = rr[P + i] = nullptr;
    }
  } else {
    const int r0 = (blockIdx.x * kWaves + wave) * R;
#pragma unroll
    for (int i = 0; i < R; i++) {
      int g = r0 + i, s = 0;
      while (s < a.nseg - 1 && g >= a.seg[s].rows) g -= a.seg[s++].rows;
      ok[i] = g < a.seg[s].rows;
      if (!ok[i]) s = 0, g = 0;
      rp[i] = a.seg[s].w + g * rowbytes;
      yp[i] = a.seg[s].y + g;
      rr[i] = MODE == MV_RESID ? a.seg[s].r + g : nullptr;
    }
  }

  float acc[R];
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = 0.f;
  for (int t = 0; t < ntile; t++) {
    const int b = t * BPT + bt;
    const bool bok = b < nb;
    const int bc = bok ? b : nb - 1;
    typename T::Frag f[R];
#pragma unroll
    for (int i = 0; i < R; i++) T::load(f[i], rp[i], bc, part);
    typename T::X x;
    T::load_x(x, xs, bc, part);
#pragma unroll
    for (int i = 0; i < R; i++) {
      const float v = T::dot(f[i], x, part);
      acc[i] += bok ? v : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = gq_wave_sum(acc[i]);

  if (MODE == MV_SWIGLU) {
    constexpr int P = R / 2;
#pragma unroll
    for (int i = 0; i < P; i++)
      if (lane == i && ok[i]) *yp[i] = silu_mul(acc[i], acc[P + i]);
  } else {
#pragma unroll
    for (int i = 0; i < R; i++) {
      if (lane == i && ok[i]) {
        if (MODE == MV_RESID)
          *yp[i] = acc[i] + *rr[i];
        else
          *yp[i] = acc[i];
      }
    }
  }
}

template <int DT, int MODE>
int launch_dm(const MvArgs &a, hipStream_t s) {
  constexpr int R = 4;
  int rows;
  if (MODE == MV_SWIGLU) {
    if (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows) return -1;
    rows = a.seg[0].rows;
  } else {
    rows = 0;
    for (int i = 0; i < a.nseg; i++) rows += a.seg[i].rows;
  }
  const int per_wg = kWaves * (MODE == MV_SWIGLU ? R / 2 : R);
  const int grid = (rows + per_wg - 1) / per_wg;
  if (grid <= 0) return -1;
  const size_t lds = (size_t)a.cols * sizeof(float);
  hipLaunchKernelGGL((mv_kernel<DT, R, MODE>), dim3(grid), dim3(kThreads), lds, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <int DT>
int launch_dt(int mode, const MvArgs &a, hipStream_t s) {
  switch (mode) {
  case MV_STORE: return launch_dm<DT, MV_STORE>(a, s);
  case MV_RESID: return launch_dm<DT, MV_RESID>(a, s);
  case MV_SWIGLU: return launch_dm<DT, MV_SWIGLU>(a, s);
  default: return -1;
  }
}

} // namespace

int gq_launch_matvec(int dtype, int mode, const MvArgs &a, hipStream_t s) {
  if (a.nseg < 1 || a.nseg > 3 || a.cols <= 0 || a.cols > 16384 || (a.cols & 3)) return -1;
  switch (dtype) {
  case GQ_Q4_K: return a.cols % 256 ? -2 : launch_dt<GQ_Q4_K>(mode, a, s);
  case GQ_Q6_K: return a.cols % 256 ? -2 : launch_dt<GQ_Q6_K>(mode, a, s);
  case GQ_Q8_0: return a.cols % 32 ? -2 : launch_dt<GQ_Q8_0>(mode, a, s);
  default: return -1;
  }
}
