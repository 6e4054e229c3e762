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
#include <stdlib.h>

#include <algorithm>

#include "gq_device.h"
#include "gq_internal.h"

namespace {

constexpr int kThreads = 256;

/* x staged in LDS by the split-K kernel has its 16-byte units permuted
 * inside each 256-byte row: unit u sits at (u & ~15) | ((u ^ (u >> 4)) & 15),
 * an involution.  The traits' lanes read the same unit of different rows at
 * once (a 4-lane Q4_K wave reads 64 units 256 bytes apart), which the
 * permutation spreads over all the banks. */
__device__ __forceinline__ uint32_t xswz(uint32_t byteoff) {
  const uint32_t u = byteoff >> 4;
  return ((u & ~15u) | ((u ^ (u >> 4)) & 15u)) << 4;
}
template <bool SW>
__device__ __forceinline__ float4 lldx(const GQ_LDS uint8_t *p, uint32_t off) {
  return lld<float4>(p, SW ? xswz(off) : off);
}
constexpr int kWaves = kThreads / GQ_WAVE;

template <int DT>
struct Tr;

/* ---------------------------------------------------------------- Q4_K
 * Lane part p (0..3) of a block owns chunk p of 64 weights: it reads
 * qs[32p .. 32p+31], whose low nibbles are weights 64p + i of sub-block 2p
 * and high nibbles weights 64p + 32 + i of sub-block 2p+1, i = 0..31
 * (quant_matvec_q4_k.c:93-132). */
template <>
struct Tr<GQ_Q4_K> {
  static constexpr int QK = 256, BB = 144, LPB = 4;
  struct Frag {
    uint4 h, q0, q1;
  };
  struct X {
    float lo[32], hi[32];
    float slo, shi;
  };
  /* x slice of block b from x staged in LDS (byte base xs), times the
   * RMSNorm weight staged at nw when given; *ss (when given) accumulates the
   * raw x^2 of the slice */
  template <bool SW = false>
  __device__ static void load_x(X &x, const GQ_LDS uint8_t *xs, const GQ_LDS uint8_t *nw, int b, int p,
                                float *ss = nullptr) {
    const uint32_t a = 4u * (256 * b + 64 * p), c = a + 128;
    float sl = 0.f, sh = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float4 u = lldx<SW>(xs, a + 16 * k), v = lldx<SW>(xs, c + 16 * k);
      if (ss) {
        float q = *ss;
        q = __builtin_fmaf(u.x, u.x, q), q = __builtin_fmaf(u.y, u.y, q), q = __builtin_fmaf(u.z, u.z, q);
        q = __builtin_fmaf(u.w, u.w, q), q = __builtin_fmaf(v.x, v.x, q), q = __builtin_fmaf(v.y, v.y, q);
        q = __builtin_fmaf(v.z, v.z, q), q = __builtin_fmaf(v.w, v.w, q);
        *ss = q;
      }
      if (nw) {
        const float4 wu = lldx<SW>(nw, a + 16 * k), wv = lldx<SW>(nw, c + 16 * k);
        u = make_float4(wu.x * u.x, wu.y * u.y, wu.z * u.z, wu.w * u.w);
        v = make_float4(wv.x * v.x, wv.y * v.y, wv.z * v.z, wv.w * v.w);
      }
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
    f.h = gld<uint4>(blk);
    f.q0 = gld<uint4>(blk + 16 + 32 * p);
    f.q1 = gld<uint4>(blk + 32 + 32 * p);
  }
  __device__ static void load_lds(Frag &f, const GQ_LDS uint8_t *base, uint32_t blk, int p) {
    f.h = lld<uint4>(base, blk);
    f.q0 = lld<uint4>(base, blk + 16 + 32 * p);
    f.q1 = lld<uint4>(base, blk + 32 + 32 * p);
  }
  __device__ static float dot(const Frag &f, const X &x, int p) {
    const float d = gq_h2f(f.h.x), dm = gq_h2f(f.h.x >> 16);
    /* 6-bit (scale, min) of sub-blocks j = 2p, 2p+1 (quant_matvec_q4_k.c:47-56):
     * j < 4:  sc = s[j] & 63,  m = s[j+4] & 63
     * j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4,
     *         m  = (s[j+4] >> 4) | (s[j] >> 6) << 4
     * with s[0..3] = h.y, s[4..7] = h.z, s[8..11] = h.w; both sub-blocks at
     * once in bytes 0 and 1 of S and M, without branching on p */
    const uint32_t sh = 16u * (uint32_t)(p & 1);
    const bool hi = p >= 2;
    const uint32_t y = f.h.y >> sh, z = f.h.z >> sh, w = f.h.w >> sh;
    const uint32_t mlo = hi ? 0x0f0fu : 0x3f3fu, mhi = hi ? 0x3030u : 0u;
    const uint32_t S = ((hi ? w : y) & mlo) | ((y >> 2) & mhi);
    const uint32_t M = ((hi ? (w >> 4) : z) & mlo) | ((z >> 2) & mhi);
    const uint32_t qw[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
    /* al, ah: 2^-9 * sum q x over the chunk's two sub-blocks (q converted as
     * fp8, see gq_nib2f) */
    float al = 0.f, ah = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t lo = qw[k] & 0x0f0f0f0fu, hq = (qw[k] >> 4) & 0x0f0f0f0fu;
      const gq_f32x2 l01 = gq_nib2f<false>(lo), l23 = gq_nib2f<true>(lo);
      const gq_f32x2 h01 = gq_nib2f<false>(hq), h23 = gq_nib2f<true>(hq);
      al = __builtin_fmaf(l01.x, x.lo[4 * k], al);
      ah = __builtin_fmaf(h01.x, x.hi[4 * k], ah);
      al = __builtin_fmaf(l01.y, x.lo[4 * k + 1], al);
      ah = __builtin_fmaf(h01.y, x.hi[4 * k + 1], ah);
      al = __builtin_fmaf(l23.x, x.lo[4 * k + 2], al);
      ah = __builtin_fmaf(h23.x, x.hi[4 * k + 2], ah);
      al = __builtin_fmaf(l23.y, x.lo[4 * k + 3], al);
      ah = __builtin_fmaf(h23.y, x.hi[4 * k + 3], ah);
    }
    /* (d 2^9 sc)(2^-9 sum q x): power-of-two rescalings are exact, so this
     * rounds as (d sc)(sum q x) */
    const float d9 = d * 512.f;
    float r = (d9 * (float)(S & 0xffu)) * al;
    r = __builtin_fmaf(-(dm * (float)(M & 0xffu)), x.slo, r);
    r = __builtin_fmaf(d9 * (float)((S >> 8) & 0xffu), ah, r);
    r = __builtin_fmaf(-(dm * (float)((M >> 8) & 0xffu)), x.shi, r);
    return r;
  }
};

/* Q4_K with 8 lanes per block, for the kernels that split a row's columns
 * over the waves of a workgroup (a wave covers 8 blocks per column tile).
 * Lane part p (0..7) reads qs[16p .. 16p+15]: chunk cc = p/2 of 64 weights,
 * half (p&1).  Low nibbles are weights 64cc + 16(p&1) + i of sub-block 2cc,
 * high nibbles weights 64cc + 32 + 16(p&1) + i of sub-block 2cc+1
 * (quant_matvec_q4_k.c:93-132). */
struct TrQ4K8 {
  static constexpr int QK = 256, BB = 144, LPB = 8;
  struct Frag {
    uint4 h, q;
  };
  struct X {
    float lo[16], hi[16];
    float slo, shi;
  };
  __device__ static void fill(X &x, float4 (&u)[4], float4 (&v)[4]) {
    float sl = 0.f, sh = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      x.lo[4 * k] = u[k].x, x.lo[4 * k + 1] = u[k].y, x.lo[4 * k + 2] = u[k].z, x.lo[4 * k + 3] = u[k].w;
      x.hi[4 * k] = v[k].x, x.hi[4 * k + 1] = v[k].y, x.hi[4 * k + 2] = v[k].z, x.hi[4 * k + 3] = v[k].w;
      sl += (u[k].x + u[k].y) + (u[k].z + u[k].w);
      sh += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    x.slo = sl;
    x.shi = sh;
  }
  template <bool SW = false>
  __device__ static void load_x(X &x, const GQ_LDS uint8_t *xs, const GQ_LDS uint8_t *nw, int b, int p,
                                float *ss = nullptr) {
    const uint32_t a = 4u * (256 * b + 64 * (p >> 1) + 16 * (p & 1));
    float4 u[4], v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      u[k] = lldx<SW>(xs, a + 16 * k), v[k] = lldx<SW>(xs, a + 128 + 16 * k);
      if (ss) {
        float q = *ss;
        q = __builtin_fmaf(u[k].x, u[k].x, q), q = __builtin_fmaf(u[k].y, u[k].y, q);
        q = __builtin_fmaf(u[k].z, u[k].z, q), q = __builtin_fmaf(u[k].w, u[k].w, q);
        q = __builtin_fmaf(v[k].x, v[k].x, q), q = __builtin_fmaf(v[k].y, v[k].y, q);
        q = __builtin_fmaf(v[k].z, v[k].z, q), q = __builtin_fmaf(v[k].w, v[k].w, q);
        *ss = q;
      }
      if (nw) {
        const float4 wu = lldx<SW>(nw, a + 16 * k), wv = lldx<SW>(nw, a + 128 + 16 * k);
        u[k] = make_float4(wu.x * u[k].x, wu.y * u[k].y, wu.z * u[k].z, wu.w * u[k].w);
        v[k] = make_float4(wv.x * v[k].x, wv.y * v[k].y, wv.z * v[k].z, wv.w * v[k].w);
      }
    }
    fill(x, u, v);
  }
  /* x slice straight from global memory, times the RMSNorm weight when given;
   * ss accumulates the raw x^2 of the slice */
  __device__ static void load_xg(X &x, const float *xg, const float *nw, int b, int p, float &ss) {
    const int base = 256 * b + 64 * (p >> 1) + 16 * (p & 1);
    /* every load first (the norm weight, or x again in its place), so the
     * slice costs one memory round trip */
    const float *np = nw ? nw : xg;
    float4 u[4], v[4], wu[4], wv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      u[k] = gld<float4>(xg + base + 4 * k), v[k] = gld<float4>(xg + base + 32 + 4 * k);
      wu[k] = gld<float4>(np + base + 4 * k), wv[k] = gld<float4>(np + base + 32 + 4 * k);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      ss = __builtin_fmaf(u[k].x, u[k].x, ss), ss = __builtin_fmaf(u[k].y, u[k].y, ss);
      ss = __builtin_fmaf(u[k].z, u[k].z, ss), ss = __builtin_fmaf(u[k].w, u[k].w, ss);
      ss = __builtin_fmaf(v[k].x, v[k].x, ss), ss = __builtin_fmaf(v[k].y, v[k].y, ss);
      ss = __builtin_fmaf(v[k].z, v[k].z, ss), ss = __builtin_fmaf(v[k].w, v[k].w, ss);
      if (nw) {
        u[k] = make_float4(wu[k].x * u[k].x, wu[k].y * u[k].y, wu[k].z * u[k].z, wu[k].w * u[k].w);
        v[k] = make_float4(wv[k].x * v[k].x, wv[k].y * v[k].y, wv[k].z * v[k].z, wv[k].w * v[k].w);
      }
    }
    fill(x, u, v);
  }
  __device__ static void load(Frag &f, const uint8_t *row, int b, int p) {
    const uint8_t *blk = row + (size_t)b * BB;
    f.h = gld<uint4>(blk);
    f.q = gld<uint4>(blk + 16 + 16 * p);
  }
  __device__ static void load_lds(Frag &f, const GQ_LDS uint8_t *base, uint32_t blk, int p) {
    f.h = lld<uint4>(base, blk);
    f.q = lld<uint4>(base, blk + 16 + 16 * p);
  }
  __device__ static float dot(const Frag &f, const X &x, int p) {
    const float d = gq_h2f(f.h.x), dm = gq_h2f(f.h.x >> 16);
    /* (scale, min) of sub-blocks 2cc, 2cc+1 decoded as in Tr<GQ_Q4_K>::dot */
    const int cc = p >> 1;
    const uint32_t sh = 16u * (uint32_t)(cc & 1);
    const bool hi = cc >= 2;
    const uint32_t y = f.h.y >> sh, z = f.h.z >> sh, w = f.h.w >> sh;
    const uint32_t mlo = hi ? 0x0f0fu : 0x3f3fu, mhi = hi ? 0x3030u : 0u;
    const uint32_t S = ((hi ? w : y) & mlo) | ((y >> 2) & mhi);
    const uint32_t M = ((hi ? (w >> 4) : z) & mlo) | ((z >> 2) & mhi);
    const uint32_t qw[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
    float al = 0.f, ah = 0.f; /* 2^-9 sum q x (gq_nib2f) */
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t lo = qw[k] & 0x0f0f0f0fu, hq = (qw[k] >> 4) & 0x0f0f0f0fu;
      const gq_f32x2 l01 = gq_nib2f<false>(lo), l23 = gq_nib2f<true>(lo);
      const gq_f32x2 h01 = gq_nib2f<false>(hq), h23 = gq_nib2f<true>(hq);
      al = __builtin_fmaf(l01.x, x.lo[4 * k], al);
      ah = __builtin_fmaf(h01.x, x.hi[4 * k], ah);
      al = __builtin_fmaf(l01.y, x.lo[4 * k + 1], al);
      ah = __builtin_fmaf(h01.y, x.hi[4 * k + 1], ah);
      al = __builtin_fmaf(l23.x, x.lo[4 * k + 2], al);
      ah = __builtin_fmaf(h23.x, x.hi[4 * k + 2], ah);
      al = __builtin_fmaf(l23.y, x.lo[4 * k + 3], al);
      ah = __builtin_fmaf(h23.y, x.hi[4 * k + 3], ah);
    }
    const float d9 = d * 512.f;
    float r = (d9 * (float)(S & 0xffu)) * al;
    r = __builtin_fmaf(-(dm * (float)(M & 0xffu)), x.slo, r);
    r = __builtin_fmaf(d9 * (float)((S >> 8) & 0xffu), ah, r);
    r = __builtin_fmaf(-(dm * (float)((M >> 8) & 0xffu)), x.shi, r);
    return r;
  }
};

/* Eight bytes at a 2-byte-aligned address inside a block, read through a
 * dword window that starts 2 or 4 bytes early (never past addr + 10). */
__device__ __forceinline__ uint2 load8_back(const uint8_t *p) {
  const uintptr_t a = (uintptr_t)p;
  const uintptr_t base = (a - 2) & ~(uintptr_t)3;
  const uint3 w = gld12((const void *)base);
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
  template <bool SW = false>
  __device__ static void load_x(X &x, const GQ_LDS uint8_t *xs, const GQ_LDS uint8_t *nw, int b, int p,
                                float *ss = nullptr) {
    const uint32_t base = 4u * (256 * b + 128 * (p >> 2) + 8 * (p & 3));
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float4 u = lldx<SW>(xs, base + 128 * r), v = lldx<SW>(xs, base + 128 * r + 16);
      if (ss) {
        float q = *ss;
        q = __builtin_fmaf(u.x, u.x, q), q = __builtin_fmaf(u.y, u.y, q), q = __builtin_fmaf(u.z, u.z, q);
        q = __builtin_fmaf(u.w, u.w, q), q = __builtin_fmaf(v.x, v.x, q), q = __builtin_fmaf(v.y, v.y, q);
        q = __builtin_fmaf(v.z, v.z, q), q = __builtin_fmaf(v.w, v.w, q);
        *ss = q;
      }
      if (nw) {
        const float4 wu = lldx<SW>(nw, base + 128 * r), wv = lldx<SW>(nw, base + 128 * r + 16);
        u = make_float4(wu.x * u.x, wu.y * u.y, wu.z * u.z, wu.w * u.w);
        v = make_float4(wv.x * v.x, wv.y * v.y, wv.z * v.z, wv.w * v.w);
      }
      x.v[r][0] = u.x, x.v[r][1] = u.y, x.v[r][2] = u.z, x.v[r][3] = u.w;
      x.v[r][4] = v.x, x.v[r][5] = v.y, x.v[r][6] = v.z, x.v[r][7] = v.w;
      x.s[r] = ((u.x + u.y) + (u.z + u.w)) + ((v.x + v.y) + (v.z + v.w));
    }
  }
  __device__ static void load_xg(X &x, const float *xg, const float *nw, int b, int p, float &ss) {
    const int base = 256 * b + 128 * (p >> 2) + 8 * (p & 3);
    /* every load first (one memory round trip), as in TrQ4K8::load_xg */
    const float *np = nw ? nw : xg;
    float4 uu[4], vv[4], wu[4], wv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      uu[r] = gld<float4>(xg + base + 32 * r), vv[r] = gld<float4>(xg + base + 32 * r + 4);
      wu[r] = gld<float4>(np + base + 32 * r), wv[r] = gld<float4>(np + base + 32 * r + 4);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float4 u = uu[r], v = vv[r];
      ss = __builtin_fmaf(u.x, u.x, ss), ss = __builtin_fmaf(u.y, u.y, ss);
      ss = __builtin_fmaf(u.z, u.z, ss), ss = __builtin_fmaf(u.w, u.w, ss);
      ss = __builtin_fmaf(v.x, v.x, ss), ss = __builtin_fmaf(v.y, v.y, ss);
      ss = __builtin_fmaf(v.z, v.z, ss), ss = __builtin_fmaf(v.w, v.w, ss);
      if (nw) {
        u = make_float4(wu[r].x * u.x, wu[r].y * u.y, wu[r].z * u.z, wu[r].w * u.w);
        v = make_float4(wv[r].x * v.x, wv[r].y * v.y, wv[r].z * v.z, wv[r].w * v.w);
      }
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
    f.d = gld<uint16_t>(blk + 208);
  }
  __device__ static void load_lds(Frag &f, const GQ_LDS uint8_t *base, uint32_t blk, int p) {
    const int h = p >> 2, l0 = 8 * (p & 3);
    f.a = lld8_a2(base, blk + 64 * h + l0);
    f.b = lld8_a2(base, blk + 64 * h + 32 + l0);
    f.h = lld8_a2(base, blk + 128 + 32 * h + l0);
    f.s = lld8_a2(base, blk + 192 + 8 * h);
    f.d = lld<uint16_t>(base, blk + 208);
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
  template <bool SW = false>
  __device__ static void load_x(X &x, const GQ_LDS uint8_t *xs, const GQ_LDS uint8_t *nw, int b, int p,
                                float *ss = nullptr) {
    (void)p;
    const uint32_t base = 128u * b;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float4 u = lldx<SW>(xs, base + 16 * k);
      if (ss) {
        float q = *ss;
        q = __builtin_fmaf(u.x, u.x, q), q = __builtin_fmaf(u.y, u.y, q);
        q = __builtin_fmaf(u.z, u.z, q), q = __builtin_fmaf(u.w, u.w, q);
        *ss = q;
      }
      if (nw) {
        const float4 w = lldx<SW>(nw, base + 16 * k);
        u = make_float4(w.x * u.x, w.y * u.y, w.z * u.z, w.w * u.w);
      }
      x.v[4 * k] = u.x, x.v[4 * k + 1] = u.y, x.v[4 * k + 2] = u.z, x.v[4 * k + 3] = u.w;
    }
  }
  __device__ static void load_xg(X &x, const float *xg, const float *nw, int b, int p, float &ss) {
    (void)p;
    /* every load first (one memory round trip), as in TrQ4K8::load_xg */
    const float *np = nw ? nw : xg;
    float4 uu[8], ww[8];
#pragma unroll
    for (int k = 0; k < 8; k++) uu[k] = gld<float4>(xg + 32 * b + 4 * k), ww[k] = gld<float4>(np + 32 * b + 4 * k);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float4 u = uu[k];
      ss = __builtin_fmaf(u.x, u.x, ss), ss = __builtin_fmaf(u.y, u.y, ss);
      ss = __builtin_fmaf(u.z, u.z, ss), ss = __builtin_fmaf(u.w, u.w, ss);
      if (nw) {
        const float4 w = ww[k];
        u = make_float4(w.x * u.x, w.y * u.y, w.z * u.z, w.w * u.w);
      }
      x.v[4 * k] = u.x, x.v[4 * k + 1] = u.y, x.v[4 * k + 2] = u.z, x.v[4 * k + 3] = u.w;
    }
  }
  __device__ static void load(Frag &f, const uint8_t *row, int b, int p) {
    (void)p;
    const uint8_t *blk = row + (size_t)b * BB;
    f.d = gld<uint16_t>(blk);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint2 v = gq_load8_a2(blk + 2 + 8 * k);
      f.q[2 * k] = v.x, f.q[2 * k + 1] = v.y;
    }
  }
  __device__ static void load_lds(Frag &f, const GQ_LDS uint8_t *base, uint32_t blk, int p) {
    (void)p;
    f.d = lld<uint16_t>(base, blk);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint2 v = lld8_a2(base, blk + 2 + 8 * k);
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

/* Traits of the kernels that split a row's columns over the waves of a
 * workgroup (the split-K LDS kernel and the register-path kernel): Q4_K with
 * 8 lanes per block there, 4 in the whole-row kernels. */
template <int DT>
struct TrSplit {
  using type = Tr<DT>;
};
template <>
struct TrSplit<GQ_Q4_K> {
  using type = TrQ4K8;
};

/* The split-K LDS kernel's traits: with x staged in LDS (XL) a Q4_K lane
 * takes a 64-weight chunk of each block (4 lanes per block: half the
 * per-weight cost of decoding scales and reducing, but x slices twice as
 * long, which only pays when they come from LDS); otherwise as TrSplit. */
template <int DT, bool XL>
struct TrL {
  using type = typename TrSplit<DT>::type;
};
template <>
struct TrL<GQ_Q4_K, true> {
  using type = Tr<GQ_Q4_K>;
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
      const float4 v = gld<float4>(x4 + i);
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
      const float4 v = gld<float4>(x4 + i), w = gld<float4>(w4 + i);
      s4[i] = make_float4(w.x * (v.x * r), w.y * (v.y * r), w.z * (v.z * r), w.w * (v.w * r));
    }
  } else {
    for (int i = tid; i < n4; i += kThreads) s4[i] = gld<float4>(x4 + i);
  }
  __syncthreads();
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  /* silu(g) * u with silu(g) = g * (1 / (1 + expf(-g))) (kernels_cpu.c:322-336) */
  const float sig = 1.0f / (1.0f + expf(0.0f - g));
  return (g * sig) * u;
}

/* Segment and local row of global output row gr. */
__device__ __forceinline__ void locate(const MvArgs &a, int gr, int &s, int &lr) {
  s = 0;
  lr = gr;
  while (s < a.nseg - 1 && lr >= a.seg[s].rows) lr -= a.seg[s++].rows;
}

__device__ __forceinline__ int total_rows(const MvArgs &a, int mode) {
  if (mode == MV_SWIGLU) return a.seg[0].rows;
  int t = 0;
  for (int i = 0; i < a.nseg; i++) t += a.seg[i].rows;
  return t;
}

/* Weight row pointers of the R rows a wave computes in row group g (rows past
 * the end are clamped to the last row: loaded, never stored). */
template <int R, int MODE>
__device__ __forceinline__ void group_rows(const MvArgs &a, int total, int g, int wave, size_t rowbytes,
                                           const uint8_t *rp[R]) {
  if (MODE == MV_SWIGLU) {
    constexpr int P = R / 2;
    const int p0 = (g * kWaves + wave) * P;
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int pr = min(p0 + i, total - 1);
      rp[i] = a.seg[0].w + pr * rowbytes;
      rp[P + i] = a.seg[1].w + pr * rowbytes;
    }
  } else {
    const int r0 = (g * kWaves + wave) * R;
#pragma unroll
    for (int i = 0; i < R; i++) {
      int s, lr;
      locate(a, min(r0 + i, total - 1), s, lr);
      rp[i] = a.seg[s].w + lr * rowbytes;
    }
  }
}

/* Store the R reduced row values of group g (every lane holds all of them;
 * lane i stores row i). */
template <int R, int MODE>
__device__ __forceinline__ void epilogue(const MvArgs &a, int total, int g, int wave, int lane,
                                         const float (&acc)[R]) {
#pragma clang fp contract(off)
  if (MODE == MV_SWIGLU) {
    constexpr int P = R / 2;
    const int p0 = (g * kWaves + wave) * P;
#pragma unroll
    for (int i = 0; i < P; i++)
      if (lane == i && p0 + i < total) gst<float>(a.seg[0].y + p0 + i, silu_mul(acc[i], acc[P + i]));
    return;
  }
  const int r0 = (g * kWaves + wave) * R;
#pragma unroll
  for (int i = 0; i < R; i++) {
    if (lane != i || r0 + i >= total) continue;
    int s, lr;
    locate(a, r0 + i, s, lr);
    const MvSeg &sg = a.seg[s];
    if (MODE == MV_RESID) {
      gst<float>(sg.y + lr, acc[i] + gld<float>(sg.r + lr));
      continue;
    }
    float v = acc[i];
    if (sg.kind == SEG_PLAIN) {
      gst<float>(sg.y + lr, v);
      continue;
    }
    const int hd = a.rope.head_dim;
    const int pos = a.rope.pos_dev ? gld<int>(a.rope.pos_dev) : a.rope.pos;
    if (pos < 0 || pos >= a.rope.max_seq) continue; /* rejected on the host */
    const int h = lr / hd, d = lr - h * hd;
    if (sg.kind != SEG_KV) {
      /* adjacent pair (d & ~1, d | 1) rotated by the row of pos
       * (kernels_cpu.c:415-429: products and difference rounded apart) */
      const float2 cs = gld<float2>(a.rope.cs + (size_t)pos * (hd >> 1) + (d >> 1));
      const float x0 = acc[i & ~1], x1 = acc[i | 1];
      v = (d & 1) ? x0 * cs.y + x1 * cs.x : x0 * cs.x - x1 * cs.y;
    }
    if (sg.kind == SEG_ROPE)
      gst<float>(sg.y + lr, v);
    else
      gst<float>(sg.y + ((size_t)h * a.rope.max_seq + pos) * hd + d, v);
  }
}

/* Persistent grid: workgroup b handles row groups b, b + gridDim.x, ... with x
 * staged in LDS once.  A wave walks (group, tile) steps and loads the weight
 * fragments of step s+1 before computing step s; the first step's loads are
 * issued before x is staged so both latencies overlap. */
template <int DT, int R, int MODE>
__global__ __launch_bounds__(kThreads) void mv_kernel(MvArgs a) {
  using T = typename TrSplit<DT>::type;
  extern __shared__ float xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb = a.cols / T::QK;
  const size_t rowbytes = (size_t)nb * T::BB;
  constexpr int BPT = GQ_WAVE / T::LPB;
  constexpr int P = MODE == MV_SWIGLU ? R / 2 : R;
  const int ntile = (nb + BPT - 1) / BPT;
  const int part = lane % T::LPB, bt = lane / T::LPB;
  const int total = total_rows(a, MODE);
  const int ngroups = (total + kWaves * P - 1) / (kWaves * P);
  const int mygroups = (int)blockIdx.x < ngroups ? (ngroups - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int nsteps = mygroups * ntile;

  typename T::Frag cur[R], nxt[R];
  const uint8_t *rp[R];
  int g = blockIdx.x, t = 0;
  if (nsteps > 0) {
    group_rows<R, MODE>(a, total, g, wave, rowbytes, rp);
    const int bc = min(bt, nb - 1);
#pragma unroll
    for (int i = 0; i < R; i++) T::load(cur[i], rp[i], bc, part);
  }
  stage_x(a, xs);

  float acc[R];
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = 0.f;
  for (int s = 0; s < nsteps; s++) {
    int t1 = t + 1, g1 = g;
    const uint8_t *rn[R];
#pragma unroll
    for (int i = 0; i < R; i++) rn[i] = rp[i];
    if (s + 1 < nsteps) {
      if (t1 == ntile) {
        t1 = 0;
        g1 = g + gridDim.x;
        group_rows<R, MODE>(a, total, g1, wave, rowbytes, rn);
      }
      const int bc = min(t1 * BPT + bt, nb - 1);
#pragma unroll
      for (int i = 0; i < R; i++) T::load(nxt[i], rn[i], bc, part);
    }
    {
      const int b = t * BPT + bt;
      const bool bok = b < nb;
      typename T::X x;
      T::load_x(x, (const GQ_LDS uint8_t *)xs, nullptr, bok ? b : nb - 1, part);
#pragma unroll
      for (int i = 0; i < R; i++) {
        const float v = T::dot(cur[i], x, part);
        acc[i] += bok ? v : 0.f;
      }
    }
    if (t == ntile - 1) {
#pragma unroll
      for (int i = 0; i < R; i++) acc[i] = gq_wave_sum(acc[i]);
      epilogue<R, MODE>(a, total, g, wave, lane, acc);
#pragma unroll
      for (int i = 0; i < R; i++) acc[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
      cur[i] = nxt[i];
      rp[i] = rn[i];
    }
    t = t1;
    g = g1;
  }
}

/* ------------------------------------------------------------------------
 * LDS-streamed matvec.
 *
 * The weight rows of a workgroup's row groups ("stages" of rs rows) are
 * streamed into a ring of kNS LDS buffers with direct global->LDS DMA loads
 * (global_load_lds_dwordx4: 1 KB per wave instruction, no VGPRs), kNS-1
 * stages ahead of the one being computed, so each CU keeps tens of KB of HBM
 * reads in flight independent of register pressure and of the 2-byte block
 * alignment of Q6_K.  Waves keep their x slices in registers for the whole
 * kernel (RMSNorm folded as y = r * W (w .* x)); a team of ts waves splits K
 * (wave j owns tiles j, j+ts, ...).  A wave computes RW rows at a time (all
 * their LDS reads issued before the arithmetic), reduces each row over its
 * 16-lane DPP rows only, and the 4 row partials per wave meet in LDS, where
 * the epilogue adds them. */
constexpr int kNS = 3;    /* stage buffers: 4-6 measured slower (one workgroup per CU) */
constexpr int kRing = 8;  /* residual-row ring slots (>= kNS + 1) */
constexpr int kRedW = kWaves * 4; /* row partials per row: 4 per wave */
int g_stage_cap = 24576;  /* bytes of weights per stage buffer */
int g_lds_wg_per_cu = 0;  /* 0: as many workgroups per CU as LDS allows */

struct MvPlan {
  int rs;           /* weight rows per stage (MV_SWIGLU: rs/2 gate + rs/2 up) */
  int ts, nteam;    /* waves per team, teams per workgroup */
  int ntile;        /* column tiles per row */
  int ngroups;      /* stages over the whole launch */
  int rowbytes;
  int stride;       /* LDS bytes per stage buffer */
  int total;        /* output rows */
  int xl;           /* LDS offset of x staged by DMA (slot 2 onwards), XL kernels */
};

/* Wave `wave`'s 1 KB copy instructions for nbytes (a multiple of 16) split
 * over nwv waves. */
__device__ __forceinline__ int copy_count(int nbytes, int wave, int nwv = kWaves) {
  const int ng = (nbytes / 16 + 63) / 64;
  return wave < ng ? (ng - wave + nwv - 1) / nwv : 0;
}

/* [src, src + nbytes) into LDS at dst in the xswz order (nbytes a multiple
 * of 256): the lane that writes position q reads source unit xswz(q). */
__device__ __forceinline__ void copy_range_sw(const uint8_t *src, int nbytes, GQ_LDS uint8_t *dst, int wave,
                                              int lane, int nwv = kWaves) {
  const int nchunk = nbytes / 16, ng = (nchunk + 63) / 64;
  const uint32_t base = (uint32_t)(uintptr_t)dst;
  for (int g = wave; g < ng; g += nwv) {
    const int c = g * 64 + lane;
    const uint32_t d = __builtin_amdgcn_readfirstlane(base + (uint32_t)g * 1024u);
    if (c < nchunk) dma16(src + xswz(16u * (uint32_t)c), d);
  }
}

/* Rows [src, src + nbytes) into LDS at dst by 16-byte DMA (dma16), 1 KB per
 * wave instruction, instructions dealt round-robin over nwv waves. */
__device__ __forceinline__ void copy_range(const uint8_t *src, int nbytes, GQ_LDS uint8_t *dst, int wave,
                                           int lane, int nwv = kWaves) {
  const int nchunk = nbytes / 16, ng = (nchunk + 63) / 64;
  const uint32_t base = (uint32_t)(uintptr_t)dst;
  for (int g = wave; g < ng; g += nwv) {
    const int c = g * 64 + lane;
    const uint32_t d = __builtin_amdgcn_readfirstlane(base + (uint32_t)g * 1024u);
    if (c < nchunk) dma16(src + (size_t)c * 16, d);
  }
}


/* Stage `g`'s rows: global rows [g*rs, g*rs+rs) (clamped to the end of their
 * segment), or for MV_SWIGLU gate and up rows [g*rs/2, g*rs/2 + rs/2); for
 * MV_RESID also the stage's residual values into `rbuf`.  Returns this wave's
 * DMA instruction count. */
template <int MODE>
__device__ __forceinline__ int issue_stage(const MvArgs &a, const MvPlan &pl, int g, GQ_LDS uint8_t *buf,
                                           GQ_LDS float *rbuf, int wave, int lane) {
  if (MODE == MV_SWIGLU) {
    const int h = pl.rs / 2, r0 = g * h, n = min(h, pl.total - r0);
    const int nb = n * pl.rowbytes;
    copy_range(a.seg[0].w + (size_t)r0 * pl.rowbytes, nb, buf, wave, lane);
    copy_range(a.seg[1].w + (size_t)r0 * pl.rowbytes, nb, buf + h * pl.rowbytes, wave, lane);
    return 2 * copy_count(nb, wave);
  }
  const int r0 = g * pl.rs;
  int s, lr;
  locate(a, r0, s, lr);
  const int n = min(pl.rs, a.seg[s].rows - lr);
  const int nb = n * pl.rowbytes;
  copy_range(a.seg[s].w + (size_t)lr * pl.rowbytes, nb, buf, wave, lane);
  int c = copy_count(nb, wave);
  if (MODE == MV_RESID && wave == kWaves - 1) {
    const uint32_t d = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)rbuf);
    if (lane < n) dma4(a.seg[s].r + lr + lane, d);
    c++;
  }
  return c;
}


/* Store one finished output row `lr` of segment `s` (`s` is the same for the
 * whole stage: a stage never straddles segments).  No vector global loads
 * here: inside the pipelined loop every operand comes from LDS, registers or
 * scalar loads of the kernel arguments (see dma16). */
template <int MODE>
__device__ __forceinline__ void store_row(const MvArgs &a, int s, int lr, float v, float partner,
                                          float resid, int pos, const float2 *scs) {
#pragma clang fp contract(off)
  if (MODE == MV_SWIGLU) {
    gst<float>(a.seg[0].y + lr, silu_mul(v, partner));
    return;
  }
  const MvSeg &sg = a.seg[s];
  if (MODE == MV_RESID) {
    gst<float>(sg.y + lr, v + resid);
    return;
  }
  if (sg.kind == SEG_PLAIN) {
    gst<float>(sg.y + lr, v);
    return;
  }
  const int hd = a.rope.head_dim;
  if (pos < 0 || pos >= a.rope.max_seq) return; /* rejected on the host */
  const int h = lr / hd, d = lr - h * hd;
  if (sg.kind != SEG_KV) {
    /* adjacent pair rotated by the row of pos (kernels_cpu.c:415-429) */
    const float2 cs = scs[d >> 1];
    const float x0 = (d & 1) ? partner : v, x1 = (d & 1) ? v : partner;
    v = (d & 1) ? x0 * cs.y + x1 * cs.x : x0 * cs.x - x1 * cs.y;
  }
  if (sg.kind == SEG_ROPE)
    gst<float>(sg.y + lr, v);
  else
    gst<float>(sg.y + ((size_t)h * a.rope.max_seq + pos) * hd + d, v);
}

/* The split-K kernel's statically sized LDS: row partials, the RMSNorm
 * partial sums, the residual ring and the RoPE row. */
struct MvShared {
  __attribute__((aligned(16))) float red[2][32][kRedW];
  float red_ss[kWaves];
  __attribute__((aligned(16))) float rres[kRing][32];
  float2 scs[256];
};

/* One launch's work as workgroup `bid` of `nblk` (the whole grid, or one
 * side of a paired launch) */
template <int DT, int MODE, int TPW, int RW, bool XL, int NS>
__device__ __forceinline__ void mvl_body(const MvArgs &a, const MvPlan &pl, int bid, int nblk, MvShared &sh) {
  using T = typename TrL<DT, XL>::type;
  static_assert(NS >= 3 && NS + 1 <= kRing, "ring of NS stage slots, NS - 1 stages in flight");
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  GQ_LDS uint8_t *lds = (GQ_LDS uint8_t *)smem;
  auto &red = sh.red;
  auto &red_ss = sh.red_ss;
  auto &rres = sh.rres;
  float2 *scs = sh.scs;
  GQ_LDS float *lres = (GQ_LDS float *)&rres[0][0];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); /* scalar: the DMA counts are too */
  constexpr int BPT = GQ_WAVE / T::LPB;
  const int nb = a.cols / T::QK;
  const int part = lane % T::LPB, bt = lane / T::LPB;
  const int team = wave / pl.ts, wj = wave - team * pl.ts;
  const bool active = team < pl.nteam;
  const int mygroups = bid < pl.ngroups ? (pl.ngroups - 1 - bid) / nblk + 1 : 0;

  typename T::X xs[TPW];
  float ss = 0.f;
  int pos = 0;
  /* this wave's DMA instructions of stages k .. k + NS - 2 at the top of
   * iteration k */
  int cnt[NS - 1];
  if constexpr (XL) {
    /* x, the norm weight and the RoPE row go to LDS by DMA (x at slot NS-1,
     * which stage NS-1 overwrites only after the barrier below), followed by
     * the first NS-1 stages: x's latency overlaps theirs */
    const int xb = a.cols * 4;
    copy_range_sw((const uint8_t *)a.x, xb, lds + pl.xl, wave, lane);
    if (a.norm_w) copy_range_sw((const uint8_t *)a.norm_w, xb, lds + pl.xl + xb, wave, lane);
    if (MODE == MV_STORE && a.rope.cs) {
      pos = a.rope.pos_dev ? gq_sld<int>(a.rope.pos_dev) : a.rope.pos;
      const int hd = a.rope.head_dim; /* floats in one table row (hd/2 pairs) */
      if (wave == 0 && pos >= 0 && pos < a.rope.max_seq) {
        const float *crow = (const float *)(a.rope.cs + (size_t)pos * (hd >> 1));
        const uint32_t base = (uint32_t)(uintptr_t)(GQ_LDS float2 *)scs;
        for (int o = 0; o < hd; o += 64)
          if (lane < hd - o) dma4(crow + o + lane, __builtin_amdgcn_readfirstlane(base + 4u * o));
      }
    }
    int sum = 0;
#pragma unroll
    for (int j = 0; j < NS - 1; j++) {
      cnt[j] = j < mygroups ? issue_stage<MODE>(a, pl, bid + j * nblk, lds + j * pl.stride,
                                                lres + j * 32, wave, lane)
                            : 0; /* mygroups >= 1 */
      sum += cnt[j];
    }
    /* VMEM loads complete in issue order: with only the stages' copies
     * outstanding, this wave's part of x has landed; the barrier extends
     * that to every wave's */
    wait_vmcnt(sum);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TPW; i++) {
      const int b = (wj + i * pl.ts) * BPT + bt;
      float s2 = 0.f;
      T::template load_x<true>(xs[i], lds + pl.xl, a.norm_w ? lds + pl.xl + xb : nullptr, min(b, nb - 1), part,
                               &s2);
      if (b < nb && (wj + i * pl.ts) < pl.ntile) ss += s2;
    }
  } else {
    /* everything the loop needs from global memory besides the weights is
     * loaded and consumed first: x slices (and the RMSNorm sum of squares
     * from team 0), the position and the RoPE table row.  (Issuing stage 0
     * before them measured slower: stage 1 then goes out a round trip
     * later.) */
#pragma unroll
    for (int i = 0; i < TPW; i++) {
      const int b = (wj + i * pl.ts) * BPT + bt;
      float s2 = 0.f;
      T::load_xg(xs[i], a.x, a.norm_w, min(b, nb - 1), part, s2);
      if (b < nb && (wj + i * pl.ts) < pl.ntile) ss += s2;
    }
    if (MODE == MV_STORE && a.rope.cs) {
      pos = a.rope.pos_dev ? gld<int>(a.rope.pos_dev) : a.rope.pos;
      const int half = a.rope.head_dim >> 1;
      if (pos >= 0 && pos < a.rope.max_seq)
        for (int i = threadIdx.x; i < half && i < 256; i += kThreads)
          scs[i] = gld<float2>(a.rope.cs + (size_t)pos * half + i);
    }
  }
  float rscale = 1.f;
  if (a.norm_w) { /* 1/sqrt(mean(x^2) + eps) (kernels_cpu.c:242-253) */
    ss = gq_wave_sum(ss);
    if (lane == 0) red_ss[wave] = active && team == 0 ? ss : 0.f;
    __syncthreads();
    float tot = (red_ss[0] + red_ss[1]) + (red_ss[2] + red_ss[3]);
    tot = tot / (float)a.cols;
    tot = tot + a.eps;
    rscale = 1.0f / sqrtf(tot);
  } else if (XL) {
    __syncthreads(); /* every wave has read x before stage 2 overwrites it */
  }
  if constexpr (!XL) {
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); /* those loads are done */
#pragma unroll
    for (int j = 0; j < NS - 1; j++)
      cnt[j] = j < mygroups ? issue_stage<MODE>(a, pl, bid + j * nblk, lds + j * pl.stride,
                                                lres + j * 32, wave, lane)
                            : 0; /* mygroups >= 1 */
  }

  /* Stage k's copies are issued at iteration k-(NS-1) into the slot stage
   * k-NS used (computed at iteration k-NS, before the barrier closing it):
   * before that iteration's wait, or with x read from global memory (the
   * long rows of the down projection) after its arithmetic, where the wait
   * for room in the memory pipeline does not hold the arithmetic up
   * (16.1 against 16.6 us for the 8B down; the short-row launches measured
   * 0.1 us slower that way).  At iteration k they are waited for, computed
   * and at iteration k+1 its rows are finished (reduced, stored). */
  constexpr bool LATE = !XL;
  const int hrows = MODE == MV_SWIGLU ? pl.rs / 2 : pl.rs;
  const int rpw = pl.rs / pl.nteam; /* rows per team and stage, a multiple of RW */
  int slot = 0;                     /* k % NS */
  for (int k = 0; k <= mygroups; k++) {
    auto issue_ahead = [&]() {
      const int kn = k + NS - 1, sn = slot == 0 ? NS - 1 : slot - 1; /* kn % NS */
      const int nn = kn < mygroups ? issue_stage<MODE>(a, pl, bid + kn * nblk, lds + sn * pl.stride,
                                                       lres + (kn % kRing) * 32, wave, lane)
                                   : 0;
#pragma unroll
      for (int j = 0; j < NS - 2; j++) cnt[j] = cnt[j + 1];
      cnt[NS - 2] = nn;
      return nn;
    };
    if (k < mygroups) {
      /* VMEM loads complete in issue order: with only the copies of later
       * stages outstanding (k+1 .. k+NS-1, or k+NS-2 when issued late),
       * this wave's copies of stage k have landed; the barrier extends that
       * to every wave's */
      int pend = 0;
#pragma unroll
      for (int j = 1; j < NS - 1; j++) pend += cnt[j]; /* stages k+1 .. k+NS-2 */
      if constexpr (!LATE) pend += issue_ahead();
      wait_vmcnt(pend);
    }
    __syncthreads();
    if (k > 0) { /* finish the rows of stage k-1: row t on lane t/4 of wave t%4 */
      const int r0 = (bid + (k - 1) * nblk) * hrows;
      int s = 0, lr0 = r0;
      if (MODE != MV_SWIGLU) locate(a, r0, s, lr0);
      s = __builtin_amdgcn_readfirstlane(s);
      lr0 = __builtin_amdgcn_readfirstlane(lr0);
      const int t = lane * kWaves + wave;
      if (t < hrows && r0 + t < pl.total) {
        const int tp = MODE == MV_SWIGLU ? t + hrows : (t ^ 1);
        const int nred = 4 * pl.ts;
        float v = 0.f, w = 0.f;
        for (int j = 0; j < nred; j++) v += red[(k - 1) & 1][t][j], w += red[(k - 1) & 1][tp][j];
        store_row<MODE>(a, s, lr0 + t, v * rscale, w * rscale,
                        MODE == MV_RESID ? rres[(k - 1) % kRing][t] : 0.f, pos, scs);
      }
    }
    if (k == mygroups) break;
    if (active) {
      const GQ_LDS uint8_t *buf = lds + slot * pl.stride;
      for (int i0 = team * rpw; i0 < (team + 1) * rpw; i0 += RW) {
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) acc[r] = 0.f;
#pragma unroll
        for (int ti = 0; ti < TPW; ti++) {
          const int t = wj + ti * pl.ts;
          const int b = t * BPT + bt;
          if (t < pl.ntile) {
            typename T::Frag f[RW];
            const uint32_t off = i0 * pl.rowbytes + min(b, nb - 1) * T::BB;
#pragma unroll
            for (int r = 0; r < RW; r++) T::load_lds(f[r], buf, off + r * pl.rowbytes, part);
#pragma unroll
            for (int r = 0; r < RW; r++) {
              const float v = T::dot(f[r], xs[ti], part);
              acc[r] += b < nb ? v : 0.f;
            }
          }
        }
#pragma unroll
        for (int r = 0; r < RW; r++) acc[r] = gq_row16_sum(acc[r]);
        if ((lane & 15) == 0)
#pragma unroll
          for (int r = 0; r < RW; r++) red[k & 1][i0 + r][wj * 4 + (lane >> 4)] = acc[r];
      }
    }
    if constexpr (LATE) issue_ahead();
    __syncthreads();
    slot = slot == NS - 1 ? 0 : slot + 1;
  }
}

template <int DT, int MODE, int TPW, int RW, bool XL, int NS>
__global__ __launch_bounds__(kThreads) void mvl_kernel(MvArgs a, MvPlan pl) {
  __shared__ MvShared sh;
  mvl_body<DT, MODE, TPW, RW, XL, NS>(a, pl, (int)blockIdx.x, (int)gridDim.x, sh);
}

/* Two MV_STORE launches of different dtypes in one: workgroups [0, g0) run
 * the first (a0, p0), the rest the second.  For the q/k/v projections of
 * layers whose v is Q6_K and q, k are Q4_K. */
template <int DT0, int TPW0, int RW0, bool XL0, int DT1, int TPW1, int RW1, bool XL1>
__global__ __launch_bounds__(kThreads) void mvl_pair_kernel(MvArgs a0, MvPlan p0, MvArgs a1, MvPlan p1, int g0) {
  __shared__ MvShared sh;
  const int b = (int)blockIdx.x;
  if (b < g0)
    mvl_body<DT0, MV_STORE, TPW0, RW0, XL0, kNS>(a0, p0, b, g0, sh);
  else
    mvl_body<DT1, MV_STORE, TPW1, RW1, XL1, kNS>(a1, p1, b - g0, (int)gridDim.x - g0, sh);
}

/* ------------------------------------------------------------------------
 * Wave-private LDS-streamed matvec, for shapes where one wave covers whole
 * rows (at most two column tiles, x slices in registers: every 4096-column
 * projection and the LM head).
 *
 * Each wave owns groups of RW weight rows (MV_SWIGLU: RW/2 gate + RW/2 up
 * rows) and streams them with DMA into a private ring of ns LDS slots, ns-1
 * groups ahead of the one it computes; it reduces each row over the wave with
 * DPP and stores.  Waves never wait for each other after the prologue: no
 * barriers in the loop, so one wave's memory latency overlaps the others'
 * arithmetic.  The ring depth ns (3..8) is chosen per launch to fill LDS.
 *
 * LDS is slot-major: slot k of every wave, for k = 0..ns-1.  The prologue
 * stages x (and the RMSNorm weight) in the last slot row, which only the
 * loop's first DMA overwrites, so x's copy overlaps the first ns-1 groups'
 * copies; the waves take their x slices into registers before the loop. */
constexpr int kMaxWaves = 16;
constexpr int kMaxNS = 8;

struct MwPlan {
  int ngroups;  /* groups over the launch */
  int rowbytes;
  int slot;     /* LDS bytes per ring slot */
  int ns;       /* ring slots per wave */
  int pre;      /* groups issued before x is waited for */
  int x_off;    /* LDS offset of staged x (the last slot row) */
  int nw_off;   /* LDS offset of the staged norm weight */
  int total;    /* output rows */
};

/* Rows of group g: first local row and count, segment (uniform). */
template <int MODE, int RW>
__device__ __forceinline__ void group_span(const MvArgs &a, const MwPlan &pl, int g, int &s, int &lr, int &n) {
  if (MODE == MV_SWIGLU) {
    constexpr int P = RW / 2;
    s = 0, lr = g * P, n = min(P, pl.total - lr);
  } else {
    locate(a, g * RW, s, lr);
    n = min(RW, a.seg[s].rows - lr);
  }
}

/* This wave's DMA instruction count for group g. */
template <int MODE, int RW>
__device__ __forceinline__ int group_count(const MvArgs &a, const MwPlan &pl, int g) {
  int s, lr, n;
  group_span<MODE, RW>(a, pl, g, s, lr, n);
  const int c = copy_count(n * pl.rowbytes, 0, 1);
  return MODE == MV_SWIGLU ? 2 * c : c + (MODE == MV_RESID ? 1 : 0);
}

/* Rows of group g into ring slot `buf` (one wave), and for MV_RESID the
 * group's residual values into `rbuf`. */
template <int MODE, int RW>
__device__ __forceinline__ void issue_group(const MvArgs &a, const MwPlan &pl, int g, GQ_LDS uint8_t *buf,
                                            GQ_LDS float *rbuf, int lane) {
  int s, lr, n;
  group_span<MODE, RW>(a, pl, g, s, lr, n);
  const int nb = n * pl.rowbytes;
  if (MODE == MV_SWIGLU) {
    copy_range(a.seg[0].w + (size_t)lr * pl.rowbytes, nb, buf, 0, lane, 1);
    copy_range(a.seg[1].w + (size_t)lr * pl.rowbytes, nb, buf + (RW / 2) * pl.rowbytes, 0, lane, 1);
    return;
  }
  copy_range(a.seg[s].w + (size_t)lr * pl.rowbytes, nb, buf, 0, lane, 1);
  if (MODE == MV_RESID) {
    const uint32_t d = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)rbuf);
    if (lane < n) dma4(a.seg[s].r + lr + lane, d);
  }
}

template <int DT, int MODE, int TPW, int RW>
__global__ __launch_bounds__(kMaxWaves * GQ_WAVE) void mvw_kernel(MvArgs a, MwPlan pl) {
  using T = Tr<DT>;
  constexpr int P = MODE == MV_SWIGLU ? RW / 2 : RW; /* output rows per group */
  static_assert(RW <= 4 && (MODE != MV_SWIGLU || RW % 2 == 0), "group shape");
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  GQ_LDS uint8_t *lds = (GQ_LDS uint8_t *)smem;
  __shared__ float red_ss[kMaxWaves];
  __shared__ __attribute__((aligned(16))) float2 scs[256];
  __shared__ __attribute__((aligned(16))) float rres[kMaxWaves][kMaxNS][4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwv = blockDim.x >> 6;
  constexpr int BPT = GQ_WAVE / T::LPB;
  const int nb = a.cols / T::QK;
  const int part = lane % T::LPB, bt = lane / T::LPB;
  const int gw = blockIdx.x * nwv + wave, W = gridDim.x * nwv;
  const int mygroups = gw < pl.ngroups ? (pl.ngroups - 1 - gw) / W + 1 : 0;
  const int ns = pl.ns, row = nwv * pl.slot; /* bytes of one slot row */
  GQ_LDS uint8_t *ring = lds + wave * pl.slot; /* slot k at ring + k * row */
  GQ_LDS float *rr = (GQ_LDS float *)&rres[wave][0][0];

  /* prologue: x, the norm weight and the RoPE row into LDS (the whole
   * workgroup), then this wave's first ns-1 groups, all with DMA */
  const int xb = a.cols * 4;
  copy_range_sw((const uint8_t *)a.x, xb, lds + pl.x_off, wave, lane, nwv);
  if (a.norm_w) copy_range_sw((const uint8_t *)a.norm_w, xb, lds + pl.nw_off, wave, lane, nwv);
  int pos = 0;
  if (MODE == MV_STORE && a.rope.cs) {
    pos = a.rope.pos_dev ? gq_sld<int>(a.rope.pos_dev) : a.rope.pos;
    const int hd = a.rope.head_dim; /* floats in one table row (hd/2 pairs) */
    if (wave == 0 && pos >= 0 && pos < a.rope.max_seq) {
      const float *crow = (const float *)(a.rope.cs + (size_t)pos * (hd >> 1));
      const uint32_t base = (uint32_t)(uintptr_t)(GQ_LDS float2 *)scs;
      for (int o = 0; o < hd; o += 64)
        if (lane < hd - o) dma4(crow + o + lane, __builtin_amdgcn_readfirstlane(base + 4u * o));
    }
  }
  /* pl.pre of the first ns-1 groups go out before x is waited for, the rest
   * after x is in registers (x queues behind whatever is issued before it
   * across the whole device) */
  int pend = 0; /* this wave's DMA instructions of the groups after the current one */
  const int npre = min(min(pl.pre, ns - 1), mygroups);
  for (int k = 0; k < npre; k++) {
    issue_group<MODE, RW>(a, pl, gw + k * W, ring + k * row, rr + 4 * k, lane);
    pend += group_count<MODE, RW>(a, pl, gw + k * W);
  }
  /* VMEM loads complete in issue order: with at most the groups' copies
   * outstanding, this wave's part of x (and the rest) has landed; the barrier
   * extends that to every wave's */
  wait_vmcnt(pend);
  __syncthreads();
  float rscale = 1.f;
  if (a.norm_w) { /* 1/sqrt(mean(x^2) + eps) (kernels_cpu.c:242-253) */
    float ss = 0.f;
    for (int i = threadIdx.x; i < (a.cols >> 2); i += blockDim.x) {
      const float4 v = lld<float4>(lds + pl.x_off, 16u * i);
      ss = __builtin_fmaf(v.x, v.x, ss), ss = __builtin_fmaf(v.y, v.y, ss);
      ss = __builtin_fmaf(v.z, v.z, ss), ss = __builtin_fmaf(v.w, v.w, ss);
    }
    ss = gq_wave_total(ss);
    if (lane == 0) red_ss[wave] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < nwv; w++) tot += red_ss[w];
    tot = tot / (float)a.cols;
    tot = tot + a.eps;
    rscale = 1.0f / sqrtf(tot);
  }
  typename T::X xs[TPW];
#pragma unroll
  for (int i = 0; i < TPW; i++)
    T::template load_x<true>(xs[i], lds + pl.x_off, a.norm_w ? lds + pl.nw_off : nullptr, min(i * BPT + bt, nb - 1),
                             part);
  __syncthreads(); /* the last slot row is free from here on */
  for (int k = npre; k < ns - 1 && k < mygroups; k++) {
    issue_group<MODE, RW>(a, pl, gw + k * W, ring + k * row, rr + 4 * k, lane);
    pend += group_count<MODE, RW>(a, pl, gw + k * W);
  }

  int slot = 0; /* j % ns */
  for (int j = 0; j < mygroups; j++) {
    const int g = gw + j * W;
    {
      const int jn = j + ns - 1, sn = slot == 0 ? ns - 1 : slot - 1; /* jn % ns: computed at j-1 */
      if (jn < mygroups) {
        issue_group<MODE, RW>(a, pl, gw + jn * W, ring + sn * row, rr + 4 * sn, lane);
        pend += group_count<MODE, RW>(a, pl, gw + jn * W);
      }
      pend -= group_count<MODE, RW>(a, pl, g);
      wait_vmcnt(pend); /* group j has landed */
    }
    const GQ_LDS uint8_t *buf = ring + slot * row;
    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = 0.f;
#pragma unroll
    for (int ti = 0; ti < TPW; ti++) {
      const int b = ti * BPT + bt;
      typename T::Frag f[RW];
      const uint32_t off = min(b, nb - 1) * T::BB;
#pragma unroll
      for (int r = 0; r < RW; r++) T::load_lds(f[r], buf, off + r * pl.rowbytes, part);
#pragma unroll
      for (int r = 0; r < RW; r++) {
        const float v = T::dot(f[r], xs[ti], part);
        acc[r] += b < nb ? v : 0.f;
      }
    }
    float tot[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) tot[r] = gq_wave_total(acc[r]) * rscale;
    /* lane r < P finishes output row r of the group */
    float v = tot[0], w = MODE == MV_SWIGLU ? tot[P] : tot[RW > 1 ? 1 : 0];
#pragma unroll
    for (int r = 1; r < P; r++)
      if (lane == r) v = tot[r], w = MODE == MV_SWIGLU ? tot[P + r] : tot[r ^ 1];
    int s, lr0, n;
    group_span<MODE, RW>(a, pl, g, s, lr0, n);
    s = __builtin_amdgcn_readfirstlane(s);
    lr0 = __builtin_amdgcn_readfirstlane(lr0);
    if (lane < n)
      store_row<MODE>(a, s, lr0 + lane, v, w, MODE == MV_RESID ? rres[wave][slot][lane] : 0.f, pos,
                      (const float2 *)scs);
    slot = slot == ns - 1 ? 0 : slot + 1;
  }
}

/* ------------------------------------------------------------------------
 * Register-ring matvec, for shapes where one wave covers whole rows.
 *
 * Each wave streams its groups of RW weight rows straight into registers
 * with ordinary global loads, kRB - 1 groups ahead of the one it computes
 * (a ring of kRB register buffers, rotated by unrolling so no data moves),
 * so the compiler tracks every load and waits on exactly the group it needs.
 * Nothing but x goes through LDS; the register file (512 KB per CU) holds
 * far more bytes in flight than LDS could.  x (times the RMSNorm weight) is
 * staged once per workgroup and each wave keeps its slices in registers and
 * computes the norm's sum of squares itself (a wave holds all of x).  Finished
 * rows are parked in LDS and stored after the loop: no store sits between a
 * load and its wait. */
constexpr int kRB = 3;

template <int DT, int TPW, int RW>
struct RBuf {
  typename Tr<DT>::Frag f[RW][TPW];
  float res;  /* MV_RESID: residual of row `lane` of the group */
  float2 cs;  /* fused RoPE: (cos, sin) of row `lane` of the group */
};

/* Loads of group g into B.  Groups past the wave's last are replaced by its
 * last group (already cached): the load sequence is the same on every path,
 * which keeps the compiler's wait counts exact. */
template <int DT, int MODE, int TPW, int RW>
__device__ __forceinline__ void rload(const MvArgs &a, const MwPlan &pl, int g, RBuf<DT, TPW, RW> &B, int lane,
                                      int part, int bt, int nb, int pos) {
  using T = Tr<DT>;
  constexpr int BPT = GQ_WAVE / T::LPB;
  int s, lr, n;
  group_span<MODE, RW>(a, pl, g, s, lr, n);
#pragma unroll
  for (int r = 0; r < RW; r++) {
    const uint8_t *row;
    if (MODE == MV_SWIGLU) {
      constexpr int H = RW / 2;
      row = a.seg[r / H].w + (size_t)(lr + min(r % H, n - 1)) * pl.rowbytes;
    } else {
      row = a.seg[s].w + (size_t)(lr + min(r, n - 1)) * pl.rowbytes;
    }
#pragma unroll
    for (int ti = 0; ti < TPW; ti++) T::load(B.f[r][ti], row, min(ti * BPT + bt, nb - 1), part);
  }
  if (MODE == MV_RESID) B.res = gld<float>(a.seg[s].r + lr + min(lane, n - 1));
  if (MODE == MV_STORE && a.rope.cs) {
    const int hd = a.rope.head_dim;
    const int d = (lr + min(lane, n - 1)) % hd;
    const int p = pos >= 0 && pos < a.rope.max_seq ? pos : 0;
    B.cs = gld<float2>(a.rope.cs + (size_t)p * (hd >> 1) + (d >> 1));
  }
}

/* Destination of output row lr of segment s (nullptr: position rejected). */
template <int MODE>
__device__ __forceinline__ float *rdest(const MvArgs &a, int s, int lr, int pos) {
  if (MODE == MV_SWIGLU) return a.seg[0].y + lr;
  const MvSeg &sg = a.seg[s];
  if (MODE == MV_RESID || sg.kind == SEG_PLAIN || sg.kind == SEG_ROPE) return sg.y + lr;
  if (pos < 0 || pos >= a.rope.max_seq) return nullptr; /* rejected on the host */
  const int hd = a.rope.head_dim, h = lr / hd, d = lr - h * hd;
  return sg.y + ((size_t)h * a.rope.max_seq + pos) * hd + d;
}

template <int DT, int MODE, int TPW, int RW>
__global__ __launch_bounds__(8 * GQ_WAVE) void mvr_kernel(MvArgs a, MwPlan pl) {
  using T = Tr<DT>;
  constexpr int P = MODE == MV_SWIGLU ? RW / 2 : RW; /* output rows per group */
  static_assert(RW <= 4 && RW % 2 == 0, "group shape");
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  GQ_LDS uint8_t *lds = (GQ_LDS uint8_t *)smem;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwv = blockDim.x >> 6;
  constexpr int BPT = GQ_WAVE / T::LPB;
  const int nb = a.cols / T::QK;
  const int part = lane % T::LPB, bt = lane / T::LPB;
  const int gw = blockIdx.x * nwv + wave, W = gridDim.x * nwv;
  const int mygroups = gw < pl.ngroups ? (pl.ngroups - 1 - gw) / W + 1 : 0;
  const int glast = gw + max(mygroups - 1, 0) * W;
  int pos = 0;
  if (MODE == MV_STORE && a.rope.cs) pos = a.rope.pos_dev ? gq_sld<int>(a.rope.pos_dev) : a.rope.pos;
  /* parked outputs: P floats per group, pl.slot groups per wave */
  GQ_LDS float *obuf = (GQ_LDS float *)(lds + pl.x_off) + (size_t)wave * pl.slot * P;

  RBuf<DT, TPW, RW> B0, B1, B2;
  if (mygroups > 0) {
    rload<DT, MODE, TPW, RW>(a, pl, gw, B0, lane, part, bt, nb, pos);
    rload<DT, MODE, TPW, RW>(a, pl, min(gw + W, glast), B1, lane, part, bt, nb, pos);
  }
  /* x and the norm weight into LDS (DMA, whole workgroup), behind the first
   * groups' loads; everything this wave issued has landed after vmcnt(0),
   * every wave's after the barrier */
  const int xb = a.cols * 4;
  copy_range((const uint8_t *)a.x, xb, lds, wave, lane, nwv);
  if (a.norm_w) copy_range((const uint8_t *)a.norm_w, xb, lds + pl.nw_off, wave, lane, nwv);
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); /* vmcnt(0) */
  __syncthreads();
  float ss = 0.f;
  typename T::X xs[TPW];
#pragma unroll
  for (int i = 0; i < TPW; i++) {
    const int b = i * BPT + bt;
    float q = 0.f;
    T::load_x(xs[i], lds, a.norm_w ? lds + pl.nw_off : nullptr, min(b, nb - 1), part, &q);
    if (b < nb) ss += q;
  }
  float rscale = 1.f;
  if (a.norm_w) { /* 1/sqrt(mean(x^2) + eps) (kernels_cpu.c:242-253) over the whole x */
    float tot = gq_wave_total(ss);
    tot = tot / (float)a.cols;
    tot = tot + a.eps;
    rscale = 1.0f / sqrtf(tot);
  }

  /* group j is computed from buffer j % 3 after the loads of group j+2 are
   * issued into the buffer group j-1 used */
  auto step = [&](int j, RBuf<DT, TPW, RW> &cur, RBuf<DT, TPW, RW> &nxt2) {
    rload<DT, MODE, TPW, RW>(a, pl, min(gw + (j + kRB - 1) * W, glast), nxt2, lane, part, bt, nb, pos);
    if (j >= mygroups) return;
    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = 0.f;
#pragma unroll
    for (int ti = 0; ti < TPW; ti++) {
      const int b = ti * BPT + bt;
#pragma unroll
      for (int r = 0; r < RW; r++) {
        const float v = T::dot(cur.f[r][ti], xs[ti], part);
        acc[r] += b < nb ? v : 0.f;
      }
    }
    float tot[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) tot[r] = gq_wave_total(acc[r]) * rscale;
    /* lane r < P finishes output row r of the group */
    float v = tot[0], w = MODE == MV_SWIGLU ? tot[P] : tot[1];
#pragma unroll
    for (int r = 1; r < P; r++)
      if (lane == r) v = tot[r], w = MODE == MV_SWIGLU ? tot[P + r] : tot[r ^ 1];
    float out;
    {
#pragma clang fp contract(off)
      if (MODE == MV_SWIGLU) {
        out = silu_mul(v, w);
      } else if (MODE == MV_RESID) {
        out = v + cur.res;
      } else {
        out = v;
        int s, lr, n;
        group_span<MODE, RW>(a, pl, gw + j * W, s, lr, n);
        const int kind = a.seg[__builtin_amdgcn_readfirstlane(s)].kind;
        if (a.rope.cs && (kind == SEG_ROPE || kind == SEG_ROPE_KV)) {
          /* adjacent pair rotated by the row of pos (kernels_cpu.c:415-429);
           * groups start on even rows */
          const float x0 = (lane & 1) ? w : v, x1 = (lane & 1) ? v : w;
          out = (lane & 1) ? x0 * cur.cs.y + x1 * cur.cs.x : x0 * cur.cs.x - x1 * cur.cs.y;
        }
      }
    }
    if (lane < P) obuf[j * P + lane] = out;
  };
  for (int j = 0; j < mygroups; j += kRB) {
    step(j, B0, B2);
    step(j + 1, B1, B0);
    step(j + 2, B2, B1);
  }
  /* the parked rows go out; nothing is loaded from here on */
  for (int j = 0; j < mygroups; j++) {
    int s, lr, n;
    group_span<MODE, RW>(a, pl, gw + j * W, s, lr, n);
    s = __builtin_amdgcn_readfirstlane(s);
    if (lane < n) {
      float *dst = rdest<MODE>(a, s, lr + lane, pos);
      if (dst) gst<float>(dst, obuf[j * P + lane]);
    }
  }
}


/* ------------------------------------------------------------------------
 * Matrix-core matvec (v_mfma_i32_16x16x64_i8).
 *
 * The dot products run on the int8 matrix cores, exactly, and the VALU only
 * unpacks quants and applies the per-sub-block scales (a third of the
 * instructions per weight of the fp32 kernels above).
 *
 *  - x (times the RMSNorm weight) becomes a 22-bit fixed point per 256-value
 *    block: x_int = rint(x * 2^e_b), e_b chosen from the block's max |x| so
 *    |x_int| < 2^22, split into three signed base-256 digits (byte planes,
 *    staged in LDS once per workgroup).  The error is at most 2^-23 of the
 *    block's max |x|, below the fp32 rounding of the reference's own sums.
 *  - An MFMA computes C[combo][row] = sum_k A[combo][k] B[k][row] over
 *    16 weight rows (B: their quants as int8, lane (row n, k-group g)) and 16
 *    "combos" (A: lane (combo c, k-group g) holds digit plane c%4 of x when
 *    c/4 == g and c%4 < 3, else zeros).  Output lane (n, g) then holds, for
 *    row n, the three plane sums of exactly the sub-block its own k-group
 *    covers: the lane that unpacked the quants also finishes them, with the
 *    scales it decoded, and no data crosses lanes until the row reduction.
 *  - Plane sums are exact int32 (|sum| <= 32*15*128); the fp32 part is
 *    (d*sc) * (s0 + 256 s1 + 65536 s2) * 2^-e_b - dmin*m*sum(x) per sub-block.
 *  - Weights stream from a tile-interleaved copy (gq_launch_mm_tile, made
 *    once when a model is bound): a stage is 16 rows x a chunk of the row's
 *    blocks, one contiguous range, so every DMA instruction reads 1 KB of
 *    consecutive bytes (row-by-row copies of the original layout with a
 *    bank-skewing pad measured 1.6x slower), and in LDS every B read is 16
 *    lanes x 16 consecutive bytes.  A ring of NS stages, NS-1 ahead.  Wave w owns blocks w,
 *    w+NW, ... of every chunk and keeps their A operands (x planes) in
 *    registers for the whole launch.
 *  - Row partials meet in LDS per tile; the epilogues are the split-K
 *    kernel's (store_row). */
typedef int gq_i32x4 __attribute__((ext_vector_type(4)));

struct MmPlan {
  int nb, cb, nch;  /* blocks per row, per chunk (stage), chunks per row */
  int bpc;          /* blocks per chunk per wave: ceil(cb / NW) */
  int ntiles;       /* 16-row tiles over the launch (MV_SWIGLU: 8 gate + 8 up rows) */
  int rowbytes, crb;
  int stride;       /* LDS bytes per ring slot */
  int ns;           /* ring slots */
  int xs;           /* LDS offset of the waves' x slices (the last xslots ring slots) */
  int xslots;
  int xwb;          /* bytes of x slices per wave: 1 KB per block, twice with a norm weight */
  int xsum, swb;    /* LDS offset of the waves' sub-block sums of x, bytes per wave */
  int planes, pwb;  /* without AREG: LDS offset of the waves' digit planes, bytes per wave */
  int eb;           /* without AREG: LDS offset of the waves' block exponents (32 bytes each) */
  int park;         /* LDS offset of the finished outputs (16 floats per tile) */
  int total;        /* output rows (MV_SWIGLU: gate rows) */
};

/* Static LDS of the matrix-core kernel: row partials per tile, the RMSNorm
 * partial sums, the residual ring and the RoPE row. */
template <int NW>
struct MmShared {
  float red[2][16][NW];
  float red_ss[NW];
  float rres[kRing][16];
  float2 scs[256];
};

__device__ __forceinline__ float gq_row16_max(float v) {
  v = fmaxf(v, gq_dpp<0x128>(v));
  v = fmaxf(v, gq_dpp<0x124>(v));
  v = fmaxf(v, gq_dpp<0x4e>(v));
  v = fmaxf(v, gq_dpp<0xb1>(v));
  return v;
}

/* Byte r of each of four dwords, packed (v_perm: selectors 0-3 take src1's
 * bytes, 4-7 src0's, 12 a zero byte). */
__device__ __forceinline__ uint32_t plane4(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3, uint32_t r) {
  const uint32_t lo = __builtin_amdgcn_perm(d1, d0, r | (4u + r) << 8 | 0x0c0c0000u);
  const uint32_t hi = __builtin_amdgcn_perm(d3, d2, 0x0c0cu | r << 16 | (4u + r) << 24);
  return lo | hi;
}

/* Maximum over the wave (DPP only); every lane receives it. */
__device__ __forceinline__ float gq_wave_maxf(float v) {
  v = gq_row16_max(v);
  int iv = __builtin_bit_cast(int, v);
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(iv, iv, 0x142, 0xa, 0xf, false)));
  iv = __builtin_bit_cast(int, v);
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(iv, iv, 0x143, 0xc, 0xf, false)));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

/* One wave's blocks of x -> its A operands' source.  Block ai (valid when
 * bit ai of `valid` is set) was staged at xw + 1024 ai (the norm weight at
 * xw + 1024 (MAXB + ai) when norm); lane L converts values 4L .. 4L+3:
 * x (times the norm weight) -> digit planes at pw + 768 ai + 256 r, the
 * block exponent E[ai] and the sub-block sums (SBW values each) at
 * sw + 4 (ai * 256/SBW + sub-block).  Returns the wave's sum of raw x^2. */
template <int SBW, int MAXB>
__device__ __forceinline__ float mm_wave_x(GQ_LDS uint8_t *lds, uint32_t xw, uint32_t pw, uint32_t sw,
                                           uint32_t valid, bool norm, int lane, int (&E)[MAXB]) {
  float ss = 0.f;
#pragma unroll
  for (int ai = 0; ai < MAXB; ai++) {
    E[ai] = 0;
    if (!(valid >> ai & 1u)) continue;
    float4 x = lld<float4>(lds, xw + 1024u * ai + 16u * lane);
    ss = __builtin_fmaf(x.x, x.x, ss), ss = __builtin_fmaf(x.y, x.y, ss);
    ss = __builtin_fmaf(x.z, x.z, ss), ss = __builtin_fmaf(x.w, x.w, ss);
    if (norm) {
      const float4 w = lld<float4>(lds, xw + 1024u * (MAXB + ai) + 16u * lane);
      x = make_float4(x.x * w.x, x.y * w.y, x.z * w.z, x.w * w.w);
    }
    const float mb = gq_wave_maxf(fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
    /* mb = f 2^E, f in [0.5, 1): x 2^(22-E) stays within 2^22 in magnitude */
    const int e = mb > 0.f ? 22 - __builtin_amdgcn_frexp_expf(mb) : 0;
    E[ai] = e;
    const float xv[4] = {x.x, x.y, x.z, x.w};
    uint32_t dg[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int xi = (int)rintf(__builtin_amdgcn_ldexpf(xv[k], e));
      /* balanced base-256 digits d0 + 256 d1 + 65536 d2, each in -128..127:
       * the bytes of xi + 0x808080, each minus 128 */
      dg[k] = ((uint32_t)xi + 0x808080u) ^ 0x808080u;
    }
#pragma unroll
    for (uint32_t r = 0; r < 3; r++)
      lst<uint32_t>(lds, pw + 768u * ai + 256u * r + 4u * lane, plane4(dg[0], dg[1], dg[2], dg[3], r));
    float su = (x.x + x.y) + (x.z + x.w);
    if (SBW == 32) {
      su = gq_row8_sum(su);
      if ((lane & 7) == 0) lst<float>(lds, sw + 4u * (8 * ai + (lane >> 3)), su);
    } else {
      su += gq_dpp<0x4e>(su);
      su += gq_dpp<0xb1>(su);
      if ((lane & 3) == 0) lst<float>(lds, sw + 4u * (16 * ai + (lane >> 2)), su);
    }
  }
  return ss;
}

/* Q4_K block for a 16-row tile.  Lane (row n, k-group g) reads the block's
 * header and qs[32g .. 32g+31]: low nibbles are weights 64g + i of
 * sub-block 2g, high nibbles 64g + 32 + i of sub-block 2g+1
 * (quant_matvec_q4_k.c:93-132).  MFMA j takes weights 64g + 16j .. +15, so
 * A operand j holds x digits 64g + 16j .. +15 of the block; MFMAs 0, 1
 * accumulate sub-block 2g, MFMAs 2, 3 sub-block 2g+1. */
struct MmQ4K {
  static constexpr int BB = 144, SBW = 32, NA = 4;
  __device__ static uint32_t aoff(int g, int j) { return 64u * g + 16u * j; }
  struct Frag {
    uint4 h, q0, q1;
  };
  /* row n's block in the tile-interleaved layout at blk: 16-byte chunk k
   * at 256 k + 16 n (chunk 0 the header, 1 + 2g and 2 + 2g this lane's
   * quants): every read is 16 lanes x 16 consecutive bytes */
  __device__ static void load(Frag &f, const GQ_LDS uint8_t *blk, int n, int g) {
    f.h = lld<uint4>(blk, 16 * n);
    f.q0 = lld<uint4>(blk, 256 * (1 + 2 * g) + 16 * n);
    f.q1 = lld<uint4>(blk, 256 * (2 + 2 * g) + 16 * n);
  }
  /* the block's MFMAs: C sets for sub-blocks 2g and 2g+1 */
  struct Acc {
    gq_i32x4 c0, c1;
  };
  __device__ static void mma(Acc &r, const Frag &f, const gq_i32x4 (&A)[NA]) {
    const uint4 q0 = f.q0, q1 = f.q1;
    const int M = 0x0f0f0f0f;
    const gq_i32x4 b0 = {(int)q0.x & M, (int)q0.y & M, (int)q0.z & M, (int)q0.w & M};
    const gq_i32x4 b1 = {(int)q1.x & M, (int)q1.y & M, (int)q1.z & M, (int)q1.w & M};
    const gq_i32x4 b2 = {(int)(q0.x >> 4) & M, (int)(q0.y >> 4) & M, (int)(q0.z >> 4) & M, (int)(q0.w >> 4) & M};
    const gq_i32x4 b3 = {(int)(q1.x >> 4) & M, (int)(q1.y >> 4) & M, (int)(q1.z >> 4) & M, (int)(q1.w >> 4) & M};
    const gq_i32x4 z = {0, 0, 0, 0};
    r.c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], b0, z, 0, 0, 0);
    r.c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], b1, r.c0, 0, 0, 0);
    r.c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], b2, z, 0, 0, 0);
    r.c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], b3, r.c1, 0, 0, 0);
  }
  /* the block's contribution to row n from its plane sums */
  __device__ static float fin(const Acc &r, const Frag &f, int g, float2 xs, int e) {
    const uint4 h = f.h;
    const gq_i32x4 c0 = r.c0, c1 = r.c1;
    /* 6-bit (scale, min) of sub-blocks 2g, 2g+1 (quant_matvec_q4_k.c:47-56),
     * both at once in bytes 0 and 1 of S and M, as in Tr<GQ_Q4_K>::dot */
    const uint32_t sh = 16u * (uint32_t)(g & 1);
    const bool hi = g >= 2;
    const uint32_t y = h.y >> sh, zz = h.z >> sh, w = h.w >> sh;
    const uint32_t mlo = hi ? 0x0f0fu : 0x3f3fu, mhi = hi ? 0x3030u : 0u;
    const uint32_t S = ((hi ? w : y) & mlo) | ((y >> 2) & mhi);
    const uint32_t Mm = ((hi ? (w >> 4) : zz) & mlo) | ((zz >> 2) & mhi);
    const float d = gq_h2f(h.x), dm = gq_h2f(h.x >> 16);
    const float s0 = __builtin_fmaf(65536.f, (float)c0.z, __builtin_fmaf(256.f, (float)c0.y, (float)c0.x));
    const float s1 = __builtin_fmaf(65536.f, (float)c1.z, __builtin_fmaf(256.f, (float)c1.y, (float)c1.x));
    float t = (d * (float)(S & 0xffu)) * s0;
    t = __builtin_fmaf(d * (float)((S >> 8) & 0xffu), s1, t);
    float r2 = __builtin_amdgcn_ldexpf(t, -e);
    r2 = __builtin_fmaf(-(dm * (float)(Mm & 0xffu)), xs.x, r2);
    r2 = __builtin_fmaf(-(dm * (float)((Mm >> 8) & 0xffu)), xs.y, r2);
    return r2;
  }
  /* sums of sub-blocks 2g, 2g+1 of block ai among the wave's sums at sw */
  __device__ static float2 xsums(const GQ_LDS uint8_t *lds, uint32_t sw, int ai, int g) {
    return lld<float2>(lds, sw + 4u * (8 * ai + 2 * g));
  }
};


/* Q6_K block for a 16-row tile (quant_matvec_q6_k.c:62-95: half h = 0, 1 of
 * 128 weights; for l < 32, weight 128h + l + 32i takes the low (i = 0, 1)
 * or high (i = 2, 3) nibble of ql[64h + l + 32(i & 1)] and bits 2i, 2i+1 of
 * qh[32h + l], minus 32, scale sc[8h + 2i + l / 16]).  Lane (row n, k-group
 * g) takes h = g / 2, l = 16 (g & 1) .. +15: MFMA j covers weights
 * 128h + 32j + l, one 16-weight sub-block (8h + 2j + (g & 1)) each, into a
 * C set of its own.  In the tile-interleaved layout the block's chunks are
 * ql 0..7, qh 8..11, scales 12, and the 16 rows' d at 13 * 256 + 2n. */
struct MmQ6K {
  static constexpr int BB = 210, SBW = 16, NA = 4;
  __device__ static uint32_t aoff(int g, int j) { return 128u * (g >> 1) + 32u * j + 16u * (g & 1); }
  struct Frag {
    uint4 a, b, h, sc;
    uint32_t d;
  };
  __device__ static void load(Frag &f, const GQ_LDS uint8_t *blk, int n, int g) {
    const int h = g >> 1, o = g & 1;
    f.a = lld<uint4>(blk, 256 * (4 * h + o) + 16 * n);
    f.b = lld<uint4>(blk, 256 * (4 * h + 2 + o) + 16 * n);
    f.h = lld<uint4>(blk, 256 * (8 + 2 * h + o) + 16 * n);
    f.sc = lld<uint4>(blk, 256 * 12 + 16 * n);
    f.d = lld<uint16_t>(blk, 256 * 13 + 2 * n);
  }
  struct Acc {
    gq_i32x4 c[4];
  };
  __device__ static void mma(Acc &r, const Frag &f, const gq_i32x4 (&A)[NA]) {
    const uint32_t A4[4] = {f.a.x, f.a.y, f.a.z, f.a.w}, B4[4] = {f.b.x, f.b.y, f.b.z, f.b.w};
    const uint32_t H4[4] = {f.h.x, f.h.y, f.h.z, f.h.w};
    int u[4][4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t M = 0x0f0f0f0fu, Q = 0x30303030u;
      u[0][k] = (int)((A4[k] & M) | ((H4[k] << 4) & Q));
      u[1][k] = (int)((B4[k] & M) | ((H4[k] << 2) & Q));
      u[2][k] = (int)(((A4[k] >> 4) & M) | (H4[k] & Q));
      u[3][k] = (int)(((B4[k] >> 4) & M) | ((H4[k] >> 2) & Q));
    }
    const gq_i32x4 z = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const gq_i32x4 b = {u[j][0], u[j][1], u[j][2], u[j][3]};
      r.c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[j], b, z, 0, 0, 0);
    }
  }
  __device__ static float fin(const Acc &r, const Frag &f, int g, float4 xs, int e) {
    /* scales sc[8h + 2j + (g & 1)], j = 0..3: bytes (g & 1) + 2j of the
     * half's 8 (dwords 2h, 2h + 1 of the 16 scale bytes) */
    const uint32_t s0 = (g >> 1) ? f.sc.z : f.sc.x, s1 = (g >> 1) ? f.sc.w : f.sc.y;
    const uint32_t sh = 8u * (uint32_t)(g & 1);
    const float xsj[4] = {xs.x, xs.y, xs.z, xs.w};
    const uint32_t sw[4] = {s0 >> sh, s0 >> (sh + 16), s1 >> sh, s1 >> (sh + 16)};
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const gq_i32x4 c = r.c[j];
      const float sj = __builtin_fmaf(65536.f, (float)c.z, __builtin_fmaf(256.f, (float)c.y, (float)c.x));
      /* sum (u - 32) x = sum u x - 32 sum x */
      const float v = __builtin_fmaf(-32.f, xsj[j], __builtin_amdgcn_ldexpf(sj, -e));
      t = __builtin_fmaf((float)(int8_t)(sw[j] & 0xffu), v, t);
    }
    return gq_h2f(f.d) * t;
  }
  /* sums of sub-blocks 8h + (g & 1) + 2j, j = 0..3, of block ai */
  __device__ static float4 xsums(const GQ_LDS uint8_t *lds, uint32_t sw, int ai, int g) {
    const uint32_t o = sw + 4u * (16 * ai + 8 * (g >> 1));
    const float4 p = lld<float4>(lds, o), q = lld<float4>(lds, o + 16);
    return (g & 1) ? make_float4(p.y, p.w, q.y, q.w) : make_float4(p.x, p.z, q.x, q.z);
  }
};

template <int DT>
struct MmTr;
template <>
struct MmTr<GQ_Q4_K> {
  using type = MmQ4K;
  typedef float2 XS;
};
template <>
struct MmTr<GQ_Q6_K> {
  using type = MmQ6K;
  typedef float4 XS;
};

/* This wave's DMA instructions for stage (tile t, chunk c): cb blocks of
 * the tile-interleaved tensor, one contiguous range (16 * BB * cb bytes)
 * into ring slot `buf` in 1 KB instructions; for MV_RESID with c == 0 also
 * the tile's residual values into rbuf.  Returns their count. */
template <int MODE, int NW, int BB>
__device__ __forceinline__ int mm_issue(const MvArgs &a, const MmPlan &pl, int t, int c, GQ_LDS uint8_t *buf,
                                        GQ_LDS float *rbuf, int wave, int lane) {
  const int sb = 16 * BB * pl.cb;
  copy_range(a.mm + ((size_t)t * pl.nb + (size_t)c * pl.cb) * (16 * BB), sb, buf, wave, lane, NW);
  int cnt = copy_count(sb, wave, NW);
  if (MODE == MV_RESID && c == 0 && wave == NW - 1) {
    int s, lr0;
    locate(a, 16 * t, s, lr0);
    const int last = a.seg[s].rows - 1;
    const uint32_t d = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)rbuf);
    if (lane < 16) dma4(a.seg[s].r + min(lr0 + lane, last), d);
    cnt++;
  }
  return cnt;
}

/* AREG: the wave's A operands live in registers for the whole launch (up to
 * MAXB blocks, every chunk); otherwise the digit planes stay in LDS (up to
 * 8 blocks per wave) and each stage loads the A operands of its MAXB
 * blocks per wave, for rows longer than registers hold. */
template <int DT, int MODE, int NW, int MAXB, int NS, bool AREG>
__global__ __launch_bounds__(NW * GQ_WAVE) void mvm_kernel(MvArgs a, MmPlan pl) {
  using T = typename MmTr<DT>::type;
  static_assert(NS >= 3, "ring of NS stage slots, NS - 1 stages in flight");
  constexpr int MAXT = AREG ? MAXB : 8; /* blocks a wave converts */
  __shared__ MmShared<NW> sh;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  GQ_LDS uint8_t *lds = (GQ_LDS uint8_t *)smem;
  GQ_LDS float *lres = (GQ_LDS float *)&sh.rres[0][0];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int bid = blockIdx.x, nblk = gridDim.x;
  const int mytiles = bid < pl.ntiles ? (pl.ntiles - 1 - bid) / nblk + 1 : 0;
  const int nst = mytiles * pl.nch;
  auto issue = [&](int q) -> int { /* stage q into slot q % NS */
    const int tl = q / pl.nch;
    return mm_issue<MODE, NW, T::BB>(a, pl, bid + tl * nblk, q - tl * pl.nch, lds + (q % NS) * pl.stride,
                                     lres + (tl % kRing) * 16, wave, lane);
  };

  /* This wave's blocks: ti = c * bpc + s is block c*cb + wave + s*NW.  Its
   * slices of x (and of the norm weight) go by DMA to the wave's own area
   * in the last pl.xslots ring slots, ahead of the stages whose slots they
   * leave free; each wave converts its own blocks, so the prologue has no
   * barrier (the RMSNorm sum of squares crosses the loop's first one,
   * before which no stage lands in those slots). */
  uint32_t valid = 0;
  int blk[MAXT];
#pragma unroll
  for (int ti = 0; ti < MAXT; ti++) {
    const int c = ti / pl.bpc, s = ti - c * pl.bpc;
    const int bl = wave + s * NW;
    blk[ti] = c * pl.cb + bl;
    if (c < pl.nch && bl < pl.cb) valid |= 1u << ti;
  }
  const bool norm = a.norm_w != nullptr;
  /* digit planes: AREG, over the wave's x slice of each block once it is
   * read (768 <= 1024 bytes per block); else in their own region */
  const uint32_t xw = pl.xs + wave * pl.xwb, pw = AREG ? xw : pl.planes + wave * pl.pwb;
  const uint32_t sw = pl.xsum + wave * pl.swb, ew = pl.eb + wave * 4 * MAXT;
#pragma unroll
  for (int ti = 0; ti < MAXT; ti++) {
    if (!(valid >> ti & 1u)) continue;
    const uint32_t base = (uint32_t)(uintptr_t)lds;
    dma16(a.x + 256 * blk[ti] + 4 * lane, __builtin_amdgcn_readfirstlane(base + xw + 1024u * ti));
    if (norm)
      dma16(a.norm_w + 256 * blk[ti] + 4 * lane, __builtin_amdgcn_readfirstlane(base + xw + 1024u * (MAXT + ti)));
  }
  int pos = 0;
  if (MODE == MV_STORE && a.rope.cs) {
    pos = a.rope.pos_dev ? gq_sld<int>(a.rope.pos_dev) : a.rope.pos;
    const int hd = a.rope.head_dim;
    if (wave == 0 && pos >= 0 && pos < a.rope.max_seq) {
      const float *crow = (const float *)(a.rope.cs + (size_t)pos * (hd >> 1));
      const uint32_t b = (uint32_t)(uintptr_t)(GQ_LDS float2 *)sh.scs;
      for (int o = 0; o < hd; o += 64)
        if (lane < hd - o) dma4(crow + o + lane, __builtin_amdgcn_readfirstlane(b + 4u * o));
    }
  }
  /* cnt[j]: this wave's DMA instructions of stage k + j at the top of
   * iteration k, j = 0 .. NS-2; stages npre .. NS-2 land in x's slots and go
   * out after the loop's first barrier */
  int cnt[NS - 1];
  const int npre = NS - pl.xslots;
  int issued = 0, sum = 0;
#pragma unroll
  for (int j = 0; j < NS - 1; j++) {
    cnt[j] = 0;
    if (j < npre && j < nst) cnt[j] = issue(j), issued = j + 1;
    sum += cnt[j];
  }
  /* VMEM loads complete in issue order: with only the stages' copies
   * outstanding, this wave's x slices have landed */
  wait_vmcnt(sum);
  int E[MAXT];
  float ss = mm_wave_x<T::SBW, MAXT>(lds, xw, pw, sw, valid, norm, lane, E);
  ss = gq_wave_total(ss);
  if (lane == 0) sh.red_ss[wave] = ss;
  /* AREG: A operands (x digit planes), sub-block sums and exponents stay in
   * registers for the whole launch (the wave's LDS writes above are ordered
   * before these reads); else the exponents go to LDS beside the sums */
  gq_i32x4 A[AREG ? MAXB : 1][T::NA];
  typename MmTr<DT>::XS X[AREG ? MAXB : 1];
  const bool nz = (n >> 2) == g && (n & 3) < 3;
  if constexpr (AREG) {
#pragma unroll
    for (int ai = 0; ai < MAXB; ai++) {
      const uint32_t po = pw + 768u * ai + 256u * (uint32_t)(n & 3);
#pragma unroll
      for (int j = 0; j < T::NA; j++) {
        gq_i32x4 v = {0, 0, 0, 0};
        if (nz && (valid >> ai & 1u)) v = lld<gq_i32x4>(lds, po + T::aoff(g, j));
        A[ai][j] = v;
      }
      X[ai] = T::xsums(lds, sw, (valid >> ai & 1u) ? ai : 0, g);
    }
  } else if (lane == 0) {
#pragma unroll
    for (int ti = 0; ti < MAXT; ti++) lst<int>(lds, ew + 4 * ti, E[ti]);
  }
  float rscale = 1.f;
  bool have_rscale = !norm;

  /* Iteration k: wait for stage k, one barrier (stage k landed for every
   * wave, and every wave is done with stage k-1, whose slot stage k+NS-1
   * then takes), finish the tile completed at k-1 into the parking area,
   * compute stage k.  Outputs are stored after the loop: a store inside it
   * would hold up the next wait on the vector memory counter. */
  GQ_LDS float *park = (GQ_LDS float *)(lds + pl.park);
  const bool full = AREG && pl.nch == 1 && valid == (1u << MAXB) - 1u;
  constexpr int RPW = 16 / NW; /* rows of a finished tile each wave completes */
  float acc = 0.f;
  for (int k = 0; k <= nst; k++) {
    if (k < nst) {
      int pend = 0;
#pragma unroll
      for (int j = 1; j < NS - 1; j++) pend += cnt[j];
      wait_vmcnt(pend);
    }
    __syncthreads();
    /* stages up to k + NS - 1 (the first iteration also those x held back),
     * into the slots of stages already computed; issued after this stage's
     * LDS reads and MFMAs, so that the wait for room in the memory pipeline
     * overlaps the matrix cores instead of holding every wave at once */
    auto issue_ahead = [&]() {
#pragma unroll
      for (int j = 0; j < NS - 2; j++) cnt[j] = cnt[j + 1];
      cnt[NS - 2] = 0;
#pragma unroll
      for (int j = 1; j < NS; j++) {
        const int q = k + j;
        if (q < nst && q >= issued && j <= NS - 1) {
          cnt[j - 1] += issue(q);
          issued = q + 1;
        }
      }
    };
    const int c = k < nst ? k % pl.nch : 0;
    if (!have_rscale) { /* 1/sqrt(mean(x^2) + eps) (kernels_cpu.c:242-253) */
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < NW; w++) tot += sh.red_ss[w];
      tot = tot / (float)a.cols;
      tot = tot + a.eps;
      rscale = 1.0f / sqrtf(tot);
      have_rscale = true;
    }
    if (k > 0 && c == 0 && lane < RPW) { /* rows of the tile completed at k-1 */
      const int tl = (k - 1) / pl.nch, r = wave * RPW + lane;
      if (MODE != MV_SWIGLU || r < 8) {
        const int tp = MODE == MV_SWIGLU ? r + 8 : r ^ 1;
        float v = 0.f, w = 0.f;
#pragma unroll
        for (int j = 0; j < NW; j++) v += sh.red[tl & 1][r][j], w += sh.red[tl & 1][tp][j];
        v *= rscale, w *= rscale;
        float out = v;
        {
#pragma clang fp contract(off)
          if (MODE == MV_SWIGLU) {
            out = silu_mul(v, w);
          } else if (MODE == MV_RESID) {
            out = v + sh.rres[tl % kRing][r];
          } else if (a.rope.cs) {
            int s, lr0;
            locate(a, 16 * (bid + tl * nblk), s, lr0);
            const int kind = a.seg[s].kind;
            if (kind == SEG_ROPE || kind == SEG_ROPE_KV) {
              /* adjacent pair rotated by the row of pos
               * (kernels_cpu.c:415-429); tiles start on even rows */
              const int d = (lr0 + r) % a.rope.head_dim;
              const float2 cs = sh.scs[d >> 1];
              const float x0 = (r & 1) ? w : v, x1 = (r & 1) ? v : w;
              out = (r & 1) ? x0 * cs.y + x1 * cs.x : x0 * cs.x - x1 * cs.y;
            }
          }
        }
        park[16 * tl + r] = out;
      }
    }
    if (k == nst) break;
    /* every LDS read of the stage first, then every MFMA, then the copies of
     * the stages ahead, then the epilogues (the fast path when the launch
     * has one chunk and every block slot of the wave is used; uniform: all
     * waves take it) */
    const GQ_LDS uint8_t *buf = lds + (k % NS) * pl.stride;
    typename T::Frag f[MAXB];
    typename T::Acc r[MAXB];
    if constexpr (!AREG) {
      /* this stage's blocks of the wave: A operands, sums and exponents from
       * the planes in LDS */
#pragma unroll
      for (int ai = 0; ai < MAXB; ai++) {
        const int ti = c * pl.bpc + ai;
        if (ai >= pl.bpc || !(valid >> ti & 1u)) continue;
        gq_i32x4 Ab[T::NA];
        const uint32_t po = pw + 768u * ti + 256u * (uint32_t)(n & 3);
#pragma unroll
        for (int j = 0; j < T::NA; j++) {
          gq_i32x4 v = {0, 0, 0, 0};
          if (nz) v = lld<gq_i32x4>(lds, po + T::aoff(g, j));
          Ab[j] = v;
        }
        const int eb = __builtin_amdgcn_readfirstlane(lld<int>(lds, ew + 4 * ti));
        T::load(f[ai], buf + (blk[ti] - c * pl.cb) * (16 * T::BB), n, g);
        T::mma(r[ai], f[ai], Ab);
        acc += T::fin(r[ai], f[ai], g, T::xsums(lds, sw, ti, g), eb);
      }
      issue_ahead();
    } else if (full) {
#pragma unroll
      for (int ai = 0; ai < MAXB; ai++) T::load(f[ai], buf + blk[ai] * (16 * T::BB), n, g);
#pragma unroll
      for (int ai = 0; ai < MAXB; ai++) T::mma(r[ai], f[ai], A[ai]);
      issue_ahead();
#pragma unroll
      for (int ai = 0; ai < MAXB; ai++) acc += T::fin(r[ai], f[ai], g, X[ai], E[ai]);
    } else {
#pragma unroll
      for (int ai = 0; ai < MAXB; ai++)
        if (ai / pl.bpc == c && (valid >> ai & 1u)) T::load(f[ai], buf + (blk[ai] - c * pl.cb) * (16 * T::BB), n, g);
#pragma unroll
      for (int ai = 0; ai < MAXB; ai++)
        if (ai / pl.bpc == c && (valid >> ai & 1u)) T::mma(r[ai], f[ai], A[ai]);
      issue_ahead();
#pragma unroll
      for (int ai = 0; ai < MAXB; ai++)
        if (ai / pl.bpc == c && (valid >> ai & 1u)) acc += T::fin(r[ai], f[ai], g, X[ai], E[ai]);
    }
    if (c == pl.nch - 1) { /* the tile's last chunk: reduce over the k-groups */
      float v = acc;
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (lane < 16) sh.red[(k / pl.nch) & 1][lane][wave] = v;
      acc = 0.f;
    }
  }
  __syncthreads();
  /* the parked rows go out */
  const int prow = MODE == MV_SWIGLU ? 8 : 16;
  for (int i = threadIdx.x; i < mytiles * 16; i += NW * GQ_WAVE) {
    const int tl = i >> 4, r = i & 15, t = bid + tl * nblk;
    if (r >= prow) continue;
    int s = 0, lr = 8 * t + r;
    if (MODE != MV_SWIGLU) {
      locate(a, 16 * t, s, lr);
      lr += r;
      if (lr >= a.seg[s].rows) continue;
    } else if (lr >= pl.total) {
      continue;
    }
    float *dst = rdest<MODE>(a, s, lr, pos);
    if (dst) gst<float>(dst, park[i]);
  }
}

int g_n_cu = 256;
int g_wg_per_cu = 4;
constexpr size_t kMaxDynLds = 144 * 1024;
constexpr size_t kMaxDynLdsW = 152 * 1024;
/* matvec kernels: 0 register path, 1 split-K LDS, 2 wave-private LDS ring,
 * 3 register ring, 5 matrix cores (each where it fits, falling back down the
 * list), 4 auto */
int g_use_lds = 4;

template <int DT, int MODE, int R>
int launch_r(const MvArgs &a, int total, hipStream_t s) {
  constexpr int P = MODE == MV_SWIGLU ? R / 2 : R;
  const int ngroups = (total + kWaves * P - 1) / (kWaves * P);
  /* enough workgroups to fill every CU a few times over, never more than
   * there are row groups */
  const int grid = g_wg_per_cu > 0 ? min(ngroups, g_wg_per_cu * g_n_cu) : ngroups;
  const size_t lds = (size_t)a.cols * sizeof(float);
  hipLaunchKernelGGL((mv_kernel<DT, R, MODE>), dim3(grid), dim3(kThreads), lds, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

/* Plan the LDS-streamed kernel for traits T: stage rows, teams, LDS bytes
 * and workgroups per CU; false when the shape does not fit it (rows not a
 * multiple of 16 bytes, more than 8 column tiles, or segments that a stage
 * would straddle).  With xl, x (and the norm weight) are staged from slot 2
 * onwards, growing the LDS past the three slots when they need more. */
template <typename T, int MODE>
bool plan_lds(const MvArgs &a, int total, bool xl, int ns, MvPlan &pl, size_t &lds, int &per_cu, int &tpw,
              int &rw) {
  const int nb = a.cols / T::QK;
  const int rowbytes = nb * T::BB;
  if (rowbytes % 16) return false;
  if (a.rope.cs && a.rope.head_dim > 512) return false; /* the kernel's RoPE row holds 256 pairs */
  constexpr int BPT = GQ_WAVE / T::LPB;
  const int ntile = (nb + BPT - 1) / BPT;
  tpw = ntile <= kWaves ? 1 : 2;
  const int ts = (ntile + tpw - 1) / tpw;
  if (ts > kWaves) return false;
  const int nteam = kWaves / ts;
  /* rs: two rows per team at least, so a wave's step covers a RoPE pair */
  const int unit = 2 * nteam;
  int rs = min(32, g_stage_cap / rowbytes);
  rs -= rs % unit;
  /* with several segments a stage must not straddle two: rs divides them all */
  if (MODE != MV_SWIGLU && a.nseg > 1)
    for (int i = 0; i < a.nseg && rs >= unit;) {
      if (a.seg[i].rows % rs)
        rs -= unit, i = 0;
      else
        i++;
    }
  if (rs < unit || rs < 2) return false;
  pl.rs = rs, pl.ts = ts, pl.nteam = nteam, pl.ntile = ntile, pl.rowbytes = rowbytes, pl.total = total;
  pl.stride = (rs * rowbytes + 64 + 1023) / 1024 * 1024;
  const int per = MODE == MV_SWIGLU ? rs / 2 : rs;
  pl.ngroups = (total + per - 1) / per;
  lds = (size_t)ns * pl.stride;
  pl.xl = -1;
  if (xl) {
    pl.xl = (ns - 1) * pl.stride;
    lds = std::max(lds, (size_t)pl.xl + (size_t)a.cols * 4 * (a.norm_w ? 2 : 1));
  }
  if (lds > kMaxDynLds) return false;
  per_cu = max(1, (int)(160 * 1024 / (lds + 8192)));
  if (g_lds_wg_per_cu > 0) per_cu = min(per_cu, g_lds_wg_per_cu);
  /* rows per team per stage is even (rs is a multiple of 2 nteam) */
  rw = (rs / nteam) % 4 == 0 ? 4 : 2;
  return true;
}

template <int DT, int MODE, bool XL, int NS>
int launch_lds_as(const MvArgs &a, const MvPlan &pl, size_t lds, int per_cu, int tpw, int rw, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    const void *fs[] = {
        (const void *)mvl_kernel<DT, MODE, 1, 2, XL, NS>, (const void *)mvl_kernel<DT, MODE, 2, 2, XL, NS>,
        (const void *)mvl_kernel<DT, MODE, 1, 4, XL, NS>, (const void *)mvl_kernel<DT, MODE, 2, 4, XL, NS>};
    for (const void *f : fs) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds);
    attr_set = true;
  }
  const dim3 g(min(pl.ngroups, per_cu * g_n_cu)), b(kThreads);
  if (rw == 2 && tpw == 1) hipLaunchKernelGGL((mvl_kernel<DT, MODE, 1, 2, XL, NS>), g, b, lds, s, a, pl);
  if (rw == 2 && tpw == 2) hipLaunchKernelGGL((mvl_kernel<DT, MODE, 2, 2, XL, NS>), g, b, lds, s, a, pl);
  if (rw == 4 && tpw == 1) hipLaunchKernelGGL((mvl_kernel<DT, MODE, 1, 4, XL, NS>), g, b, lds, s, a, pl);
  if (rw == 4 && tpw == 2) hipLaunchKernelGGL((mvl_kernel<DT, MODE, 2, 4, XL, NS>), g, b, lds, s, a, pl);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int g_mv_xl = -1; /* x staged in LDS by the split-K kernel: -1 auto, 0 never, 1 whenever it fits */

/* Plan and launch the LDS-streamed kernel; returns 1 when the shape does not
 * fit it, so the caller uses mv_kernel.  x goes through LDS (the XL kernel)
 * when that costs no workgroup per CU (auto: gate/up, q/k/v, o at the 8B
 * shape measured 8-12% faster; the LM head, which would drop from three
 * workgroups per CU to two, 13% slower), else each wave loads its x slices
 * from global memory. */
template <int DT, int MODE>
int launch_lds(const MvArgs &a, int total, hipStream_t s) {
  MvPlan pl, px;
  size_t lds, lx;
  int per_cu, tpw, rw, pcx, tpx, rwx;
  const bool base = plan_lds<typename TrL<DT, false>::type, MODE>(a, total, false, kNS, pl, lds, per_cu, tpw, rw);
  if (g_mv_xl != 0 && plan_lds<typename TrL<DT, true>::type, MODE>(a, total, true, kNS, px, lx, pcx, tpx, rwx) &&
      (g_mv_xl == 1 || !base || pcx >= per_cu))
    return launch_lds_as<DT, MODE, true, kNS>(a, px, lx, pcx, tpx, rwx, s);
  if (!base) return 1;
  return launch_lds_as<DT, MODE, false, kNS>(a, pl, lds, per_cu, tpw, rw, s);
}

/* q/k (Q4_K) and v (Q6_K) in one launch; returns 1 when the shapes do not
 * fit the paired kernel (the caller launches them one by one) */
template <int RW0, int RW1>
int launch_pair_as(const MvArgs &a0, const MvPlan &p0, const MvArgs &a1, const MvPlan &p1, int g0, int g1, size_t lds,
                   hipStream_t s) {
  static bool attr_set = false;
  auto f = mvl_pair_kernel<GQ_Q4_K, 1, RW0, true, GQ_Q6_K, 1, RW1, true>;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLds);
    attr_set = true;
  }
  hipLaunchKernelGGL(f, dim3(g0 + g1), dim3(kThreads), lds, s, a0, p0, a1, p1, g0);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

int g_mw_rw = 4;   /* rows per group of the wave-private kernel */
int g_mw_waves = 0; /* waves per workgroup of the wave-private kernel (0: chosen per shape) */
int g_mw_pre = -1;  /* groups issued before x is waited for (-1: all ns-1) */

template <int DT, int MODE, int TPW>
int launch_w_rw(int rw, const MvArgs &a, const MwPlan &pl, int grid, int nwv, size_t lds, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    const void *fs[] = {(const void *)mvw_kernel<DT, MODE, TPW, 2>, (const void *)mvw_kernel<DT, MODE, TPW, 4>};
    for (const void *f : fs) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLdsW);
    attr_set = true;
  }
  const dim3 g(grid), b(nwv * GQ_WAVE);
  if (rw == 4) hipLaunchKernelGGL((mvw_kernel<DT, MODE, TPW, 4>), g, b, lds, s, a, pl);
  else hipLaunchKernelGGL((mvw_kernel<DT, MODE, TPW, 2>), g, b, lds, s, a, pl);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

/* Plan and launch the wave-private kernel; returns 1 when the shape does not
 * fit it (more than two column tiles, rows not a multiple of 16 bytes,
 * segments that a group would straddle, or too little LDS). */
template <int DT, int MODE>
int launch_w(const MvArgs &a, int total, hipStream_t s) {
  using T = Tr<DT>;
  const int nb = a.cols / T::QK;
  const int rowbytes = nb * T::BB;
  if (rowbytes % 16) return 1;
  constexpr int BPT = GQ_WAVE / T::LPB;
  const int ntile = (nb + BPT - 1) / BPT;
  if (ntile > 2) return 1;
  bool rope = false;
  if (MODE == MV_STORE)
    for (int i = 0; i < a.nseg; i++) rope = rope || a.seg[i].kind != SEG_PLAIN;
  if (rope && a.rope.head_dim > 512) return 1; /* the kernel's RoPE row holds 256 pairs */
  const int rw = g_mw_rw >= 4 ? 4 : 2; /* even: RoPE pairs rows (2i, 2i+1) inside a group */
  if (MODE != MV_SWIGLU && a.nseg > 1)
    for (int i = 0; i < a.nseg; i++)
      if (a.seg[i].rows % rw) return 1;
  MwPlan pl;
  pl.rowbytes = rowbytes;
  pl.total = total;
  const int per = MODE == MV_SWIGLU ? rw / 2 : rw;
  pl.ngroups = (total + per - 1) / per;
  pl.slot = (rw * rowbytes + 64 + 255) / 256 * 256;
  const int xneed = a.cols * 4 * (a.norm_w ? 2 : 1); /* staged in the last slot row */
  /* waves per workgroup: 4 (or the override), as many ring slots as LDS
   * holds (at most kMaxNS), the last slot row large enough for x */
  int nwv = g_mw_waves > 0 ? std::min(g_mw_waves, kMaxWaves) : 4;
  while (nwv < kMaxWaves && nwv * pl.slot < xneed) nwv *= 2;
  const int ns = std::min(kMaxNS, (int)(kMaxDynLdsW / ((size_t)nwv * pl.slot)));
  if (ns < 3 || nwv * pl.slot < xneed) return 1;
  pl.ns = ns;
  pl.pre = g_mw_pre < 0 ? ns - 1 : g_mw_pre;
  pl.x_off = (ns - 1) * nwv * pl.slot;
  pl.nw_off = pl.x_off + a.cols * 4;
  const size_t lds = (size_t)ns * nwv * pl.slot;
  const int per_cu = std::max(1, (int)((160 * 1024) / (lds + 4096)));
  const int grid = std::min((pl.ngroups + nwv - 1) / nwv, per_cu * g_n_cu);
  if (ntile == 1) return launch_w_rw<DT, MODE, 1>(rw, a, pl, grid, nwv, lds, s);
  return launch_w_rw<DT, MODE, 2>(rw, a, pl, grid, nwv, lds, s);
}

/* Plan and launch the register-ring kernel; returns 1 when the shape does
 * not fit it (more than one column tile: the two-tile ring does not fit the
 * register file; or segments a group would straddle). */
template <int DT, int MODE>
int launch_reg(const MvArgs &a, int total, hipStream_t s) {
  using T = Tr<DT>;
  const int nb = a.cols / T::QK;
  constexpr int BPT = GQ_WAVE / T::LPB;
  const int ntile = (nb + BPT - 1) / BPT;
  if (ntile > 1) return 1;
  /* 4 rows per group when that still gives every wave of a full grid work
   * (and the loads of 3 groups fit the 63 outstanding loads), else 2 */
  const int nw = 8;
  const int per4 = MODE == MV_SWIGLU ? 2 : 4;
  int rw = (total + per4 - 1) / per4 >= 2 * nw * g_n_cu ? 4 : 2;
  if (g_mw_rw == 2) rw = 2;
  if (MODE != MV_SWIGLU && a.nseg > 1)
    for (int i = 0; i < a.nseg; i++)
      if (a.seg[i].rows % rw) return 1;
  MwPlan pl;
  pl.rowbytes = nb * T::BB;
  pl.total = total;
  const int per = MODE == MV_SWIGLU ? rw / 2 : rw;
  pl.ngroups = (total + per - 1) / per;
  const int grid = std::min((pl.ngroups + nw - 1) / nw, g_n_cu);
  const int mg = (pl.ngroups + grid * nw - 1) / (grid * nw); /* groups per wave, at most */
  const int xb = (a.cols * 4 + 255) / 256 * 256;
  pl.nw_off = xb;
  pl.x_off = xb * (a.norm_w ? 2 : 1); /* parked outputs after x and the norm weight */
  pl.slot = mg + 2;                    /* parked groups per wave (+ the unrolled tail) */
  pl.ns = 0, pl.pre = 0;
  const size_t lds = (size_t)pl.x_off + (size_t)nw * pl.slot * per * 4;
  if (lds > kMaxDynLdsW) return 1;
  static bool attr_set = false;
  if (!attr_set) {
    const void *fs[] = {(const void *)mvr_kernel<DT, MODE, 1, 2>, (const void *)mvr_kernel<DT, MODE, 1, 4>};
    for (const void *f : fs) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLdsW);
    attr_set = true;
  }
  const dim3 g(grid), b(nw * GQ_WAVE);
  if (rw == 2) hipLaunchKernelGGL((mvr_kernel<DT, MODE, 1, 2>), g, b, lds, s, a, pl);
  else hipLaunchKernelGGL((mvr_kernel<DT, MODE, 1, 4>), g, b, lds, s, a, pl);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

/* Plan and launch the matrix-core kernel; returns 1 when the shape does not
 * fit it (a dtype without int8 traits, segments a 16-row tile would
 * straddle, rows not a multiple of 16 bytes, or x not fitting the ring's
 * last slot during the prologue). */
int g_mm_waves = 8;          /* waves per workgroup: 4 or 8 */
constexpr size_t kMmLds = 160 * 1024; /* LDS of a CU (gfx950) */
int g_mm_ns = 3;             /* ring slots: 3, 4 or 6 */
int g_mm_stage_cap = 40960;  /* bytes of weights per stage at most */

template <int DT, int MODE, int NW, int MAXB, int NS, bool AREG = true>
int launch_mm_as(const MvArgs &a, const MmPlan &pl, size_t lds, int grid, hipStream_t s) {
  static bool attr_set = false;
  auto f = mvm_kernel<DT, MODE, NW, MAXB, NS, AREG>;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLdsW);
    (void)hipGetLastError(); /* a refusal shows up as the launch's error instead */
    attr_set = true;
  }
  hipLaunchKernelGGL(f, dim3(grid), dim3(NW * GQ_WAVE), lds, s, a, pl);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <int DT, int MODE, int NW, int NS>
int launch_mm_b(int maxb, bool areg, const MvArgs &a, const MmPlan &pl, size_t lds, int grid, hipStream_t s) {
  if (!areg) return pl.bpc <= 1 ? launch_mm_as<DT, MODE, NW, 1, NS, false>(a, pl, lds, grid, s)
                                : launch_mm_as<DT, MODE, NW, 2, NS, false>(a, pl, lds, grid, s);
  if (maxb <= 1) return launch_mm_as<DT, MODE, NW, 1, NS>(a, pl, lds, grid, s);
  if (maxb <= 2) return launch_mm_as<DT, MODE, NW, 2, NS>(a, pl, lds, grid, s);
  return launch_mm_as<DT, MODE, NW, 4, NS>(a, pl, lds, grid, s);
}

template <int DT, int MODE, int NW>
int launch_mm_w(const MvArgs &a, int total, hipStream_t s) {
  using T = typename MmTr<DT>::type;
  MmPlan pl;
  pl.nb = a.cols / 256;
  pl.rowbytes = pl.nb * T::BB;
  if (MODE == MV_STORE && a.rope.cs && a.rope.head_dim > 512) return 1; /* the RoPE row holds 256 pairs */
  if (MODE != MV_SWIGLU && a.nseg > 1)
    for (int i = 0; i < a.nseg; i++)
      if (a.seg[i].rows % 16) return 1;
  /* blocks per stage: the whole row when 16 rows fit the cap, else the
   * largest divisor of the row's blocks that fits */
  int cb = pl.nb;
  while (cb > 1 && (16 * cb * T::BB > g_mm_stage_cap || pl.nb % cb)) cb--;
  pl.cb = cb;
  pl.crb = cb * T::BB;
  pl.nch = pl.nb / cb;
  pl.bpc = (cb + NW - 1) / NW;
  const int maxb = pl.nch * pl.bpc;
  /* up to four blocks per wave keep their A operands in registers (eight
   * spill); up to eight keep their planes in LDS, two per stage */
  const bool areg = maxb <= 4;
  if (!areg && (maxb > 8 || pl.bpc > 2)) return 1;
  const int mt = areg ? (maxb <= 1 ? 1 : maxb <= 2 ? 2 : 4) : 8; /* the kernel's MAXT */
  pl.stride = (16 * pl.crb + 255) / 256 * 256;
  /* the waves' x slices in the ring's last slots; after the ring their
   * sub-block sums, (without AREG) their digit planes and exponents, then
   * the parked outputs */
  pl.xwb = 1024 * mt * (a.norm_w ? 2 : 1);
  pl.xslots = (NW * pl.xwb + pl.stride - 1) / pl.stride;
  int ns = std::max(g_mm_ns >= 6 ? 6 : g_mm_ns == 4 ? 4 : 3, pl.xslots + 1);
  if (ns == 5) ns = 6; /* the kernels are built for 3, 4 and 6 slots */
  if (ns > 6) return 1;
  pl.ns = ns;
  pl.xs = (ns - pl.xslots) * pl.stride;
  pl.swb = 4 * (areg ? mt : maxb) * (256 / T::SBW);
  pl.xsum = ns * pl.stride;
  pl.pwb = areg ? 0 : 768 * maxb;
  pl.planes = pl.xsum + NW * pl.swb;
  pl.eb = pl.planes + NW * pl.pwb;
  pl.park = pl.eb + NW * 4 * mt;
  pl.total = total;
  pl.ntiles = MODE == MV_SWIGLU ? (total + 7) / 8 : (total + 15) / 16;
  /* workgroups per CU from LDS, then the grid; the parking area holds
   * every tile a workgroup finishes */
  const size_t shb = sizeof(MmShared<NW>);
  int grid = 0;
  size_t lds = 0;
  for (int pc = 2; pc >= 1 && !grid; pc--) {
    const int gr = std::min(pl.ntiles, pc * g_n_cu);
    const size_t l = (size_t)pl.park + 64 * (size_t)((pl.ntiles + gr - 1) / gr);
    if (l <= kMaxDynLdsW && pc * (l + shb + 1024) <= kMmLds + 1024) grid = gr, lds = l;
  }
  if (!grid) return 1;
  if (ns == 3) return launch_mm_b<DT, MODE, NW, 3>(maxb, areg, a, pl, lds, grid, s);
  if (ns == 4) return launch_mm_b<DT, MODE, NW, 4>(maxb, areg, a, pl, lds, grid, s);
  return launch_mm_b<DT, MODE, NW, 6>(maxb, areg, a, pl, lds, grid, s);
}

template <int DT, int MODE>
int launch_mm(const MvArgs &a, int total, hipStream_t s) {
  if constexpr (DT != GQ_Q4_K && DT != GQ_Q6_K) {
    return 1;
  } else {
    if (!a.mm) return 1;
    return g_mm_waves >= 8 ? launch_mm_w<DT, MODE, 8>(a, total, s) : launch_mm_w<DT, MODE, 4>(a, total, s);
  }
}

/* ---------------------------------------------------------------- tiling */
__global__ void mm_tile_kernel(uint8_t *dst, const uint8_t *w0, const uint8_t *w1, int rows, int nb, int bb,
                               long long units) {
  /* one thread per (tile, block, row n) */
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= units) return;
  const int n = (int)(i & 15);
  const long long tb = i >> 4, tile = tb / nb;
  const int b = (int)(tb - tile * nb);
  const uint8_t *src;
  int row;
  if (w1) {
    row = 8 * (int)tile + (n & 7);
    src = n < 8 ? w0 : w1;
  } else {
    row = 16 * (int)tile + n;
    src = w0;
  }
  uint8_t *out = dst + (size_t)tb * 16 * bb;
  const uint16_t *in = (const uint16_t *)(src + ((size_t)row * nb + b) * bb); /* blocks are 2-byte aligned */
  const bool ok = row < rows;
  for (int o = 0; o < bb; o += 2) {
    const uint16_t v = ok ? in[o >> 1] : (uint16_t)0;
    const int at = o < 208 ? (o >> 4) * 256 + 16 * n + (o & 15) : 13 * 256 + 2 * n + (o - 208);
    *(uint16_t *)(out + at) = v;
  }
}

template <int DT, int MODE>
int launch_dm(const MvArgs &a, hipStream_t s) {
  int total = 0;
  if (MODE == MV_SWIGLU) {
    if (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows) return -1;
    total = a.seg[0].rows;
  } else {
    bool fused = false;
    for (int i = 0; i < a.nseg; i++) {
      if (a.seg[i].kind != SEG_PLAIN) {
        fused = true;
        if (MODE != MV_STORE || !a.rope.cs || a.rope.head_dim <= 0 || (a.rope.head_dim & 1) ||
            a.seg[i].rows % a.rope.head_dim)
          return -1;
      }
      total += a.seg[i].rows;
    }
    /* fused RoPE pairs rows inside a wave: every segment must start on a wave
     * boundary */
    if (fused)
      for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].rows % 4) return -1;
  }
  if (total <= 0) return -1;
  /* the matrix-core kernel: selected explicitly (5), or by auto (4) for the
   * launches it measured faster on: gate/up + SwiGLU and the LM head (8B
   * shape: 16.1 vs 20.3 us and 88 vs 108 us); the split-K kernel stays
   * faster for q/k/v (10.0 vs 12.1 us), o and down */
  if (g_use_lds == 5 || (g_use_lds == 4 && (MODE == MV_SWIGLU || (MODE == MV_STORE && total >= 16384)))) {
    const int rc = launch_mm<DT, MODE>(a, total, s);
    if (rc <= 0) return rc;
  }
  if (g_use_lds == 3) {
    const int rc = launch_reg<DT, MODE>(a, total, s);
    if (rc <= 0) return rc;
  }
  /* auto: the split-K kernel for every op (the wave-private ring is selected
   * explicitly; it measured 5% slower than split-K for gate/up in the 8B
   * decode step) */
  if (g_use_lds == 2 || g_use_lds == 3) {
    const int rc = launch_w<DT, MODE>(a, total, s);
    if (rc <= 0) return rc;
  }
  if (g_use_lds) {
    const int rc = launch_lds<DT, MODE>(a, total, s);
    if (rc <= 0) return rc;
  }
  return launch_r<DT, MODE, 4>(a, total, s);
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

void gq_matvec_set_cus(int n_cu) {
  if (n_cu > 0) g_n_cu = n_cu;
  static bool env_read = false;
  if (env_read) return;
  env_read = true;
  /* GQ_MV_WG_PER_CU: workgroups per CU of the register-path kernel's
   * persistent grid (0 = one workgroup per row group); default 4 */
  if (const char *e = getenv("GQ_MV_WG_PER_CU")) g_wg_per_cu = atoi(e);
  /* GQ_MV_LDS=0: register-path kernel only (same as gq_hip_set_matvec_path(0)) */
  if (const char *e = getenv("GQ_MV_LDS")) g_use_lds = std::min(std::max(atoi(e), 0), 5);
  /* wave-private kernel: rows per group (GQ_MV_RW, 2 or 4) and waves per
   * workgroup (GQ_MV_WAVES, 4..16; 0 = chosen per shape) */
  if (const char *e = getenv("GQ_MV_RW")) g_mw_rw = atoi(e) >= 4 ? 4 : 2;
  if (const char *e = getenv("GQ_MV_WAVES")) g_mw_waves = std::max(atoi(e), 0);
  /* GQ_MV_XPRE: groups each wave issues before x is waited for (-1 = all) */
  if (const char *e = getenv("GQ_MV_XPRE")) g_mw_pre = atoi(e);
  /* LDS-streamed kernel: bytes of weights per stage (GQ_MV_STAGE_BYTES, at
   * most 40 KB) and workgroups per CU (GQ_MV_LDS_WG, 0 = as many as LDS
   * allows) */
  if (const char *e = getenv("GQ_MV_STAGE_BYTES")) g_stage_cap = std::min(std::max(atoi(e), 4096), 40960);
  if (const char *e = getenv("GQ_MV_LDS_WG")) g_lds_wg_per_cu = std::max(atoi(e), 0);
  /* GQ_MV_XL: x through LDS in the split-K kernel (-1 auto, 0 never, 1 when it fits) */
  if (const char *e = getenv("GQ_MV_XL")) g_mv_xl = std::min(std::max(atoi(e), -1), 1);
  /* matrix-core kernel: waves per workgroup (GQ_MM_WAVES, 4 or 8), ring
   * slots (GQ_MM_NS, 3, 4 or 6) and bytes of weights per stage
   * (GQ_MM_STAGE_BYTES, at most 64 KB) */
  if (const char *e = getenv("GQ_MM_WAVES")) g_mm_waves = atoi(e) >= 8 ? 8 : 4;
  if (const char *e = getenv("GQ_MM_NS")) g_mm_ns = atoi(e);
  if (const char *e = getenv("GQ_MM_STAGE_BYTES")) g_mm_stage_cap = std::min(std::max(atoi(e), 2048), 65536);
}

bool gq_matvec_mm_enabled() { return g_use_lds == 5; }  /* every launch with a tiled copy */
bool gq_matvec_mm_forced() { return g_use_lds == 5; }

size_t gq_mm_tile_bytes(int dtype, int rows, int cols, bool swiglu) {
  const int bb = dtype == GQ_Q4_K ? 144 : dtype == GQ_Q6_K ? 210 : 0;
  if (!bb || cols % 256) return 0;
  const size_t tiles = swiglu ? (rows + 7) / 8 : (rows + 15) / 16;
  return tiles * (cols / 256) * 16 * bb;
}

int gq_launch_mm_tile(void *dst, int dtype, const void *w0, const void *w1, int rows, int cols, hipStream_t s) {
  const int bb = dtype == GQ_Q4_K ? 144 : dtype == GQ_Q6_K ? 210 : 0;
  if (!bb || !dst || !w0 || rows <= 0 || cols <= 0 || cols % 256) return -1;
  const int nb = cols / 256;
  const long long tiles = w1 ? (rows + 7) / 8 : (rows + 15) / 16;
  const long long units = tiles * nb * 16;
  hipLaunchKernelGGL(mm_tile_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, s, (uint8_t *)dst,
                     (const uint8_t *)w0, (const uint8_t *)w1, rows, nb, bb, units);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

extern "C" int gq_hip_set_matvec_path(int path) {
  const int prev = g_use_lds;
  if (path >= 0 && path <= 5) g_use_lds = path;
  return prev;
}

int gq_launch_matvec_pair(int dt0, const MvArgs &a0, int dt1, const MvArgs &a1, hipStream_t s) {
  if (g_use_lds != 4 || g_mv_xl == 0 || dt0 != GQ_Q4_K || dt1 != GQ_Q6_K) return 1;
  const MvArgs *as[2] = {&a0, &a1};
  int totals[2];
  for (int k = 0; k < 2; k++) {
    const MvArgs &a = *as[k];
    if (a.nseg < 1 || a.nseg > 3 || a.cols <= 0 || a.cols > 16384 || a.cols % 256) return 1;
    int total = 0;
    bool fused = false;
    for (int i = 0; i < a.nseg; i++) {
      if (a.seg[i].kind != SEG_PLAIN) {
        fused = true;
        if (!a.rope.cs || a.rope.head_dim <= 0 || (a.rope.head_dim & 1) || a.seg[i].rows % a.rope.head_dim)
          return 1;
      }
      total += a.seg[i].rows;
    }
    if (fused)
      for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].rows % 4) return 1;
    if (total <= 0) return 1;
    totals[k] = total;
  }
  MvPlan p0, p1;
  size_t l0, l1;
  int c0, c1, t0, t1, r0, r1;
  if (!plan_lds<typename TrL<GQ_Q4_K, true>::type, MV_STORE>(a0, totals[0], true, kNS, p0, l0, c0, t0, r0) ||
      !plan_lds<typename TrL<GQ_Q6_K, true>::type, MV_STORE>(a1, totals[1], true, kNS, p1, l1, c1, t1, r1))
    return 1;
  if (t0 != 1 || t1 != 1) return 1;
  const size_t lds = std::max(l0, l1);
  int per_cu = max(1, (int)(160 * 1024 / (lds + 8192)));
  if (g_lds_wg_per_cu > 0) per_cu = min(per_cu, g_lds_wg_per_cu);
  /* one resident wave of workgroups, split in proportion to the bytes */
  const int slots = per_cu * g_n_cu;
  const double b0 = (double)totals[0] * p0.rowbytes, b1 = (double)totals[1] * p1.rowbytes;
  int g1 = (int)(slots * b1 / (b0 + b1) + 0.5);
  g1 = min(max(g1, 1), p1.ngroups);
  const int g0 = min(max(slots - g1, 1), p0.ngroups);
  if (r0 == 2 && r1 == 2) return launch_pair_as<2, 2>(a0, p0, a1, p1, g0, g1, lds, s);
  if (r0 == 2 && r1 == 4) return launch_pair_as<2, 4>(a0, p0, a1, p1, g0, g1, lds, s);
  if (r0 == 4 && r1 == 2) return launch_pair_as<4, 2>(a0, p0, a1, p1, g0, g1, lds, s);
  if (r0 == 4 && r1 == 4) return launch_pair_as<4, 4>(a0, p0, a1, p1, g0, g1, lds, s);
  return 1;
}

int gq_launch_matvec(int dtype, int mode, const MvArgs &a, hipStream_t s) {
  if (a.nseg < 1 || a.nseg > 3 || a.cols <= 0 || a.cols > 16384 || (a.cols & 3)) return -1;
  switch (dtype) {
  case GQ_Q4_K: return a.cols % 256 ? -2 : launch_dt<GQ_Q4_K>(mode, a, s);
  case GQ_Q6_K: return a.cols % 256 ? -2 : launch_dt<GQ_Q6_K>(mode, a, s);
  case GQ_Q8_0: return a.cols % 32 ? -2 : launch_dt<GQ_Q8_0>(mode, a, s);
  default: return -1;
  }
}
