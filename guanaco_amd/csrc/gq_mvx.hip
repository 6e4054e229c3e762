/*
 * gq_mvx.hip — quantised matvec on the vector ALUs (gfx950), and the launch
 * dispatch between it and the int8 matrix-core kernel (gq_matvec.hip).
 *
 * y = W x for Q4_K, Q6_K and Q8_0 weights in the reference's block layouts
 * (quant_matvec_q4_k.c:9-16, quant_matvec_q6_k.c:5-12,
 * quant_matvec_q8_0.c:5-10), rows = out_features, x fp32, with the decode
 * path's fused prologue (RMSNorm) and epilogues (RoPE + K/V append, residual
 * add, SwiGLU) described in gq_internal.h.
 *
 * Work layout ("x-stationary").  Every 32 columns of a row are one unit of 16
 * quant bytes: Q4_K half of a 64-weight chunk (low nibbles 16 weights of
 * sub-block 2c, high nibbles 16 of sub-block 2c+1), Q6_K 16 bytes of ql with
 * the matching 16 of qh, Q8_0 one whole block.  A row group of L lanes gives
 * lane u the u-th unit of each of the R rows it computes: the lane loads its
 * 32 x values (times the RMSNorm weight) into registers once and streams the
 * R rows past them, every row's loads issued before the arithmetic.
 * Consecutive lanes read consecutive quant bytes, so one wave instruction
 * reads the quants of 8 whole blocks of a row; rows of more than 1024 units
 * loop over column tiles.  Measured against a plain streaming-read kernel on
 * MI355X this layout was 1.5x faster than staging x in LDS per workgroup for
 * the long rows of the down projection (x re-reads were the cost).  Where a
 * workgroup holds two or more row groups of one column tile, they split the x
 * loads and share the unit through LDS instead (kShx below).
 *
 * Per unit and row a lane decodes only what its 32 weights need.  Q4_K lanes
 * share the 16-byte block header: each of the 8 lanes of a block loads one of
 * its dwords, quad DPP broadcasts them, each lane decodes the (scale, min)
 * of sub-block (lane & 7) and the two lanes using it read it by DPP.  Q6_K
 * and Q8_0 blocks are only 2-byte aligned in a row: their quants are read as
 * aligned dwords and funnel-shifted (v_alignbyte), never past the block.
 *
 * The arithmetic is the reference's formula refactored so each weight costs
 * one convert and one FMA: Q4_K d*sc*sum(q*x) - dmin*m*sum(x) with nibbles
 * converted two at a time by v_cvt_pk_f32_fp8 (gq_nib2f, exact), Q6_K
 * d*sc*(sum(q*x) - 32*sum(x)), Q8_0 d*sum(q*x) with q sign-extended.  Row
 * sums reduce by DPP over 8- or 16-lane segments, then in LDS, in a fixed
 * order: outputs are deterministic.
 */
#include <math.h>

#include <algorithm>

#include "gq_device.h"
#include "gq_internal.h"

namespace {

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

/* quad_perm controls: broadcast lane 0/1/2/3 of the quad, and the pair
 * selections [0,0,2,2] / [1,1,3,3] */
constexpr int kQuad0 = 0x00, kQuad1 = 0x55, kQuad2 = 0xAA, kQuad3 = 0xFF, kQuadEven = 0xA0, kQuadOdd = 0xF5;
/* [0,0,1,1] and [2,2,3,3]; [1,0,3,2] */
constexpr int kQuadLoPair = 0x50, kQuadHiPair = 0xFA, kQuadSwap = 0xB1;

__device__ __forceinline__ float sum4(const float4 &v) { return (v.x + v.y) + (v.z + v.w); }

/* Unit traits: the block bytes a unit lives in (boff), its first column
 * (col; the second 16 columns start XHI later), its loads and its dot
 * product with the lane's x slices. */
template <int DT>
struct Ux;

/* Q4_K (quant_matvec_q4_k.c:9-16, 47-56): unit j = u & 7 of a block is
 * qs[16j .. 16j+15], chunk c = j/2, half h = j&1: low nibbles are weights
 * 64c + 16h + i (sub-block 2c), high nibbles 64c + 32 + 16h + i (2c+1). */
template <>
struct Ux<GQ_Q4_K> {
  static constexpr int BB = 144, XHI = 32;
  struct Raw {
    uint4 q;
    uint32_t h; /* header dword (j & 3): d|dmin, scales 0-3, 4-7, 8-11 */
  };
  static __device__ __forceinline__ uint32_t boff(int u) { return (uint32_t)BB * (uint32_t)(u >> 3); }
  static __device__ __forceinline__ int col(int u) { return 256 * (u >> 3) + 64 * ((u >> 1) & 3) + 16 * (u & 1); }
  /* blk: this lane's block (a per-lane 64-bit address: measured faster
   * than a scalar row base with 32-bit lane offsets) */
  static __device__ __forceinline__ Raw load(const uint8_t *row, int u, int) {
    const uint8_t *blk = row + boff(u);
    const int j = u & 7;
    Raw r;
    r.q = gld<uint4>(blk + 16 + 16 * j);
    r.h = gld<uint32_t>(blk + 4 * (j & 3));
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw &r, int j, const float4 (&xl)[4], const float4 (&xh)[4],
                                              float sxl, float sxh, uint32_t) {
    /* the 8 lanes of the block hold the header's 4 dwords twice (one quad
     * each): broadcast within the quad */
    const uint32_t D = dpp_u<kQuad0>(r.h), H1 = dpp_u<kQuad1>(r.h), H2 = dpp_u<kQuad2>(r.h),
                   H3 = dpp_u<kQuad3>(r.h);
    /* this lane's sub-block j (get_scale_min_k4, quant_matvec_q4_k.c:47-56):
     * j < 4: sc = q[j] & 63, m = q[j+4] & 63; else sc = (q[j+4] & 15) |
     * (q[j-4] >> 6) << 4, m = (q[j+4] >> 4) | (q[j] >> 6) << 4 */
    const uint32_t o = 8u * (uint32_t)(j & 3);
    const uint32_t sl = __builtin_amdgcn_ubfe(H1, o, 6), ml = __builtin_amdgcn_ubfe(H2, o, 6);
    const uint32_t sh = __builtin_amdgcn_ubfe(H3, o, 4) | (__builtin_amdgcn_ubfe(H1, o + 6, 2) << 4);
    const uint32_t mh = __builtin_amdgcn_ubfe(H3, o + 4, 4) | (__builtin_amdgcn_ubfe(H2, o + 6, 2) << 4);
    const bool hi = j >= 4;
    /* d * sc with the 2^9 of the fp8 nibble convert folded in (exact) */
    const float fd = (gq_h2f(D) * 512.f) * (float)(hi ? sh : sl);
    const float fm = gq_h2f(D >> 16) * (float)(hi ? mh : ml);
    /* sub-blocks 2c and 2c+1 come from lanes (j & ~1) and (j | 1) */
    const float ds0 = dpp_f<kQuadEven>(fd), ds1 = dpp_f<kQuadOdd>(fd);
    const float dm0 = dpp_f<kQuadEven>(fm), dm1 = dpp_f<kQuadOdd>(fm);
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    float dl = 0.f, dh = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hn = (w[i] >> 4) & 0x0F0F0F0Fu;
      const gq_f32x2 a = gq_nib2f<false>(lo), b = gq_nib2f<true>(lo);
      const gq_f32x2 e = gq_nib2f<false>(hn), f = gq_nib2f<true>(hn);
      dl = __builtin_fmaf(a.x, xl[i].x, dl);
      dl = __builtin_fmaf(a.y, xl[i].y, dl);
      dl = __builtin_fmaf(b.x, xl[i].z, dl);
      dl = __builtin_fmaf(b.y, xl[i].w, dl);
      dh = __builtin_fmaf(e.x, xh[i].x, dh);
      dh = __builtin_fmaf(e.y, xh[i].y, dh);
      dh = __builtin_fmaf(f.x, xh[i].z, dh);
      dh = __builtin_fmaf(f.y, xh[i].w, dh);
    }
    float acc = ds0 * dl;
    acc = __builtin_fmaf(ds1, dh, acc);
    acc = __builtin_fmaf(-dm0, sxl, acc);
    return __builtin_fmaf(-dm1, sxh, acc);
  }
};

/* Q6_K (quant_matvec_q6_k.c:5-12, 62-95): unit j = u & 7 of a block is half
 * h = j/4, group v = j&3: ql_h[16v .. 16v+15] with the 2-bit fields of
 * qh_h[16(v&1) ..] (bits 0-1 / 4-5 for v < 2, 2-3 / 6-7 for v >= 2); low
 * nibbles are weights 128h + 16v + i (scale sc_h[v]), high nibbles
 * 128h + 64 + 16v + i (scale sc_h[v+4]). */
template <>
struct Ux<GQ_Q6_K> {
  static constexpr int BB = 210, XHI = 64;
  struct Raw {
    uint4 l4, h4;
    uint32_t l1, h1, d;
    uint32_t sw; /* scales sc_h[2v], sc_h[2v+1] (lane v of the half's quad) */
  };
  static __device__ __forceinline__ uint32_t boff(int u) { return (uint32_t)BB * (uint32_t)(u >> 3); }
  static __device__ __forceinline__ int col(int u) { return 256 * (u >> 3) + 128 * ((u >> 2) & 1) + 16 * (u & 3); }
  static __device__ __forceinline__ Raw load(const uint8_t *row, int u, int) {
    const uint8_t *blk = row + boff(u);
    const int j = u & 7;
    Raw r;
    const int h = j >> 2, v = j & 3;
    /* ql at 64h+16v and qh at 128+32h+16(v&1): both at the block's 2-byte
     * phase, 20 aligned bytes each cover the 16 wanted (ending by byte 194) */
    const uintptr_t al = (uintptr_t)(blk + 64 * h + 16 * v) & ~(uintptr_t)3;
    const uintptr_t ah = (uintptr_t)(blk + 128 + 32 * h + 16 * (v & 1)) & ~(uintptr_t)3;
    r.l4 = gld<uint4>((const void *)al);
    r.l1 = gld<uint32_t>((const void *)(al + 16));
    r.h4 = gld<uint4>((const void *)ah);
    r.h1 = gld<uint32_t>((const void *)(ah + 16));
    r.sw = gld<unsigned short>(blk + 192 + 8 * h + 2 * v);
    r.d = gld<unsigned short>(blk + 208);
    return r;
  }
  /* sh: the block's byte phase (0 or 2) */
  static __device__ __forceinline__ float dot(const Raw &r, int j, const float4 (&xl)[4], const float4 (&xh)[4],
                                              float sxl, float sxh, uint32_t sh) {
    const uint32_t ql[4] = {__builtin_amdgcn_alignbyte(r.l4.y, r.l4.x, sh),
                            __builtin_amdgcn_alignbyte(r.l4.z, r.l4.y, sh),
                            __builtin_amdgcn_alignbyte(r.l4.w, r.l4.z, sh),
                            __builtin_amdgcn_alignbyte(r.l1, r.l4.w, sh)};
    const uint32_t qh[4] = {__builtin_amdgcn_alignbyte(r.h4.y, r.h4.x, sh),
                            __builtin_amdgcn_alignbyte(r.h4.z, r.h4.y, sh),
                            __builtin_amdgcn_alignbyte(r.h4.w, r.h4.z, sh),
                            __builtin_amdgcn_alignbyte(r.h1, r.h4.w, sh)};
    /* sc_h[v] sits in lane v/2 of the quad, sc_h[v+4] in lane 2 + v/2,
     * byte v & 1 of each (int8) */
    const uint32_t sb = 8u * (uint32_t)(j & 1);
    const int s0 = __builtin_amdgcn_sbfe((int)dpp_u<kQuadLoPair>(r.sw), sb, 8);
    const int s1 = __builtin_amdgcn_sbfe((int)dpp_u<kQuadHiPair>(r.sw), sb, 8);
    const uint32_t qs = 2u * (uint32_t)((j & 3) >> 1); /* qh field pair of this group */
    float dl = 0.f, dh = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t hb = qh[i] >> qs;
      const uint32_t lo = (ql[i] & 0x0F0F0F0Fu) | ((hb << 4) & 0x30303030u); /* 6-bit q, 0..63 */
      const uint32_t hi = ((ql[i] >> 4) & 0x0F0F0F0Fu) | (hb & 0x30303030u);
      dl = __builtin_fmaf((float)(lo & 0xffu), xl[i].x, dl);
      dl = __builtin_fmaf((float)((lo >> 8) & 0xffu), xl[i].y, dl);
      dl = __builtin_fmaf((float)((lo >> 16) & 0xffu), xl[i].z, dl);
      dl = __builtin_fmaf((float)(lo >> 24), xl[i].w, dl);
      dh = __builtin_fmaf((float)(hi & 0xffu), xh[i].x, dh);
      dh = __builtin_fmaf((float)((hi >> 8) & 0xffu), xh[i].y, dh);
      dh = __builtin_fmaf((float)((hi >> 16) & 0xffu), xh[i].z, dh);
      dh = __builtin_fmaf((float)(hi >> 24), xh[i].w, dh);
    }
    const float d = gq_h2f(r.d);
    const float acc = (d * (float)s0) * __builtin_fmaf(-32.f, sxl, dl);
    return __builtin_fmaf(d * (float)s1, __builtin_fmaf(-32.f, sxh, dh), acc);
  }
};

/* Q8_0 (quant_matvec_q8_0.c:5-10, 60-75): unit u is block u (d, then 32
 * int8 quants at a 2-byte phase): read as two aligned 16-byte loads plus the
 * block's last two bytes. */
template <>
struct Ux<GQ_Q8_0> {
  static constexpr int BB = 34, XHI = 16;
  struct Raw {
    uint4 a, b;
    uint32_t t, d;
  };
  static __device__ __forceinline__ uint32_t boff(int u) { return (uint32_t)BB * (uint32_t)u; }
  static __device__ __forceinline__ int col(int u) { return 32 * u; }
  static __device__ __forceinline__ Raw load(const uint8_t *row, int u, int) {
    const uint8_t *blk = row + boff(u);
    Raw r;
    /* quants from blk + 2: the aligned start is the block or 2 bytes in */
    const uintptr_t a = (uintptr_t)(blk + 2) & ~(uintptr_t)3;
    r.a = gld<uint4>((const void *)a);
    r.b = gld<uint4>((const void *)(a + 16));
    r.t = gld<unsigned short>(blk + 32);
    r.d = gld<unsigned short>(blk);
    return r;
  }
  /* sh: the block's byte phase (0 or 2); its quants start 2 bytes later */
  static __device__ __forceinline__ float dot(const Raw &r, int, const float4 (&xl)[4], const float4 (&xh)[4],
                                              float sxl, float sxh, uint32_t sh) {
    (void)sxl, (void)sxh;
    const uint32_t qsh = (sh + 2u) & 3u;
    const uint32_t w[9] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.t};
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      /* the int8 quants sign-extended, so the sum is of q*x itself, as the
       * reference's (quant_matvec_q8_0.c:60-75): no large offset to cancel */
      const uint32_t q = __builtin_amdgcn_alignbyte(w[i + 1], w[i], qsh);
      const float4 &x = i < 4 ? xl[i] : xh[i - 4];
      s = __builtin_fmaf((float)(int8_t)q, x.x, s);
      s = __builtin_fmaf((float)(int8_t)(q >> 8), x.y, s);
      s = __builtin_fmaf((float)(int8_t)(q >> 16), x.z, s);
      s = __builtin_fmaf((float)(int8_t)(q >> 24), x.w, s);
    }
    return gq_h2f(r.d) * s;
  }
};

/* Q6_K re-laid out per row for this kernel (gq_launch_q6k_units, made once
 * at model bind; the same 210 bytes per block, every field naturally
 * aligned): unit u (block u/8, half h, group v as for Q6_K) has its 16
 * bytes of ql_h[16v ..] at 24u, then two dwords of its 2-bit fields: byte k
 * of quant dword m's fields (bits 0-1 and 4-5 of (qh_h[16(v&1) + 4m + k] >>
 * 2(v/2)), the pair Q6_K uses for that quant's low and high nibble) sits in
 * byte k of dword m/2 shifted left by 2(m&1); its two scales (sc_h[v],
 * sc_h[v+4]) are the int8 pair at 192*nb + 2u, and its block's d the fp16
 * at 208*nb + 2(u/8).  A lane holds 8 dwords per row (12 for the reference
 * layout, whose 2-byte block phase costs an extra dword per field and the
 * funnel shifts), so 8-row groups fit 128 VGPRs.  The products and their
 * order are Q6_K's: results are bit-identical to it. */
template <>
struct Ux<GQ_Q6_KX> {
  static constexpr int XHI = 64;
  struct Raw {
    uint4 q;
    uint2 h;
    uint32_t s, d;
  };
  static __device__ __forceinline__ uint32_t boff(int u) { return 24u * (uint32_t)u; }
  static __device__ __forceinline__ int col(int u) { return Ux<GQ_Q6_K>::col(u); }
  static __device__ __forceinline__ Raw load(const uint8_t *row, int u, int nb) {
    Raw r;
    r.q = gld<uint4>(row + boff(u));
    r.h = gld<uint2>(row + boff(u) + 16);
    r.s = gld<unsigned short>(row + 192 * nb + 2 * u);
    r.d = gld<unsigned short>(row + 208 * nb + 2 * (u >> 3));
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw &r, int, const float4 (&xl)[4], const float4 (&xh)[4],
                                              float sxl, float sxh, uint32_t) {
    const uint32_t ql[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    const uint32_t hf[4] = {r.h.x, r.h.x >> 2, r.h.y, r.h.y >> 2};
    const int s0 = __builtin_amdgcn_sbfe((int)r.s, 0, 8), s1 = __builtin_amdgcn_sbfe((int)r.s, 8, 8);
    float dl = 0.f, dh = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t lo = (ql[i] & 0x0F0F0F0Fu) | ((hf[i] << 4) & 0x30303030u); /* 6-bit q, 0..63 */
      const uint32_t hi = ((ql[i] >> 4) & 0x0F0F0F0Fu) | (hf[i] & 0x30303030u);
      dl = __builtin_fmaf((float)(lo & 0xffu), xl[i].x, dl);
      dl = __builtin_fmaf((float)((lo >> 8) & 0xffu), xl[i].y, dl);
      dl = __builtin_fmaf((float)((lo >> 16) & 0xffu), xl[i].z, dl);
      dl = __builtin_fmaf((float)(lo >> 24), xl[i].w, dl);
      dh = __builtin_fmaf((float)(hi & 0xffu), xh[i].x, dh);
      dh = __builtin_fmaf((float)((hi >> 8) & 0xffu), xh[i].y, dh);
      dh = __builtin_fmaf((float)((hi >> 16) & 0xffu), xh[i].z, dh);
      dh = __builtin_fmaf((float)(hi >> 24), xh[i].w, dh);
    }
    const float d = gq_h2f(r.d);
    const float acc = (d * (float)s0) * __builtin_fmaf(-32.f, sxl, dl);
    return __builtin_fmaf(d * (float)s1, __builtin_fmaf(-32.f, sxh, dh), acc);
  }
};

/* One thread per (row, unit): the Q6_K row in the reference layout (src) to
 * the unit layout above (dst, same size). */
__global__ __launch_bounds__(256) void q6k_units_kernel(const uint8_t *src, uint8_t *dst, int rows, int nb) {
  const int upr = 8 * nb;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)rows * upr) return;
  const int row = (int)(t / upr), u = (int)(t - (long long)row * upr);
  const int b = u >> 3, j = u & 7, h = j >> 2, v = j & 3;
  const uint8_t *blk = src + ((size_t)row * nb + b) * 210;
  uint8_t *drow = dst + (size_t)row * nb * 210, *du = drow + 24 * u;
  for (int i = 0; i < 16; i++) du[i] = blk[64 * h + 16 * v + i];
  const int qs = 2 * (v >> 1);
  uint32_t P[2] = {0u, 0u};
  for (int i = 0; i < 16; i++) {
    const uint32_t f = ((uint32_t)blk[128 + 32 * h + 16 * (v & 1) + i] >> qs) & 0x33u;
    const int m = i >> 2, k = i & 3;
    P[m >> 1] |= f << (8 * k + 2 * (m & 1));
  }
  for (int i = 0; i < 8; i++) du[16 + i] = (uint8_t)(P[i >> 2] >> (8 * (i & 3)));
  drow[192 * nb + 2 * u] = blk[192 + 8 * h + v];
  drow[192 * nb + 2 * u + 1] = blk[192 + 8 * h + v + 4];
  if (j == 0) {
    drow[208 * nb + 2 * b] = blk[208];
    drow[208 * nb + 2 * b + 1] = blk[209];
  }
}

struct MxPlan {
  int L;        /* lanes per row group, a multiple of 8 */
  int G;        /* row groups per workgroup (blockDim.x = G * L) */
  int nt;       /* column tiles: lane u covers units u, u + L, ... */
  int upr;      /* units (32 columns) per row */
  int total;    /* output rows (MV_SWIGLU: gate rows) */
  int nwg;      /* workgroups of this launch */
  int rowbytes;
};

/* sum over aligned groups of SEGW lanes, valid in the group's last lane */
template <int SEGW>
__device__ __forceinline__ float seg_sum(float v) {
  return SEGW == 16 ? gq_row16_sum(v) : gq_row8_sum(v);
}

/* One launch's work as workgroup `bid` (of p.nwg; a paired launch runs two
 * of these bodies side by side).  red: LDS of (blockDim / SEGW) * (R + 1)
 * floats. */
/* Flags of a launch: NORM the RMSNorm prologue (a.norm_w set), MT rows of
 * more than one column tile (cols > 32768): both compile-time, a runtime
 * branch or loop around the loads measured 0.6-2 us slower. */
constexpr int kNorm = 1, kMT = 2;
/* SHX: launches of two or more row groups (G >= 2, so L <= 128) share x
 * (times the norm weights) through LDS: groups 0 and 1 load the low and the
 * high half of each unit, every group reads the whole unit back.  With every
 * group loading its own copy the 8B q/k/v launch took 8.5 us (49 MB of
 * L2-to-CU reads at 768 workgroups) and o 5.1; shared, 7.5 and 4.65, and the
 * graph-replayed decode step 499 -> 509 tok/s. */
constexpr int kShx = 4;
constexpr int kShxLanes = 128; /* xsh: 8 float4 per lane, lane-major rows */

template <int DT, int MODE, int R, int SEGW, bool UNI, int FL>
__device__ __forceinline__ void mvx_body(const MvArgs &a, const MxPlan &p, int bid, float *red, float2 *scs,
                                         float4 *xsh) {
#pragma clang fp contract(off)
  using T = Ux<DT>;
  static_assert(R % 2 == 0, "row pairs (RoPE, SwiGLU) stay inside a group");
  constexpr int P = MODE == MV_SWIGLU ? R / 2 : R; /* output rows per group */
  constexpr int NV = R + 1;                        /* row sums, sum of x^2 */
  const int tid = threadIdx.x;
  /* every kernel-argument field this body uses, read at entry and pinned
   * into scalar registers by ONE asm statement: one batch of scalar loads
   * and one wait (pinned one by one, the compiler issued them in three
   * batches, each a kernel-argument round trip before the first weight
   * load).  Pinned values keep selects between segments as selects of
   * registers (see MvSegs). */
  const float *xp = a.x, *nw = a.norm_w;
  int cols = a.cols;
  float eps = a.eps;
  const float2 *rcs = a.rope.cs;
  const int *rpd = a.rope.pos_dev;
  int rpos = a.rope.pos, hd = a.rope.head_dim, msq = a.rope.max_seq;
  int L = p.L, upr = p.upr, nt = p.nt, rowbytes = p.rowbytes, G = p.G, total = p.total;
  const uint8_t *sw0 = a.seg[0].w, *sw1 = a.seg[1].w, *sw2 = a.seg[2].w;
  float *sy0 = a.seg[0].y, *sy1 = a.seg[1].y, *sy2 = a.seg[2].y;
  const float *sr0 = a.seg[0].r; /* MV_RESID launches have one segment */
  int sn0 = a.seg[0].rows, sn1 = a.seg[1].rows, nseg = a.nseg;
  int sk0 = a.seg[0].kind, sk1 = a.seg[1].kind, sk2 = a.seg[2].kind;
  asm volatile(""
               : "+s"(xp), "+s"(nw), "+s"(cols), "+s"(eps), "+s"(rcs), "+s"(rpd), "+s"(rpos), "+s"(hd),
                 "+s"(msq), "+s"(L), "+s"(upr), "+s"(nt), "+s"(rowbytes), "+s"(G), "+s"(total), "+s"(sw0),
                 "+s"(sw1), "+s"(sw2), "+s"(sy0), "+s"(sy1), "+s"(sy2), "+s"(sr0), "+s"(sn0), "+s"(sn1),
                 "+s"(nseg), "+s"(sk0), "+s"(sk1), "+s"(sk2));
  const int nbq = cols >> 8; /* 256-column blocks per row (the Q6_K unit layout) */
  /* UNI: row groups are whole waves (L % 64 == 0), so the group, its rows
   * and their addresses are wave-uniform (scalar registers) */
  const int g = UNI ? __builtin_amdgcn_readfirstlane(tid / L) : tid / L;
  const int ul = tid - g * L;
  constexpr bool norm = (FL & kNorm) != 0, MT = (FL & kMT) != 0, SHX = (FL & kShx) != 0;
  static_assert(!(SHX && MT), "shared x covers one column tile");
#define GQ_SEL3(s, a0, a1, a2) ((s) == 0 ? (a0) : (s) == 1 ? (a1) : (a2))
#define GQ_LOCATE(gr, s, lr)                                                                                \
  do {                                                                                                      \
    (s) = 0, (lr) = (gr);                                                                                   \
    if (nseg > 1 && (lr) >= sn0) {                                                                          \
      (lr) -= sn0, (s) = 1;                                                                                 \
      if (nseg > 2 && (lr) >= sn1) (lr) -= sn1, (s) = 2;                                                    \
    }                                                                                                       \
  } while (0)

  /* the epilogue role of this thread (tid < G * P finishes output row i of
   * group gg): its residual (MV_RESID launches have one segment) is loaded
   * first, with nothing waiting on it before the epilogue */
  float e_res = 0.f;
  if (MODE == MV_RESID && tid < G * P) {
    const int erow = (bid * G + tid / P) * P + tid % P;
    if (erow < total) e_res = gld<float>(sr0 + erow);
  }
  int epos = 0; /* the device position, read behind the first tile's weights */
  /* weight rows of this group (rows past the end clamp to the last: loaded,
   * never stored) */
  const uint8_t *rp[R];
  const int rg = bid * G + g;
  if (MODE == MV_SWIGLU) {
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int pr = min(rg * P + i, total - 1);
      rp[i] = sw0 + (size_t)pr * rowbytes;
      rp[P + i] = sw1 + (size_t)pr * rowbytes;
    }
  } else if (nseg == 1) {
#pragma unroll
    for (int i = 0; i < R; i++) rp[i] = sw0 + (size_t)min(rg * R + i, total - 1) * rowbytes;
  } else {
    /* several segments: R divides each one's rows (the host picks R so),
     * so a group's rows lie in one segment; groups past the end take the
     * last group's rows */
    int s0, lr0;
    GQ_LOCATE(min(rg * R, total - R), s0, lr0);
    const uint8_t *base = GQ_SEL3(s0, sw0, sw1, sw2) + (size_t)lr0 * rowbytes;
#pragma unroll
    for (int i = 0; i < R; i++) rp[i] = base + (size_t)i * rowbytes;
  }

  float2 cs_pre = make_float2(1.f, 0.f);
  float acc[R], ss = 0.f;
#pragma unroll
  for (int k = 0; k < R; k++) acc[k] = 0.f;
  if (g < G) {
    for (int t = 0; t < (MT ? nt : 1); t++) {
      const int u = ul + t * L;
      /* whole 8-lane blocks are in or out together; Q4_K/Q6_K single tiles
       * have L == upr */
      const bool act = !(MT || DT == GQ_Q8_0) || u < upr;
      /* x slices first (their latency hides under the rows'), then every
       * row's quants */
      const int c0 = act ? T::col(u) : 0;
      float4 xl[4], xh[4], wv[4];
      if constexpr (SHX) { /* this group's half: x in xl, norm weights in wv */
        if (g < 2) {
          const int cb = c0 + (g ? T::XHI : 0);
#pragma unroll
          for (int i = 0; i < 4; i++) xl[i] = gld<float4>(xp + cb + 4 * i);
          if constexpr (norm) {
#pragma unroll
            for (int i = 0; i < 4; i++) wv[i] = gld<float4>(nw + cb + 4 * i);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          xl[i] = gld<float4>(xp + c0 + 4 * i);
          xh[i] = gld<float4>(xp + c0 + T::XHI + 4 * i);
          if (!act) xl[i] = xh[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      if constexpr (norm && !SHX) { /* y = r * W (w .* x): raw sum of squares, x times w */
        float4 wl[4], wh[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          wl[i] = gld<float4>(nw + c0 + 4 * i);
          wh[i] = gld<float4>(nw + c0 + T::XHI + 4 * i);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
          ss = __builtin_fmaf(xl[i].x, xl[i].x, ss);
          ss = __builtin_fmaf(xl[i].y, xl[i].y, ss);
          ss = __builtin_fmaf(xl[i].z, xl[i].z, ss);
          ss = __builtin_fmaf(xl[i].w, xl[i].w, ss);
          ss = __builtin_fmaf(xh[i].x, xh[i].x, ss);
          ss = __builtin_fmaf(xh[i].y, xh[i].y, ss);
          ss = __builtin_fmaf(xh[i].z, xh[i].z, ss);
          ss = __builtin_fmaf(xh[i].w, xh[i].w, ss);
          xl[i] = make_float4(xl[i].x * wl[i].x, xl[i].y * wl[i].y, xl[i].z * wl[i].z, xl[i].w * wl[i].w);
          xh[i] = make_float4(xh[i].x * wh[i].x, xh[i].y * wh[i].y, xh[i].z * wh[i].z, xh[i].w * wh[i].w);
        }
      }
      /* every wave's x requests ahead of any wave's weight requests: a
       * CU's memory pipeline serves its waves' requests in about the order
       * they were issued, and without this barrier a late wave's x queued
       * behind the early waves' rows (down: x in at 1.2-5.8 us, so most
       * rows' arithmetic waited for x; q/k/v 9.1 -> 8.9 us) */
      if (!MT) __builtin_amdgcn_s_barrier();
      typename T::Raw raw[R];
      if (act) {
#pragma unroll
        for (int k = 0; k < R; k++) raw[k] = T::load(rp[k], u, nbq);
      }
      /* the device position and its RoPE row, behind the weights (kept in a
       * register until the reduction puts it in LDS) */
      if (MODE == MV_STORE && t == 0 && rcs) {
        epos = rpd ? gq_sld<int>(rpd) : rpos;
        if (tid < (hd >> 1) && epos >= 0 && epos < msq) cs_pre = gld<float2>(rcs + (size_t)epos * (hd >> 1) + tid);
      }
      if constexpr (SHX) {
        if (g < 2) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float4 v = act ? xl[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (norm) {
              ss = __builtin_fmaf(v.x, v.x, ss);
              ss = __builtin_fmaf(v.y, v.y, ss);
              ss = __builtin_fmaf(v.z, v.z, ss);
              ss = __builtin_fmaf(v.w, v.w, ss);
              v = make_float4(v.x * wv[i].x, v.y * wv[i].y, v.z * wv[i].z, v.w * wv[i].w);
            }
            xsh[(4 * g + i) * kShxLanes + ul] = v;
          }
        }
        /* LDS only: the rows' loads stay in flight across this barrier */
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
        for (int i = 0; i < 4; i++) {
          xl[i] = xsh[i * kShxLanes + ul];
          xh[i] = xsh[(4 + i) * kShxLanes + ul];
        }
      }
      if (!act) continue;
      const float sxl = (sum4(xl[0]) + sum4(xl[1])) + (sum4(xl[2]) + sum4(xl[3]));
      const float sxh = (sum4(xh[0]) + sum4(xh[1])) + (sum4(xh[2]) + sum4(xh[3]));
#pragma unroll
      for (int k = 0; k < R; k++) {
        acc[k] += T::dot(raw[k], u & 7, xl, xh, sxl, sxh, (uint32_t)(((uintptr_t)rp[k] + T::boff(u)) & 3u));
        /* finish a row before waiting for the next one's bytes */
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  /* row sums: DPP over SEGW-lane segments, then LDS */
  float v[NV];
#pragma unroll
  for (int k = 0; k < R; k++) v[k] = seg_sum<SEGW>(acc[k]);
  v[R] = norm ? seg_sum<SEGW>(ss) : 0.f;
  if ((tid & (SEGW - 1)) == SEGW - 1) {
#pragma unroll
    for (int k = 0; k < NV; k++) red[(tid / SEGW) * NV + k] = v[k];
  }
  if (MODE == MV_STORE && rcs && tid < (hd >> 1)) scs[tid] = cs_pre;
  __syncthreads();

  /* epilogue: this thread's output row (see its role above) */
  if (tid >= G * P) return;
  const int egg = tid / P, ei = tid - egg * P;
  const int erow = (bid * G + egg) * P + ei;
  if (erow >= total) return;
  int es = 0, elr = erow;
  if (MODE != MV_SWIGLU) GQ_LOCATE(erow, es, elr);
  const int spg = L / SEGW;
  const float *rr = red + egg * spg * NV;
  float rs = 1.f;
  if constexpr (norm) { /* 1/sqrt(mean(x^2) + eps) (kernels_cpu.c:242-253) */
    float tot = 0.f;
    if constexpr (SHX) /* groups 0 and 1 summed the halves of x */
      for (int s = 0; s < 2 * spg; s++) tot += red[s * NV + R];
    else
      for (int s = 0; s < spg; s++) tot += rr[s * NV + R];
    tot = tot / (float)cols;
    tot = tot + eps;
    rs = 1.0f / sqrtf(tot);
  }
#define GQ_ROWSUM(k, out)                                                                                   \
  do {                                                                                                      \
    float t_ = 0.f;                                                                                         \
    for (int s_ = 0; s_ < spg; s_++) t_ += rr[s_ * NV + (k)];                                                \
    (out) = t_ * rs;                                                                                        \
  } while (0)
  if (MODE == MV_SWIGLU) {
    float gv, uv;
    GQ_ROWSUM(ei, gv);
    GQ_ROWSUM(P + ei, uv);
    gst<float>(sy0 + erow, gq_silu_mul(gv, uv));
    return;
  }
  float *const sy = GQ_SEL3(es, sy0, sy1, sy2);
  const int kind = GQ_SEL3(es, sk0, sk1, sk2);
  float val;
  GQ_ROWSUM(ei, val);
  if (MODE == MV_RESID) {
    gst<float>(sy + elr, val + e_res);
    return;
  }
  if (kind == SEG_PLAIN) {
    gst<float>(sy + elr, val);
    return;
  }
  if (epos < 0 || epos >= msq) return; /* rejected on the host */
  const int h = elr / hd, d = elr - h * hd;
  if (kind != SEG_KV) {
    /* adjacent pair (d & ~1, d | 1) rotated by the row of pos
     * (kernels_cpu.c:415-429: products and difference rounded apart);
     * rows 2m, 2m+1 are in the same group */
    const float2 cs = scs[d >> 1];
    /* the partner row is the adjacent lane's (P is even, so row parity is
     * lane parity), active here with this one: its finished sum by DPP */
    const float partner = dpp_f<kQuadSwap>(val);
    const float x0 = (d & 1) ? partner : val, x1 = (d & 1) ? val : partner;
    val = (d & 1) ? x0 * cs.y + x1 * cs.x : x0 * cs.x - x1 * cs.y;
  }
  if (kind == SEG_ROPE)
    gst<float>(sy + elr, val);
  else
    gst<float>(sy + ((size_t)h * msq + epos) * hd + d, val);
#undef GQ_ROWSUM
#undef GQ_LOCATE
#undef GQ_SEL3
}

template <int DT, int MODE, int R, int SEGW, int MAXNT, bool UNI, int FL>
__global__ __launch_bounds__(MAXNT) void mvx_kernel(MvArgs a, MxPlan p) {
  __shared__ float red[(MAXNT / SEGW) * (R + 1)];
  __shared__ float2 scs[MODE == MV_STORE ? 256 : 1]; /* RoPE row (head_dim <= 512) */
  __shared__ float4 xsh[(FL & kShx) ? 8 * kShxLanes : 1];
  mvx_body<DT, MODE, R, SEGW, UNI, FL>(a, p, blockIdx.x, red, scs, xsh);
}

/* Two MV_STORE launches of different dtypes over the same x in one grid:
 * workgroups [0, p1.nwg) run the second, the rest the first (Q4_K q/k and
 * Q6_K v of a Q4_K_M layer; v from its unit-layout copy where bind made one:
 * 8B decode 514.9-515.1 -> 515.2-515.9 tok/s). */
template <int DT0, int R0, int DT1, int R1, int SEGW, int MAXNT, int FL>
__global__ __launch_bounds__(MAXNT) void mvx_pair_kernel(MvArgs a0, MxPlan p0, MvArgs a1, MxPlan p1) {
  __shared__ float red[(MAXNT / SEGW) * ((R0 > R1 ? R0 : R1) + 1)];
  __shared__ float2 scs[256];
  __shared__ float4 xsh[(FL & kShx) ? 8 * kShxLanes : 1];
  /* the second launch's workgroups first: its (Q6_K) rows cost more each,
   * so they do not form the tail */
  if ((int)blockIdx.x < p1.nwg)
    mvx_body<DT1, MV_STORE, R1, SEGW, true, FL>(a1, p1, blockIdx.x, red, scs, xsh);
  else
    mvx_body<DT0, MV_STORE, R0, SEGW, true, FL>(a0, p0, (int)blockIdx.x - p1.nwg, red, scs, xsh);
}

/* 0: this kernel for every launch; 1 (default): the matrix-core kernel for
 * gate/up + SwiGLU and the LM head, where the weights have tiled copies;
 * 2: the matrix-core kernel wherever it fits; 3: as 1, with every Q6_K
 * launch on the reference layout (no unit-layout copies) */
int g_path = 1;

int rows_out(const MvArgs &a, int mode) {
  if (mode == MV_SWIGLU) return a.seg[0].rows;
  int t = 0;
  for (int i = 0; i < a.nseg; i++) t += a.seg[i].rows;
  return t;
}

/* Lanes, groups and column tiles for a row of `cols` columns; rows per
 * group from the measured shapes (8B decode on MI355X): 8 for launches of
 * >= 4096 output rows (4096 x 4096 Q4_K: 4.7 us against 4.8 with 4), 6 for
 * such Q6_K launches (four waves per SIMD; down 15 us against 18 at three),
 * else 4 (1024-row Q6_K v: 3.6 us against 4.3 with 8); in 1024-thread
 * launches (rows of more than 16384 columns) 4 for Q4_K and 2 for Q6_K and
 * Q8_0, whose 4-row groups spill past the 128 VGPRs such launches allow. */
void plan(int dt, int mode, const MvArgs &a, int total, MxPlan &p, int &r, int &segw, int &maxnt) {
  p.upr = a.cols / 32;
  p.nt = (p.upr + 1023) / 1024;
  p.L = ((p.upr + p.nt - 1) / p.nt + 7) & ~7;
  segw = p.L % 16 == 0 ? 16 : 8;
  p.G = p.L <= 128 ? 256 / p.L : 1;
  const int nt = p.G * p.L;
  maxnt = nt <= 256 ? 256 : nt <= 512 ? 512 : 1024;
  if (maxnt == 1024)
    r = dt == GQ_Q4_K || dt == GQ_Q6_KX ? 4 : 2; /* 1024 threads leave 128 VGPRs: 4 rows of Q6_K or Q8_0 spill */
  else if (dt == GQ_Q8_0)
    r = 4;
  else if (dt == GQ_Q6_K && total >= 4096)
    r = 6; /* 8 rows of Q6_K quants do not fit 128 VGPRs */
  else if (mode == MV_STORE && a.rope.cs)
    r = 4; /* the decode step's q/k/v launch: twice the workgroups (768 at the 8B shape) */
  else if (mode == MV_RESID && a.cols <= 4096)
    r = 4; /* the o projection + residual: 512 workgroups at the 8B shape */
  else
    r = total >= 4096 ? 8 : 4;
  if (mode != MV_SWIGLU && a.nseg > 1) { /* groups must not straddle segments */
    auto fits = [&](int rr) {
      for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].rows % rr) return false;
      return true;
    };
    if (!fits(r)) {
      if (maxnt == 1024 && dt != GQ_Q4_K && dt != GQ_Q6_KX) r = fits(2) ? 2 : 0;
      else r = fits(4) ? 4 : fits(6) && maxnt != 1024 && dt != GQ_Q8_0 && dt != GQ_Q6_KX ? 6 : 0;
    }
  }
  p.total = total;
  const int per = mode == MV_SWIGLU ? r / 2 : r;
  const int ngroups = (total + per - 1) / per;
  p.nwg = (ngroups + p.G - 1) / p.G;
  int qk = 256, bb = 0;
  if (dt == GQ_Q4_K) bb = 144;
  else if (dt == GQ_Q6_K || dt == GQ_Q6_KX) bb = 210;
  else bb = 34, qk = 32;
  p.rowbytes = (a.cols / qk) * bb;
}

template <int DT, int MODE, int R, int SEGW, int MAXNT, int FL>
int launch_one(const MvArgs &a, const MxPlan &p, hipStream_t s) {
  if (p.L % 64 == 0)
    hipLaunchKernelGGL((mvx_kernel<DT, MODE, R, SEGW, MAXNT, true, FL>), dim3(p.nwg), dim3(p.G * p.L), 0, s, a, p);
  else
    hipLaunchKernelGGL((mvx_kernel<DT, MODE, R, SEGW, MAXNT, false, FL>), dim3(p.nwg), dim3(p.G * p.L), 0, s, a, p);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

/* the RMSNorm flag: only launches that take it (STORE, SWIGLU); shared x
 * for launches of two or more row groups (plan() gives those 256 threads) */
template <int DT, int MODE, int R, int SEGW, int MAXNT, int FL>
int launch_fl(const MvArgs &a, const MxPlan &p, hipStream_t s) {
  constexpr bool shx = !(FL & kMT) && MAXNT == 256;
  if constexpr (MODE != MV_RESID) {
    if constexpr (shx)
      if (a.norm_w && p.G >= 2) return launch_one<DT, MODE, R, SEGW, MAXNT, FL | kNorm | kShx>(a, p, s);
    if (a.norm_w) return launch_one<DT, MODE, R, SEGW, MAXNT, FL | kNorm>(a, p, s);
  } else {
    if (a.norm_w) return -1;
  }
  if constexpr (shx)
    if (p.G >= 2) return launch_one<DT, MODE, R, SEGW, MAXNT, FL | kShx>(a, p, s);
  return launch_one<DT, MODE, R, SEGW, MAXNT, FL>(a, p, s);
}

template <int DT, int MODE, int R>
int launch_r(const MvArgs &a, const MxPlan &p, int segw, int maxnt, hipStream_t s) {
  if (maxnt == 1024) {
    constexpr bool four = DT == GQ_Q4_K || DT == GQ_Q6_KX;
    if constexpr ((R == 4 && four) || (R == 2 && !four)) {
      if (p.nt > 1)
        return segw == 16 ? launch_fl<DT, MODE, R, 16, 1024, kMT>(a, p, s) : launch_fl<DT, MODE, R, 8, 1024, kMT>(a, p, s);
      return segw == 16 ? launch_fl<DT, MODE, R, 16, 1024, 0>(a, p, s) : launch_fl<DT, MODE, R, 8, 1024, 0>(a, p, s);
    }
    return -1;
  }
  if constexpr (R == 2) return -1;
  if (maxnt == 512)
    return segw == 16 ? launch_fl<DT, MODE, R, 16, 512, 0>(a, p, s) : launch_fl<DT, MODE, R, 8, 512, 0>(a, p, s);
  return segw == 16 ? launch_fl<DT, MODE, R, 16, 256, 0>(a, p, s) : launch_fl<DT, MODE, R, 8, 256, 0>(a, p, s);
}

template <int DT, int MODE>
int launch_mvx(const MvArgs &a, int total, hipStream_t s) {
  MxPlan p;
  int r, segw, maxnt;
  plan(DT, MODE, a, total, p, r, segw, maxnt);
  if (r == 0) { /* no group size divides every segment: one launch each */
    for (int i = 0; i < a.nseg; i++) {
      MvArgs b = a;
      b.seg[0] = a.seg[i];
      b.nseg = 1;
      const int rc = launch_mvx<DT, MODE>(b, a.seg[i].rows, s);
      if (rc) return rc;
    }
    return 0;
  }
  if constexpr (DT == GQ_Q8_0) {
    return r == 2 ? launch_r<DT, MODE, 2>(a, p, segw, maxnt, s) : launch_r<DT, MODE, 4>(a, p, segw, maxnt, s);
  } else {
    if (r == 8) return launch_r<DT, MODE, 8>(a, p, segw, maxnt, s);
    if constexpr (DT != GQ_Q6_KX)
      if (r == 6) return launch_r<DT, MODE, 6>(a, p, segw, maxnt, s);
    if constexpr (DT == GQ_Q6_K)
      if (r == 2) return launch_r<DT, MODE, 2>(a, p, segw, maxnt, s);
    return launch_r<DT, MODE, 4>(a, p, segw, maxnt, s);
  }
}

/* Validate the segments of a launch; returns the output rows or -1. */
int check_args(int mode, const MvArgs &a) {
  if (a.nseg < 1 || a.nseg > 3 || a.cols <= 0 || !a.x) return -1;
  for (int i = 0; i < a.nseg; i++)
    if (!a.seg[i].w || !a.seg[i].y || a.seg[i].rows <= 0) {
      if (!(mode == MV_SWIGLU && i == 1 && a.seg[1].w && a.seg[1].rows > 0)) return -1;
    }
  if (mode == MV_SWIGLU) {
    if (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows) return -1;
    return a.seg[0].rows;
  }
  if (mode == MV_RESID && a.nseg != 1) return -1; /* the kernel reads the residual of segment 0 */
  int total = 0;
  for (int i = 0; i < a.nseg; i++) {
    const MvSeg &sg = a.seg[i];
    if (mode == MV_RESID && !sg.r) return -1;
    if (sg.kind != SEG_PLAIN) {
      /* fused RoPE / append: head rows stay whole and pairs stay in a group */
      if (mode != MV_STORE || !a.rope.cs || a.rope.head_dim <= 0 || (a.rope.head_dim & 1) ||
          a.rope.head_dim > 512 || sg.rows % a.rope.head_dim)
        return -1;
    }
    if (sg.rows & 1) { /* an odd segment would shift the pairs of the next one */
      for (int k = i + 1; k < a.nseg; k++)
        if (a.seg[k].kind != SEG_PLAIN && a.seg[k].kind != SEG_KV) return -1;
    }
    total += sg.rows;
  }
  return total;
}

template <int DT>
int launch_dt(int mode, const MvArgs &a, int total, hipStream_t s) {
  switch (mode) {
  case MV_STORE: return launch_mvx<DT, MV_STORE>(a, total, s);
  case MV_RESID: return launch_mvx<DT, MV_RESID>(a, total, s);
  case MV_SWIGLU: return launch_mvx<DT, MV_SWIGLU>(a, total, s);
  default: return -1;
  }
}

} // namespace

size_t gq_q6k_units_bytes(int rows, int cols) { return (size_t)rows * (size_t)(cols / 256) * 210; }

int gq_launch_q6k_units(void *dst, const void *src, int rows, int cols, hipStream_t s) {
  if (!dst || !src || rows <= 0 || cols <= 0 || cols % 512) return -1; /* an even count of blocks per row */
  const long long n = (long long)rows * (cols / 32);
  hipLaunchKernelGGL(q6k_units_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint8_t *)src,
                     (uint8_t *)dst, rows, cols / 256);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

extern "C" int gq_hip_set_matvec_path(int path) {
  const int prev = g_path;
  if (path >= 0 && path <= 3) g_path = path;
  return prev;
}

bool gq_matvec_mm_forced() { return g_path == 2; }
bool gq_matvec_q6k_ref() { return g_path == 3; }

int gq_launch_matvec(int dtype, int mode, const MvArgs &a, hipStream_t s) {
  if (dtype != GQ_Q4_K && dtype != GQ_Q6_K && dtype != GQ_Q8_0) return -1;
  if (a.cols <= 0 || a.cols % (dtype == GQ_Q8_0 ? 32 : 256)) return -2;
  const int total = check_args(mode, a);
  if (total <= 0) return -1;
  /* the matrix-core kernel where the policy picks it and a tiled copy
   * exists: gate/up + SwiGLU (8B decode: 14.9 us against 16-17 on the
   * vector ALUs) and the LM head (>= 16384 rows) by default */
  const bool mm = a.mm && (dtype == GQ_Q4_K || dtype == GQ_Q6_K) &&
                  (g_path == 2 || ((g_path == 1 || g_path == 3) && (mode == MV_SWIGLU || (mode == MV_STORE && total >= 16384))));
  if (mm) {
    const int rc = gq_launch_mm(dtype, mode, a, s);
    if (rc <= 0) return rc;
  }
  /* Q6_K residual launches with a unit-layout copy (the down projection) */
  if (dtype == GQ_Q6_K && a.dx && g_path != 3 && a.nseg == 1 && mode == MV_RESID && (a.cols / 256) % 2 == 0) {
    MvArgs b = a;
    b.seg[0].w = a.dx;
    return launch_mvx<GQ_Q6_KX, MV_RESID>(b, total, s);
  }
  switch (dtype) {
  case GQ_Q4_K: return launch_dt<GQ_Q4_K>(mode, a, total, s);
  case GQ_Q6_K: return launch_dt<GQ_Q6_K>(mode, a, total, s);
  default: return launch_dt<GQ_Q8_0>(mode, a, total, s);
  }
}

int gq_launch_matvec_pair(int dt0, const MvArgs &a0, int dt1, const MvArgs &a1, hipStream_t s) {
  if (g_path == 2 || dt0 != GQ_Q4_K || dt1 != GQ_Q6_K || a0.cols != a1.cols || a0.cols <= 0 || a0.cols % 256)
    return 1;
  const int t0 = check_args(MV_STORE, a0), t1 = check_args(MV_STORE, a1);
  if (t0 <= 0 || t1 <= 0) return -1;
  /* the Q6_K side from its unit-layout copy when one is given (bit-identical
   * outputs, aligned loads) */
  const bool ux = a1.dx && a1.nseg == 1 && (a1.cols / 256) % 2 == 0 && g_path != 3;
  MvArgs b1 = a1;
  if (ux) b1.seg[0].w = a1.dx;
  MxPlan p0, p1;
  int r0, r1, sw0, sw1, m0, m1;
  plan(GQ_Q4_K, MV_STORE, a0, t0, p0, r0, sw0, m0);
  plan(ux ? GQ_Q6_KX : GQ_Q6_K, MV_STORE, b1, t1, p1, r1, sw1, m1);
  /* one block shape for both sides */
  if (p0.G * p0.L != p1.G * p1.L || sw0 != sw1 || m0 != 256 || m1 != 256 || p0.L % 64) return 1;
  auto launch = [&](auto kern, int ra, int rb) {
    p0.nwg = ((t0 + ra - 1) / ra + p0.G - 1) / p0.G;
    p1.nwg = ((t1 + rb - 1) / rb + p1.G - 1) / p1.G;
    hipLaunchKernelGGL(kern, dim3(p0.nwg + p1.nwg), dim3(p0.G * p0.L), 0, s, a0, p0, b1, p1);
    return hipGetLastError() == hipSuccess ? 0 : -4;
  };
  if (!a0.norm_w != !a1.norm_w) return 1;
  if (sw0 != 16) return 1;
  /* 4-row groups on both sides, as plan() gives the q/k/v launch */
  if (ux && a0.norm_w) return launch(mvx_pair_kernel<GQ_Q4_K, 4, GQ_Q6_KX, 4, 16, 256, kNorm | kShx>, 4, 4);
  if (ux) return launch(mvx_pair_kernel<GQ_Q4_K, 4, GQ_Q6_KX, 4, 16, 256, kShx>, 4, 4);
  if (a0.norm_w) return launch(mvx_pair_kernel<GQ_Q4_K, 4, GQ_Q6_K, 4, 16, 256, kNorm | kShx>, 4, 4);
  return launch(mvx_pair_kernel<GQ_Q4_K, 4, GQ_Q6_K, 4, 16, 256, kShx>, 4, 4);
}
