/*
 * gq_matvec.hip — quantised matvec on the int8 matrix cores (gfx950):
 * mvm_kernel, used by the decode step for gate/up + SwiGLU and the LM head,
 * and the tile-interleaved weight copies it streams (mm_tile_kernel).  The
 * vector-ALU kernel for every other launch, and the dispatch between the
 * two, are in gq_mvx.hip.
 *
 * y = W x with W in the reference's Q4_K / Q6_K block layouts
 * (quant_matvec_q4_k.c:9-16, quant_matvec_q6_k.c:5-12), rows = out_features,
 * x fp32, fused prologue and epilogues as in gq_internal.h.
 */
#include <stdlib.h>

#include <algorithm>

#include "gq_device.h"
#include "gq_internal.h"

namespace {

constexpr int kRing = 8; /* residual-row ring slots (>= ring stages + 1) */

/* Wave `wave`'s 1 KB copy instructions for nbytes (a multiple of 16) split
 * over nwv waves. */
__device__ __forceinline__ int copy_count(int nbytes, int wave, int nwv) {
  const int ng = (nbytes / 16 + 63) / 64;
  return wave < ng ? (ng - wave + nwv - 1) / nwv : 0;
}

/* Rows [src, src + nbytes) into LDS at dst by 16-byte DMA (dma16), 1 KB per
 * wave instruction, instructions dealt round-robin over nwv waves. */
__device__ __forceinline__ void copy_range(const uint8_t *src, int nbytes, GQ_LDS uint8_t *dst, int wave,
                                           int lane, int nwv) {
  const int nchunk = nbytes / 16, ng = (nchunk + 63) / 64;
  const uint32_t base = (uint32_t)(uintptr_t)dst;
  for (int g = wave; g < ng; g += nwv) {
    const int c = g * 64 + lane;
    const uint32_t d = __builtin_amdgcn_readfirstlane(base + (uint32_t)g * 1024u);
    if (c < nchunk) dma16(src + (size_t)c * 16, d);
  }
}


/* Destination of output row lr of segment s (nullptr: position rejected). */
template <int MODE>
__device__ __forceinline__ float *rdest(const MvArgs &a, const MvSegs &sv, int s, int lr, int pos) {
  if (MODE == MV_SWIGLU) return sv.y0 + lr;
  float *const y = gq_mv_y(sv, s);
  const int kind = gq_mv_kind(sv, s);
  if (MODE == MV_RESID || kind == SEG_PLAIN || kind == SEG_ROPE) return y + lr;
  if (pos < 0 || pos >= a.rope.max_seq) return nullptr; /* rejected on the host */
  const int hd = a.rope.head_dim, h = lr / hd, d = lr - h * hd;
  return y + ((size_t)h * a.rope.max_seq + pos) * hd + d;
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
  int red;          /* NB: LDS offset of the tiles' per-wave row sums (16 x NW floats per tile) */
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
template <int MODE, int NW, int BB, bool NB>
__device__ __forceinline__ int mm_issue(const MvArgs &a, const MvSegs &sv, const MmPlan &pl, int t, int c,
                                        GQ_LDS uint8_t *buf, GQ_LDS float *rbuf, int wave, int lane) {
  if constexpr (NB) {
    /* only the blocks this wave computes (wave + s NW of the stage), each 16
     * rows x BB bytes contiguous, so no other wave reads what it copies */
    constexpr int RB = 16 * BB, NI = (RB + 1023) / 1024;
    const uint8_t *src = a.mm + ((size_t)t * pl.nb + (size_t)c * pl.cb) * RB;
    const uint32_t base = (uint32_t)(uintptr_t)buf;
    int cnt = 0;
    for (int sb = 0; sb < pl.bpc; sb++) {
      const int bl = wave + sb * NW;
      if (bl >= pl.cb) break;
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const uint32_t o = (uint32_t)(bl * RB + i * 1024);
        const uint32_t d = __builtin_amdgcn_readfirstlane(base + o);
        if (i * 1024 + 16 * lane < RB) dma16(src + o + 16 * lane, d);
        cnt++;
      }
    }
    return cnt;
  }
  const int sb = 16 * BB * pl.cb;
  copy_range(a.mm + ((size_t)t * pl.nb + (size_t)c * pl.cb) * (16 * BB), sb, buf, wave, lane, NW);
  int cnt = copy_count(sb, wave, NW);
  if (MODE == MV_RESID && c == 0 && wave == NW - 1) {
    int s, lr0;
    gq_mv_locate(sv, 16 * t, s, lr0);
    const int last = gq_mv_rows(sv, s) - 1;
    const uint32_t d = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)rbuf);
    if (lane < 16) dma4(gq_mv_r(sv, s) + min(lr0 + lane, last), d);
    cnt++;
  }
  return cnt;
}

/* AREG: the wave's A operands live in registers for the whole launch (up to
 * MAXB blocks, every chunk); otherwise the digit planes stay in LDS (up to
 * 8 blocks per wave) and each stage loads the A operands of its MAXB
 * blocks per wave, for rows longer than registers hold. */
template <int DT, int MODE, int NW, int MAXB, int NS, bool AREG, bool NB>
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
  const MvSegs sv = gq_mv_segs(a);
  const int mytiles = bid < pl.ntiles ? (pl.ntiles - 1 - bid) / nblk + 1 : 0;
  const int nst = mytiles * pl.nch;
  auto issue = [&](int q) -> int { /* stage q into slot q % NS */
    const int tl = q / pl.nch;
    return mm_issue<MODE, NW, T::BB, NB>(a, sv, pl, bid + tl * nblk, q - tl * pl.nch, lds + (q % NS) * pl.stride,
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
    /* NB: only the first (x converted by every wave before stages land in its
     * slots; the sums of squares): each wave reads only what it copied */
    if (!NB || k == 0) __syncthreads();
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
    if (!NB && k > 0 && c == 0 && lane < RPW) { /* rows of the tile completed at k-1 */
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
            out = gq_silu_mul(v, w);
          } else if (MODE == MV_RESID) {
            out = v + sh.rres[tl % kRing][r];
          } else if (a.rope.cs) {
            int s, lr0;
            gq_mv_locate(sv, 16 * (bid + tl * nblk), s, lr0);
            const int kind = gq_mv_kind(sv, s);
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
      if (lane < 16) {
        if constexpr (NB)
          lst<float>(lds, (uint32_t)pl.red + 4u * (uint32_t)(((k / pl.nch) * 16 + lane) * NW + wave), v);
        else
          sh.red[(k / pl.nch) & 1][lane][wave] = v;
      }
      acc = 0.f;
    }
  }
  __syncthreads();
  if constexpr (NB) {
    /* plain stores only (the launcher takes NB for MV_STORE without RoPE):
     * every wave's row sums of every tile are in; wave w finishes and stores
     * tiles w, w + NW, ... (lane r: row r), the sums in the same order */
    for (int tl = wave; tl < mytiles; tl += NW) {
      const int t = bid + tl * nblk, r = lane;
      int s = 0, lr = 0;
      gq_mv_locate(sv, 16 * t, s, lr);
      s = __builtin_amdgcn_readfirstlane(s);
      lr = __builtin_amdgcn_readfirstlane(lr) + r;
      if (r >= 16 || lr >= gq_mv_rows(sv, s)) continue;
      float v = 0.f;
#pragma unroll
      for (int j = 0; j < NW; j++) v += lld<float>(lds, (uint32_t)pl.red + 4u * (uint32_t)((tl * 16 + r) * NW + j));
      float *dst = rdest<MODE>(a, sv, s, lr, pos);
      if (dst) gst<float>(dst, v * rscale);
    }
    return;
  }
  /* the parked rows go out: wave w stores tiles w, w + NW, ..., so the
   * segment of a tile is uniform across the wave */
  const int prow = MODE == MV_SWIGLU ? 8 : 16;
  for (int tl = wave; tl < mytiles; tl += NW) {
    const int t = bid + tl * nblk, r = lane;
    int s = 0, lr = 8 * t + r;
    if (MODE != MV_SWIGLU) {
      gq_mv_locate(sv, 16 * t, s, lr);
      s = __builtin_amdgcn_readfirstlane(s);
      lr = __builtin_amdgcn_readfirstlane(lr) + r;
      if (r >= prow || lr >= gq_mv_rows(sv, s)) continue;
    } else if (r >= prow || lr >= pl.total) {
      continue;
    }
    float *dst = rdest<MODE>(a, sv, s, lr, pos);
    if (dst) gst<float>(dst, park[16 * tl + r]);
  }
}

int g_n_cu = 256;
constexpr size_t kMaxDynLdsW = 152 * 1024;

/* Plan and launch the matrix-core kernel; returns 1 when the shape does not
 * fit it (a dtype without int8 traits, segments a 16-row tile would
 * straddle, rows not a multiple of 16 bytes, or x not fitting the ring's
 * last slot during the prologue). */
constexpr int kMmWaves = 8; /* waves per workgroup (4 measured 18.4-19.0 us on gate/up against 14.9) */
constexpr size_t kMmLds = 160 * 1024; /* LDS of a CU (gfx950) */
constexpr int kMmNs = 3;    /* ring slots (4 and 6 measured slower: 16.5 and 20.0 us on gate/up) */
constexpr int kMmStageCap = 40960; /* bytes of weights per stage at most */
/* Plain-store workgroups (no RoPE, no residual) that run at least this many
 * stages drop the per-stage barrier: each wave copies only the blocks it
 * computes and the tiles are finished after the loop.  The LM head (64 stages a workgroup at the 8B shape)
 * measured 88-89 -> 81-84 us; gate/up (7 stages) 14.8 -> 15.4 us, so it
 * keeps the barrier. */
constexpr int kMmNbStages = 16;

template <int DT, int MODE, int NW, int MAXB, int NS, bool AREG = true, bool NB = false>
int launch_mm_as(const MvArgs &a, const MmPlan &pl, size_t lds, int grid, hipStream_t s) {
  static bool attr_set = false;
  auto f = mvm_kernel<DT, MODE, NW, MAXB, NS, AREG, NB>;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDynLdsW);
    (void)hipGetLastError(); /* a refusal shows up as the launch's error instead */
    attr_set = true;
  }
  hipLaunchKernelGGL(f, dim3(grid), dim3(NW * GQ_WAVE), lds, s, a, pl);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <int DT, int MODE, int NW, int NS>
int launch_mm_b(int maxb, bool areg, bool nb, const MvArgs &a, const MmPlan &pl, size_t lds, int grid,
                hipStream_t s) {
  if (!areg) return pl.bpc <= 1 ? launch_mm_as<DT, MODE, NW, 1, NS, false>(a, pl, lds, grid, s)
                                : launch_mm_as<DT, MODE, NW, 2, NS, false>(a, pl, lds, grid, s);
  if constexpr (MODE == MV_STORE) {
    if (nb) {
      if (maxb <= 1) return launch_mm_as<DT, MODE, NW, 1, NS, true, true>(a, pl, lds, grid, s);
      if (maxb <= 2) return launch_mm_as<DT, MODE, NW, 2, NS, true, true>(a, pl, lds, grid, s);
      return launch_mm_as<DT, MODE, NW, 4, NS, true, true>(a, pl, lds, grid, s);
    }
  }
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
  while (cb > 1 && (16 * cb * T::BB > kMmStageCap || pl.nb % cb)) cb--;
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
  int ns = std::max(kMmNs, pl.xslots + 1);
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
  bool nb = false;
  for (int pc = 2; pc >= 1 && !grid; pc--) {
    const int gr = std::min(pl.ntiles, pc * g_n_cu);
    const size_t tpw = (size_t)((pl.ntiles + gr - 1) / gr);
    /* NB (no barrier per stage, the tiles finished after the loop) where a
     * workgroup runs at least kMmNbStages stages; it needs 16 x NW floats of
     * row sums per tile */
    nb = MODE == MV_STORE && !a.rope.cs && areg && tpw * pl.nch >= (size_t)kMmNbStages;
    const size_t l = (size_t)pl.park + 64 * tpw + (nb ? (size_t)64 * NW * tpw : 0);
    if (l <= kMaxDynLdsW && pc * (l + shb + 1024) <= kMmLds + 1024) grid = gr, lds = l, pl.red = pl.park + 64 * (int)tpw;
  }
  if (!grid) return 1;
  if (ns == 3) return launch_mm_b<DT, MODE, NW, 3>(maxb, areg, nb, a, pl, lds, grid, s);
  if (ns == 4) return launch_mm_b<DT, MODE, NW, 4>(maxb, areg, nb, a, pl, lds, grid, s);
  return launch_mm_b<DT, MODE, NW, 6>(maxb, areg, nb, a, pl, lds, grid, s);
}

template <int DT, int MODE>
int launch_mm(const MvArgs &a, int total, hipStream_t s) {
  if constexpr (DT != GQ_Q4_K && DT != GQ_Q6_K) {
    return 1;
  } else {
    if (!a.mm) return 1;
    return launch_mm_w<DT, MODE, kMmWaves>(a, total, s);
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

} // namespace

void gq_matvec_set_cus(int n_cu) {
  if (n_cu > 0) g_n_cu = n_cu;
}

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

int gq_launch_mm(int dtype, int mode, const MvArgs &a, hipStream_t s) {
  int total = 0;
  if (mode == MV_SWIGLU) {
    total = a.seg[0].rows;
  } else {
    for (int i = 0; i < a.nseg; i++) total += a.seg[i].rows;
  }
  if (total <= 0) return -1;
  switch (dtype * 4 + mode) {
  case GQ_Q4_K * 4 + MV_STORE: return launch_mm<GQ_Q4_K, MV_STORE>(a, total, s);
  case GQ_Q4_K * 4 + MV_RESID: return launch_mm<GQ_Q4_K, MV_RESID>(a, total, s);
  case GQ_Q4_K * 4 + MV_SWIGLU: return launch_mm<GQ_Q4_K, MV_SWIGLU>(a, total, s);
  case GQ_Q6_K * 4 + MV_STORE: return launch_mm<GQ_Q6_K, MV_STORE>(a, total, s);
  case GQ_Q6_K * 4 + MV_RESID: return launch_mm<GQ_Q6_K, MV_RESID>(a, total, s);
  case GQ_Q6_K * 4 + MV_SWIGLU: return launch_mm<GQ_Q6_K, MV_SWIGLU>(a, total, s);
  default: return 1;
  }
}
