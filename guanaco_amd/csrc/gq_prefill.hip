/*
 * gq_prefill.hip — the prefill chunk (many tokens at once) on gfx950: a
 * K-quant x activations GEMM on the bf16 matrix cores, with fp32
 * accumulation.
 *
 * The reference computes a prefill projection as T sequential matvecs
 * (linear_dispatch, engine.c:119-152).  Here Y[T][N] = X[T][K] . W^T for
 * all T tokens in one launch, where W is N rows of Q4_K blocks
 * (quant_matvec_q4_k.c:9-16), Q6_K blocks (quant_matvec_q6_k.c:5-12) or Q8_0
 * blocks (quant_matvec_q8_0.c:5-10) and
 * X is bf16 row-major (its producer rounds it: RMSNorm, the attention merge,
 * the gate/up epilogue, or the fp32 -> bf16 pass of the op-level entry).
 *
 * Workgroup tile: 64 tokens x 128 weight rows, 4 waves; wave w owns rows
 * 32w .. 32w+31 of the tile for all 64 tokens, i.e. two 32x32 tiles of
 * v_mfma_f32_32x32x16_bf16.  K advances 64 weights per step: one Q4_K chunk
 * of two sub-blocks, or two 32-weight groups of a Q6_K half-block.
 *
 * Every step's inputs stream into an LDS ring kRing - 1 steps ahead by direct
 * global -> LDS DMA (no VGPRs, no VALU):
 *   X  8 KB per step: each DMA instruction moves 8 tokens' whole 128-byte
 *      k-slices (8 full cache lines), stored [token][k-octet] with the
 *      octet position XOR-swizzled by (token / 2) % 8, so each MFMA A
 *      operand (32 tokens, one octet) is a conflict-free ds_read_b128;
 *   W  each wave's own 32 rows, raw block bytes (Q4_K: header + the 32 quant
 *      bytes of the chunk; Q6_K: a dword-aligned window over ql, qh, scales
 *      and d of the half-block).
 * Each lane dequantizes exactly the 32 weights of its own B operands (its
 * row, its k-octets), so a weight is converted once per token tile and never
 * round-trips through LDS in bf16.  One barrier per step.
 *
 * The fused Q4_K gate/up launch runs a wide variant of the tile when its grid
 * fills the GPU: 64 rows per wave, so each A operand read feeds two MFMAs
 * (pgemm_wide_swiglu_kernel).
 *
 * MFMA operand layout (32x32x16, checked on the device): A[i][k] is element
 * k % 8 of lane i + 32 (k / 8); B[k][j] element k % 8 of lane j + 32 (k / 8);
 * D[i][j] element 4 (i / 8) + i % 4 of lane j + 32 ((i / 4) % 2).
 */
#include <algorithm>
#include <cstdlib>

#include "gq_device.h"
#include "gq_internal.h"

namespace {

typedef __bf16 gq_bf16x8 __attribute__((ext_vector_type(8)));
typedef float gq_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPThreads = 256;
constexpr int kBN = 128, kBK = 64;
/* K parts of a launch split over the grid (PgArgs.part) */
constexpr int kKParts = kPgKParts;
/* TT 32-token MFMA tiles per wave (the token tile is 32 TT); X bytes per
 * step of one K-split */
template <int TT>
constexpr int x_bytes() {
  return 32 * TT * kBK * 2;
}

typedef float gq_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 gq_bf2 __attribute__((ext_vector_type(2)));

/* two floats to a bf16 pair, round to nearest even: one v_cvt_pk_bf16_f32 */
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((gq_f2){lo, hi}, gq_bf2));
}

/* Per-dtype W staging.  Lane (row r = lane % 32 of the wave's 32, h =
 * lane / 32) builds B operands b[kk] = its row's weights k = 16 kk + 8 h + i
 * (i < 8) of the step's 64. */
template <int DT>
struct PW;

/* Q4_K: per row and step 48 bytes in LDS: the 16-byte block header, then
 * the 32 quant bytes of chunk cc = s % 4 (weights 64 cc .. 64 cc + 63 of the
 * super-block: sub-block 2cc in the low nibbles, 2cc+1 in the high ones). */
template <>
struct PW<GQ_Q4_K> {
  static constexpr int BB = 144;
  static constexpr int kRowLds = 48;
  static constexpr int kWaveLds = 2048; /* two 1-KB DMA instructions (96 pieces used) */
  static constexpr int kDma = 2;        /* W DMA instructions per wave and step */
  struct Plan {
    uint32_t off[2]; /* per instruction: row * rowbytes + offset in the block */
    bool qs[2];      /* quant bytes (move with the chunk) or header */
    bool on[2];
  };
  __device__ static void plan(Plan &p, int lane, uint32_t rowbytes) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int pc = 64 * i + lane, row = pc / 3, part = pc - 3 * row;
      p.on[i] = pc < 96;
      p.qs[i] = part != 0;
      p.off[i] = (uint32_t)row * rowbytes + (part ? 16u * (uint32_t)part : 0u);
    }
  }
  __device__ static void issue(const Plan &p, const uint8_t *w, int s, uint32_t lds) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint8_t *src = w + p.off[i] + (size_t)(s >> 2) * BB + (p.qs[i] ? 32 * (s & 3) : 0);
      const uint32_t d = __builtin_amdgcn_readfirstlane(lds + 1024u * i);
      if (p.on[i]) dma16(src, d);
    }
  }
  /* scale/min decode as in the matvec (quant_matvec_q4_k.c:47-56); weight
   * fp32(d sc q - dmin m) with one rounding (the fma), then bf16.  Nibbles go
   * to float as OCP E4M3 (exactly q 2^-9), the 2^9 folded into d sc. */
  struct Raw {
    uint4 hd;
    uint2 q0, q1;
  };
  __device__ static void read(Raw &w, const GQ_LDS uint8_t *ws, int lane, int s) {
    const uint32_t r = (uint32_t)(lane & 31), h = (uint32_t)(lane >> 5);
    (void)s;
    w.hd = lld<uint4>(ws, r * kRowLds);
    w.q0 = lld<uint2>(ws, r * kRowLds + 16u + 8u * h);
    w.q1 = lld<uint2>(ws, r * kRowLds + 32u + 8u * h);
  }
  __device__ static void dequant(const Raw &rw, int s, gq_bf16x8 b[4]) {
    const uint4 hd = rw.hd;
    const uint2 q0 = rw.q0, q1 = rw.q1;
    const int cc = s & 3;
    const float d = gq_h2f(hd.x), dm = gq_h2f(hd.x >> 16);
    const uint32_t sh = 16u * (uint32_t)(cc & 1);
    const bool hi = cc >= 2;
    const uint32_t y = hd.y >> sh, z = hd.z >> sh, w = hd.w >> sh;
    const uint32_t mlo = hi ? 0x0f0fu : 0x3f3fu, mhi = hi ? 0x3030u : 0u;
    const uint32_t S = ((hi ? w : y) & mlo) | ((y >> 2) & mhi);
    const uint32_t M = ((hi ? (w >> 4) : z) & mlo) | ((z >> 2) & mhi);
    const float a0 = d * (float)(S & 0xffu), m0 = dm * (float)(M & 0xffu);
    const float a1 = d * (float)((S >> 8) & 0xffu), m1 = dm * (float)((M >> 8) & 0xffu);
    const float A0 = a0 * 512.0f, A1 = a1 * 512.0f;
    const uint32_t src[4][2] = {{q0.x, q0.y}, {q1.x, q1.y}, {q0.x >> 4, q0.y >> 4}, {q1.x >> 4, q1.y >> 4}};
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const float A = kk < 2 ? A0 : A1, m = kk < 2 ? m0 : m1;
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const uint32_t n = src[kk][k] & 0x0f0f0f0fu;
        const gq_f32x2 f0 = gq_nib2f<false>(n), f1 = gq_nib2f<true>(n);
        o[2 * k] = pack_bf16x2(__builtin_fmaf(A, f0.x, -m), __builtin_fmaf(A, f0.y, -m));
        o[2 * k + 1] = pack_bf16x2(__builtin_fmaf(A, f1.x, -m), __builtin_fmaf(A, f1.y, -m));
      }
      b[kk] = __builtin_bit_cast(gq_bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
    }
  }
};

/* Q6_K (quant_matvec_q6_k.c:70-90): weight 128 n + 32 g + l (half n, group
 * g < 4, l < 32) has q = (ql[64 n + 32 (g & 1) + l] >> 4 (g >> 1)) & 15
 * | ((qh[32 n + l] >> 2 g) & 3) << 4, minus 32, scale scales[8 n + 2 g +
 * l / 16]; w = (d sc) q, exact in fp32.  Step chunk cc = 2 n + par holds
 * groups 2 par and 2 par + 1 of half n.  Blocks are 210 bytes, so only
 * 2-byte aligned; rows are 4-byte aligned (cols % 512 == 0).  Per row and
 * step 30 dwords of the block window aligned down to 4 bytes, in LDS as
 *   ql[64 n - sh ..] 17 dwords | qh[32 n - sh ..] 9 | scales[8 n - sh ..] 3
 *   | d 1,   sh = block offset & 3 (0 or 2). */
template <>
struct PW<GQ_Q6_K> {
  static constexpr int BB = 210;
  static constexpr int kRowLds = 120;
  static constexpr int kWaveLds = 15 * 256; /* 15 dword instructions */
  static constexpr int kDma = 15;
  struct Plan {
    uint32_t off[15]; /* row * rowbytes + 4 * window dword (half 0) */
    uint32_t dn[15];  /* extra bytes for half 1 */
  };
  __device__ static void plan(Plan &p, int lane, uint32_t rowbytes) {
#pragma unroll
    for (int i = 0; i < 15; i++) {
      const int dw = 64 * i + lane, row = dw / 30, w = dw - 30 * row;
      const int idx = w < 17 ? w : w < 26 ? 32 + (w - 17) : w < 29 ? 48 + (w - 26) : 52;
      p.off[i] = (uint32_t)row * rowbytes + 4u * (uint32_t)idx;
      p.dn[i] = w < 17 ? 64u : w < 26 ? 32u : w < 29 ? 8u : 0u;
    }
  }
  __device__ static void issue(const Plan &p, const uint8_t *w, int s, uint32_t lds) {
    const size_t blk = ((size_t)(s >> 2) * BB) & ~(size_t)3;
    const bool n1 = (s & 2) != 0;
#pragma unroll
    for (int i = 0; i < 15; i++) {
      const uint32_t d = __builtin_amdgcn_readfirstlane(lds + 256u * i);
      dma4(w + blk + p.off[i] + (n1 ? p.dn[i] : 0u), d);
    }
  }
  struct Raw {
    uint2 P[4], H0, H1;
    uint32_t sc, d;
  };
  __device__ static void read(Raw &w, const GQ_LDS uint8_t *ws, int lane, int s) {
    const uint32_t r = (uint32_t)(lane & 31), h = (uint32_t)(lane >> 5);
    const uint32_t sh = 2u * (uint32_t)((s >> 2) & 1), par = (uint32_t)(s & 1);
    const uint32_t base = r * kRowLds + sh;
#pragma unroll
    for (int k = 0; k < 4; k++) w.P[k] = lld8_a2(ws, base + 16u * k + 8u * h);
    w.H0 = lld8_a2(ws, base + 68u + 8u * h);
    w.H1 = lld8_a2(ws, base + 84u + 8u * h);
    w.sc = lld8_a2(ws, base + 104u + 4u * par).x;
    w.d = lld<uint16_t>(ws, base + 116u);
  }
  __device__ static void dequant(const Raw &rw, int s, gq_bf16x8 b[4]) {
    const uint32_t par = (uint32_t)(s & 1);
    const uint2 *P = rw.P, H0 = rw.H0, H1 = rw.H1;
    const uint32_t sc = rw.sc;
    const float d = gq_h2f(rw.d);
    const uint32_t sa = 4u * par;
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const uint2 Hq = (kk & 1) ? H1 : H0;
      const uint32_t hs = sa + ((kk >= 2) ? 2u : 0u);
      const float a = d * (float)(int8_t)((sc >> (8 * kk)) & 0xffu);
      const float m = 32.0f * a;
      const uint32_t pw[2] = {P[kk].x, P[kk].y}, hw[2] = {Hq.x, Hq.y};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const uint32_t u = ((pw[k] >> sa) & 0x0f0f0f0fu) | (((hw[k] >> hs) & 0x03030303u) << 4);
        const float v0 = __builtin_fmaf(a, (float)(u & 0xffu), -m);
        const float v1 = __builtin_fmaf(a, (float)((u >> 8) & 0xffu), -m);
        const float v2 = __builtin_fmaf(a, (float)((u >> 16) & 0xffu), -m);
        const float v3 = __builtin_fmaf(a, (float)(u >> 24), -m);
        o[2 * k] = pack_bf16x2(v0, v1);
        o[2 * k + 1] = pack_bf16x2(v2, v3);
      }
      b[kk] = __builtin_bit_cast(gq_bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
    }
  }
};


/* Q6_K in the decode matvec's unit layout (gq_launch_q6k_units; made once
 * at model bind, and read here too for rows on 16-byte boundaries, K % 2048
 * == 0).  Unit u (block u/8, half n, group v) holds the 16 ql bytes whose
 * low nibbles are weights 128 n + 16 v + i and high nibbles 128 n + 64 +
 * 16 v + i (i < 16), then two dwords of their 2-bit fields; its two int8
 * scales at 192 nb + 2u; the block's d at 208 nb + 2 (u/8).  Step s = 4 b +
 * 2 n + p takes units 8 b + 4 n + 2 p and the next: 48 contiguous quant
 * bytes at 48 s, 4 scale bytes at 192 nb + 4 s.  Its 64 weights are not
 * consecutive columns: k-octets 0-3 are the two units' low nibbles, columns
 * 256 b + 128 n + 32 p + 0..31, and octets 4-7 their high nibbles, the same
 * plus 64: k-octet o of step s is columns 64 s - 32 (s & 1) + 8 o (+32 for
 * o >= 4), and the X staging of this type fetches those.  Per weight w = (d sc) q - 32 (d sc) with PW<GQ_Q6_K>'s
 * roundings, so the bf16 weights are the reference layout's; only the order
 * of the K sums differs. */
template <>
struct PW<GQ_Q6_KX> {
  static constexpr int kWaveLds = 2048 + 256; /* quants (96 16-byte pieces), then 32 scale + 32 d dwords */
  static constexpr int kDma = 3;
  struct Plan {
    uint32_t off[3];
    bool on[2];
    bool dlane; /* lanes 32..63 of the dword instruction fetch the d pair */
  };
  __device__ static void plan(Plan &p, int lane, uint32_t rowbytes) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int pc = 64 * i + lane, row = pc / 3, part = pc - 3 * row;
      p.on[i] = pc < 96;
      p.off[i] = (uint32_t)row * rowbytes + 16u * (uint32_t)part;
    }
    const uint32_t nb = rowbytes / 210u;
    p.dlane = lane >= 32;
    p.off[2] = (uint32_t)(lane & 31) * rowbytes + (p.dlane ? 208u : 192u) * nb;
  }
  __device__ static void issue(const Plan &p, const uint8_t *w, int s, uint32_t lds) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t d = __builtin_amdgcn_readfirstlane(lds + 1024u * i);
      if (p.on[i]) dma16(w + p.off[i] + (size_t)48 * s, d);
    }
    dma4(w + p.off[2] + (p.dlane ? 4u * (uint32_t)(s >> 3) : 4u * (uint32_t)s),
         __builtin_amdgcn_readfirstlane(lds + 2048u));
  }
  struct Raw {
    uint2 q0, q1;      /* ql bytes 8 h .. 8 h + 7 of the two units */
    uint32_t h0, h1;   /* their 2-bit fields (dword h of each unit's pair) */
    uint32_t sc, dd;
  };
  __device__ static void read(Raw &w, const GQ_LDS uint8_t *ws, int lane, int) {
    const uint32_t r = (uint32_t)(lane & 31), h = (uint32_t)(lane >> 5);
    w.q0 = lld<uint2>(ws, 48u * r + 8u * h);
    w.h0 = lld<uint32_t>(ws, 48u * r + 16u + 4u * h);
    w.q1 = lld<uint2>(ws, 48u * r + 24u + 8u * h);
    w.h1 = lld<uint32_t>(ws, 48u * r + 40u + 4u * h);
    w.sc = lld<uint32_t>(ws, 2048u + 4u * r);
    w.dd = lld<uint32_t>(ws, 2176u + 4u * r);
  }
  /* b[kk]: octet 2 kk + h = unit kk & 1, low (kk < 2) or high nibbles of
   * its quant dwords 2h, 2h + 1; the unit decode of the matvec
   * (Ux<GQ_Q6_KX>::dot): 6-bit q = nibble | field << 4 */
  __device__ static void dequant(const Raw &rw, int s, gq_bf16x8 b[4]) {
    const float d = gq_h2f(rw.dd >> (16u * (uint32_t)((s >> 2) & 1)));
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const int un = kk & 1;
      const bool hi = kk >= 2;
      /* scale bytes: unit 0 (low, high), unit 1 (low, high) */
      const float a = d * (float)(int8_t)((rw.sc >> (8 * (2 * un + (hi ? 1 : 0)))) & 0xffu);
      const float m = 32.0f * a;
      const uint2 q = un ? rw.q1 : rw.q0;
      const uint32_t hf = un ? rw.h1 : rw.h0;
      const uint32_t qw[2] = {q.x, q.y}, fw[2] = {hf, hf >> 2};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const uint32_t u = hi ? (((qw[k] >> 4) & 0x0F0F0F0Fu) | (fw[k] & 0x30303030u))
                              : ((qw[k] & 0x0F0F0F0Fu) | ((fw[k] << 4) & 0x30303030u));
        const float v0 = __builtin_fmaf(a, (float)(u & 0xffu), -m);
        const float v1 = __builtin_fmaf(a, (float)((u >> 8) & 0xffu), -m);
        const float v2 = __builtin_fmaf(a, (float)((u >> 16) & 0xffu), -m);
        const float v3 = __builtin_fmaf(a, (float)(u >> 24), -m);
        o[2 * k] = pack_bf16x2(v0, v1);
        o[2 * k + 1] = pack_bf16x2(v2, v3);
      }
      b[kk] = __builtin_bit_cast(gq_bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
    }
  }
};

/* Q8_0 (quant_matvec_q8_0.c:5-10): 34-byte blocks of an fp16 d and 32 int8
 * quants, w = d q (exact in fp32: 11 x 8 significant bits).  A 64-weight
 * step is two whole blocks, 68 bytes, and rows of K % 64 == 0 weights are
 * 68 K / 64 bytes, so every step starts on a dword: per row and step the 17
 * dwords land in LDS as they are (nine dword DMA instructions per wave, 544
 * of 576 lanes used).  Lane (r, h) reads quants 16 kk + 8 h .. + 7 of the
 * step, 2-byte aligned, as three dwords and a funnel shift. */
template <>
struct PW<GQ_Q8_0> {
  static constexpr int kRowLds = 68;
  static constexpr int kWaveLds = 9 * 256;
  static constexpr int kDma = 9;
  struct Plan {
    uint32_t off[9]; /* row * rowbytes + 4 * dword of the row's step */
    bool on[9];
  };
  __device__ static void plan(Plan &p, int lane, uint32_t rowbytes) {
#pragma unroll
    for (int i = 0; i < 9; i++) {
      const int dw = 64 * i + lane, row = dw / 17, w = dw - 17 * row;
      p.on[i] = dw < 32 * 17;
      p.off[i] = (uint32_t)row * rowbytes + 4u * (uint32_t)w;
    }
  }
  __device__ static void issue(const Plan &p, const uint8_t *w, int s, uint32_t lds) {
#pragma unroll
    for (int i = 0; i < 9; i++) {
      const uint32_t d = __builtin_amdgcn_readfirstlane(lds + 256u * i);
      if (p.on[i]) dma4(w + (size_t)68 * s + p.off[i], d);
    }
  }
  struct Raw {
    uint2 q[4];
    uint32_t d0, d1;
  };
  __device__ static void read(Raw &w, const GQ_LDS uint8_t *ws, int lane, int) {
    const uint32_t r = (uint32_t)(lane & 31), h = (uint32_t)(lane >> 5), base = r * kRowLds + 8u * h;
    /* block kk / 2, quants 16 (kk & 1) + 8 h .. after the block's 2-byte d:
     * bytes 2 + 16 kk + 8 h of block 0 (2 mod 4), 36 + 16 (kk - 2) + 8 h of
     * block 1 (dword aligned) */
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      const uint32_t a = base + 16u * (uint32_t)kk;
      const uint32_t w0 = lld<uint32_t>(ws, a), w1 = lld<uint32_t>(ws, a + 4u), w2 = lld<uint32_t>(ws, a + 8u);
      w.q[kk] = make_uint2(__builtin_amdgcn_alignbyte(w1, w0, 2), __builtin_amdgcn_alignbyte(w2, w1, 2));
      w.q[kk + 2] = make_uint2(lld<uint32_t>(ws, a + 36u), lld<uint32_t>(ws, a + 40u));
    }
    w.d0 = lld<uint32_t>(ws, r * kRowLds);
    w.d1 = lld<uint32_t>(ws, r * kRowLds + 32u) >> 16;
  }
  /* d q as d (q + 128) - 128 d in one fma: both products exact, so the
   * result is d q exactly, then bf16 */
  __device__ static void dequant(const Raw &rw, int, gq_bf16x8 b[4]) {
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      const float d = gq_h2f(kk < 2 ? rw.d0 : rw.d1), m = -128.0f * d;
      const uint32_t pw[2] = {rw.q[kk].x ^ 0x80808080u, rw.q[kk].y ^ 0x80808080u};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const float v0 = __builtin_fmaf(d, (float)(pw[k] & 0xffu), m);
        const float v1 = __builtin_fmaf(d, (float)((pw[k] >> 8) & 0xffu), m);
        const float v2 = __builtin_fmaf(d, (float)((pw[k] >> 16) & 0xffu), m);
        const float v3 = __builtin_fmaf(d, (float)(pw[k] >> 24), m);
        o[2 * k] = pack_bf16x2(v0, v1);
        o[2 * k + 1] = pack_bf16x2(v2, v3);
      }
      b[kk] = __builtin_bit_cast(gq_bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
    }
  }
};

/* KS = 1 or 2 K-splits per workgroup: with KS = 2, eight waves, the second
 * four running the upper half of K for the same tile; their sums are added
 * through LDS at the end.  Two waves per SIMD hide each other's LDS, DMA and
 * MFMA latencies.  TT = 2 or 4 token tiles per wave: each dequantized B
 * operand feeds TT MFMAs. */
template <int DT, int KS, int TT>
constexpr int stage_bytes() {
  return KS * x_bytes<TT>() + 4 * KS * PW<DT>::kWaveLds;
}

/* Steps in the LDS ring: as deep as LDS (160 KB) and the 6-bit vmcnt allow
 * (each wave keeps (ring - 2) steps of DMA instructions in flight while it
 * waits), at least 3 (the pipeline reads two slots).  The four-wave shape
 * with 128-token tiles (KS 1, TT 4: 24 KB stages) takes 3 slots, 72 KB, so
 * two workgroups share a CU (two waves per SIMD): gate/up at 512 tokens ran
 * 265 -> 200 us against 4 slots and one workgroup per CU. */
template <int DT, int KS, int TT>
constexpr int ring() {
  return std::min(KS == 1 && TT == 4 ? 3 : 4, (160 * 1024) / stage_bytes<DT, KS, TT>());
}
template <int DT, int KS, int TT>
constexpr int ring_bytes() {
  return ring<DT, KS, TT>() * stage_bytes<DT, KS, TT>();
}
template <int DT, int KS, int TT>
constexpr bool fits() {
  return ring<DT, KS, TT>() >= 3 && (ring<DT, KS, TT>() - 2) * (TT + PW<DT>::kDma) < 64;
}
static_assert(fits<GQ_Q4_K, 1, 2>() && fits<GQ_Q4_K, 2, 2>() && fits<GQ_Q6_K, 1, 2>() && fits<GQ_Q6_K, 2, 2>() &&
                  fits<GQ_Q6_KX, 1, 2>() && fits<GQ_Q6_KX, 2, 2>() &&
                  fits<GQ_Q4_K, 1, 4>() && fits<GQ_Q4_K, 2, 4>() && fits<GQ_Q8_0, 1, 2>() && fits<GQ_Q8_0, 2, 2>() &&
                  fits<GQ_Q8_0, 1, 4>() && fits<GQ_Q8_0, 2, 4>(),
              "ring shapes");

/* One tile: tokens t0 .. t0 + 32 TT - 1 against this wave's 32 rows starting
 * at w, K-split kh of KS.  acc[i] holds tokens t0 + 32 i + (D layout rows)
 * for row (lane & 31). */
template <int DT, int KS, int TT>
__device__ __forceinline__ void tile_loop(const PgArgs &a, const uint8_t *w, uint32_t rowbytes, int t0,
                                          GQ_LDS uint8_t *smem, gq_f32x16 (&acc)[TT]) {
  constexpr int SB = stage_bytes<DT, KS, TT>();
  constexpr int XB = x_bytes<TT>();
  constexpr int NPS = TT + PW<DT>::kDma; /* DMA instructions per wave and step */
  constexpr int kRing = ring<DT, KS, TT>();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = wave >> 2, rw = wave & 3;
  /* this wave's steps s0 .. s0 + ns - 1: K part blockIdx.z of a.kparts,
   * then split kh of KS within the workgroup */
  const int nsp = a.K / kBK / a.kparts, ns = nsp / KS, s0 = (int)blockIdx.z * nsp + kh * ns;
  typename PW<DT>::Plan pl;
  PW<DT>::plan(pl, lane, rowbytes);
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  const uint32_t xreg = (uint32_t)(kh * XB), wreg = (uint32_t)(KS * XB + wave * PW<DT>::kWaveLds);
  /* X DMA: instruction j of wave rw covers tokens 8 (TT rw + j) + lane / 8;
   * lane position q = lane % 8 of the token's LDS row fetches octet
   * q ^ ((token / 2) % 8) */
  const __bf16 *xsrc[TT];
#pragma unroll
  for (int j = 0; j < TT; j++) {
    const int tl = 8 * (TT * rw + j) + (lane >> 3), q = lane & 7;
    const int oct = q ^ ((tl >> 1) & 7);
    /* the unit layout's steps take columns 64 s - 32 (s & 1) + 8 o (+32 for
     * o >= 4): PW<GQ_Q6_KX> */
    xsrc[j] = a.x + (size_t)min(t0 + tl, a.T - 1) * a.K + 8 * oct + (DT == GQ_Q6_KX && oct >= 4 ? 32 : 0);
  }
  auto issue = [&](int st) {
    const uint32_t slot = sbase + (uint32_t)((st % kRing) * SB);
    const int s = s0 + st, xs = DT == GQ_Q6_KX ? s * kBK - 32 * (s & 1) : s * kBK;
#pragma unroll
    for (int j = 0; j < TT; j++)
      dma16(xsrc[j] + xs, __builtin_amdgcn_readfirstlane(slot + xreg + 1024u * (uint32_t)(TT * rw + j)));
    PW<DT>::issue(pl, w, s0 + st, slot + wreg);
  };
  for (int st = 0; st < kRing - 1 && st < ns; st++) issue(st);
#pragma unroll
  for (int i = 0; i < TT; i++) acc[i] = gq_f32x16{};
  const int h = lane >> 5, i32 = lane & 31;
  /* Software pipeline: iteration s runs the MFMAs of step s with B operands
   * dequantized in iteration s - 1 while it dequantizes step s + 1, so the
   * VALU work overlaps the matrix core.  A wave's copies of a step have
   * landed once only the copies of later steps remain in flight; the
   * barrier extends that to every wave's copies and frees the slot read in
   * iteration s - 1 for step s + kRing - 1.  With TT = 2 the A operands of
   * step s + 1 are read during step s too; with TT = 4 (twice the A
   * registers) they are read at the top of their own step. */
  /* A operand addresses within a slot: token tl = 32 i + lane % 32, octet
   * 2 kk + lane / 32, swizzled */
  uint32_t aoff[4][TT];
#pragma unroll
  for (int kk = 0; kk < 4; kk++)
#pragma unroll
    for (int i = 0; i < TT; i++) {
      const int tl = 32 * i + i32, q = (2 * kk + h) ^ ((tl >> 1) & 7);
      aoff[kk][i] = xreg + (uint32_t)((tl * 8 + q) * 16);
    }
  auto wslot = [&](int st) { return smem + (st % kRing) * SB + wreg; };
  gq_bf16x8 b[4], av[4][TT];
  typename PW<DT>::Raw raw;
  wait_groups<NPS, kRing - 2>(ns - 1);
  __syncthreads();
  PW<DT>::read(raw, wslot(0), lane, s0);
  if (TT == 2) {
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
#pragma unroll
      for (int i = 0; i < TT; i++) av[kk][i] = lld<gq_bf16x8>(smem, aoff[kk][i]);
  }
  PW<DT>::dequant(raw, s0, b);
  for (int s = 0; s < ns; s++) {
    if (s + 1 < ns) wait_groups<NPS, kRing - 3>(ns - 2 - s);
    __syncthreads();
    if (s + kRing - 1 < ns) issue(s + kRing - 1);
    const GQ_LDS uint8_t *xc = smem + (s % kRing) * SB;
    if (TT == 4) {
#pragma unroll
      for (int kk = 0; kk < 4; kk++)
#pragma unroll
        for (int i = 0; i < TT; i++) av[kk][i] = lld<gq_bf16x8>(xc, aoff[kk][i]);
    }
    /* LDS reads for step s + 1 first, so their latency hides behind the
     * MFMAs of step s */
    gq_bf16x8 an[4][TT == 2 ? 2 : 1];
    const bool more = s + 1 < ns;
    if (more) {
      PW<DT>::read(raw, wslot(s + 1), lane, s0 + s + 1);
      if (TT == 2) {
        const GQ_LDS uint8_t *xn = smem + ((s + 1) % kRing) * SB;
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
          for (int i = 0; i < 2; i++) an[kk][i] = lld<gq_bf16x8>(xn, aoff[kk][i]);
      }
    }
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
#pragma unroll
      for (int i = 0; i < TT; i++) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[kk][i], b[kk], acc[i], 0, 0, 0);
    if (more) {
      PW<DT>::dequant(raw, s0 + s + 1, b);
      if (TT == 2) {
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
          for (int i = 0; i < 2; i++) av[kk][i] = an[kk][i];
      }
    }
  }
}

__device__ __forceinline__ int tile_token(int i, int e, int lane) {
  return 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}

/* Grid: x = row tiles over the segments (kBN rows each; MV_SWIGLU: 64 gate
 * rows with the same 64 up rows), y = token tiles of 32 TT; 256 KS threads. */
template <int MODE, int KS, int TT>
__global__ __launch_bounds__(kPThreads * KS) void pgemm_kernel(PgArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t pg_smem[];
  GQ_LDS uint8_t *smem = (GQ_LDS uint8_t *)pg_smem;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = wave >> 2, rw = wave & 3;
  const int t0 = blockIdx.y * 32 * TT;
  int sg = 0, tb = blockIdx.x, roff = 0; /* roff: the segment's first row among all segments' */
  if (MODE != MV_SWIGLU)
    while (sg + 1 < a.nseg && tb >= a.seg[sg].rows / kBN) tb -= a.seg[sg].rows / kBN, roff += a.seg[sg].rows, sg++;
  /* this wave's weights: rows r0 .. r0 + 31 of segment ws */
  int ws = sg, r0 = tb * kBN + 32 * rw;
  if (MODE == MV_SWIGLU) ws = rw >> 1, r0 = tb * (kBN / 2) + 32 * (rw & 1);
  const PgSeg &S = a.seg[ws];
  const int dt = a.seg[sg].dtype;
  const uint32_t rowbytes = dt == GQ_Q8_0 ? (uint32_t)(a.K / 32) * 34u : (uint32_t)(a.K / 256) * (dt == GQ_Q4_K ? 144u : 210u);
  const uint8_t *w = S.w + (size_t)r0 * rowbytes;
  gq_f32x16 acc[TT];
  if constexpr (fits<GQ_Q6_K, KS, TT>() && fits<GQ_Q6_KX, KS, TT>()) {
    if (dt == GQ_Q4_K)
      tile_loop<GQ_Q4_K, KS, TT>(a, w, rowbytes, t0, smem, acc);
    else if (dt == GQ_Q6_KX)
      tile_loop<GQ_Q6_KX, KS, TT>(a, w, rowbytes, t0, smem, acc);
    else if (dt == GQ_Q8_0)
      tile_loop<GQ_Q8_0, KS, TT>(a, w, rowbytes, t0, smem, acc);
    else
      tile_loop<GQ_Q6_K, KS, TT>(a, w, rowbytes, t0, smem, acc);
  } else if constexpr (fits<GQ_Q6_KX, KS, TT>()) { /* the launcher sends Q6_K to shapes that fit */
    if (dt == GQ_Q6_KX)
      tile_loop<GQ_Q6_KX, KS, TT>(a, w, rowbytes, t0, smem, acc);
    else if (dt == GQ_Q8_0)
      tile_loop<GQ_Q8_0, KS, TT>(a, w, rowbytes, t0, smem, acc);
    else
      tile_loop<GQ_Q4_K, KS, TT>(a, w, rowbytes, t0, smem, acc);
  } else {
    if (dt == GQ_Q8_0)
      tile_loop<GQ_Q8_0, KS, TT>(a, w, rowbytes, t0, smem, acc);
    else
      tile_loop<GQ_Q4_K, KS, TT>(a, w, rowbytes, t0, smem, acc);
  }
  constexpr int XS = 4 * TT * 16 * 64 * 4; /* bytes of one K-half's tiles */
  GQ_LDS float *xk = (GQ_LDS float *)smem;
  if (KS == 2) { /* add the upper K half (waves 4..7) into waves 0..3, in a fixed order */
    __syncthreads(); /* every wave is done reading the ring */
    if (kh == 1) {
#pragma unroll
      for (int i = 0; i < TT; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) xk[((rw * TT + i) * 16 + e) * 64 + lane] = acc[i][e];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int i = 0; i < TT; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][e] += xk[((rw * TT + i) * 16 + e) * 64 + lane];
    }
  }
  const int n = r0 + (lane & 31);
  if (MODE != MV_SWIGLU) {
    if (kh == 0) {
#pragma unroll
      for (int i = 0; i < TT; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int t = t0 + tile_token(i, e, lane);
          if (t < a.T) {
            float v = acc[i][e];
            if (a.kparts > 1) { /* this K part's sums, added up by pg_parts_kernel or the caller */
              gst<float>(a.part + ((size_t)blockIdx.z * a.T + t) * a.rows_total + roff + n, v);
              continue;
            }
            float *y = S.y + (size_t)t * S.rows + n;
            if (MODE == MV_RESID) v = gld<float>(y) + v;
            gst<float>(y, v);
          }
        }
    }
    return;
  }
  /* SwiGLU: the up waves (rw 2, 3) hand their tiles to the gate waves (rw 0,
   * 1) through LDS; act = (g * sigmoid(g)) * u as silu_inplace then
   * elemwise_mul (kernels_cpu.c:312-389), rounded to bf16 */
  __syncthreads(); /* the ring (and the K-half exchange) are free */
  GQ_LDS float *xch = (GQ_LDS float *)(smem + (KS == 2 ? XS : 0));
  if (kh == 0 && rw >= 2) {
#pragma unroll
    for (int i = 0; i < TT; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) xch[(((rw - 2) * TT + i) * 16 + e) * 64 + lane] = acc[i][e];
  }
  __syncthreads();
  if (kh == 0 && rw < 2) {
#pragma unroll
    for (int i = 0; i < TT; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int t = t0 + tile_token(i, e, lane);
        const float g = acc[i][e], u = xch[((rw * TT + i) * 16 + e) * 64 + lane];
        const float sig = 1.0f / (1.0f + expf(0.0f - g));
        const __bf16 v = (__bf16)((g * sig) * u);
        if (t < a.T) gst<unsigned short>(a.act + (size_t)t * S.rows + n, __builtin_bit_cast(unsigned short, v));
      }
  }
}

/* Q4_K for waves of 64 rows: per step 64 rows x 48 bytes (header + the
 * chunk's 32 quant bytes), three 1-KB DMA instructions, every piece used. */
struct PW4W {
  static constexpr int kRowLds = 48;
  static constexpr int kWaveLds = 3072;
  static constexpr int kDma = 3;
  struct Plan {
    uint32_t off[3];
    bool qs[3];
  };
  __device__ static void plan(Plan &p, int lane, uint32_t rowbytes) {
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const int pc = 64 * i + lane, row = pc / 3, part = pc - 3 * row;
      p.qs[i] = part != 0;
      p.off[i] = (uint32_t)row * rowbytes + 16u * (uint32_t)part;
    }
  }
  __device__ static void issue(const Plan &p, const uint8_t *w, int s, uint32_t lds) {
#pragma unroll
    for (int i = 0; i < 3; i++)
      dma16(w + p.off[i] + (size_t)(s >> 2) * 144 + (p.qs[i] ? 32 * (s & 3) : 0),
            __builtin_amdgcn_readfirstlane(lds + 1024u * i));
  }
  /* row block rb: rows 32 rb + lane % 32 */
  __device__ static void read(PW<GQ_Q4_K>::Raw &w, const GQ_LDS uint8_t *ws, int lane, int rb) {
    const uint32_t r = (uint32_t)(lane & 31) + 32u * (uint32_t)rb, h = (uint32_t)(lane >> 5);
    w.hd = lld<uint4>(ws, r * kRowLds);
    w.q0 = lld<uint2>(ws, r * kRowLds + 16u + 8u * h);
    w.q1 = lld<uint2>(ws, r * kRowLds + 32u + 8u * h);
  }
};

/* The wide tile: each wave owns 64 weight rows (two 32-row blocks) for 32 TT
 * tokens, so every A operand read from LDS feeds two MFMAs, and a step holds
 * twice the matrix work of the 32-row tile: the DMA issued two steps ahead
 * has twice as long to land, and there is one barrier per 32 MFMAs instead
 * of per 16.  X takes a 3-slot ring; the weights need only 2 slots, since a
 * step's bytes are read in the iteration before their own.  At TT = 4 the
 * ring is 3 x 16 + 2 x 12 KB = 72 KB, so two workgroups share a CU (two waves
 * per SIMD, 225 VGPRs).  Fused gate/up + SwiGLU at 512 tokens (Q4_K, 2 x
 * 14336 x 4096): 145 us against 172 us on the 32-row tile (kernel trace),
 * 512-token forward 13.56 -> 12.74 ms.  The STORE / RESID launches (o,
 * down, q/k/v) keep the 32-row tile: there the wide tile needs twice the K
 * parts for the same number of workgroups, and measured slower (q/o 45.8
 * against 39.0 us, forward 14.2 ms). */
template <int TT>
constexpr int wide_ring_bytes() {
  return 3 * x_bytes<TT>() + 2 * 4 * PW4W::kWaveLds;
}

template <int TT>
__device__ __forceinline__ void tile_loop_wide(const PgArgs &a, const uint8_t *w, uint32_t rowbytes, int t0,
                                               GQ_LDS uint8_t *smem, gq_f32x16 (&acc)[2][TT]) {
  constexpr int XB = x_bytes<TT>();
  constexpr int WSB = 4 * PW4W::kWaveLds;
  constexpr int NPS = TT + PW4W::kDma;
  constexpr int kRing = 3;
  static_assert((kRing - 2) * NPS < 64, "vmcnt");
  const int lane = threadIdx.x & 63, rw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ns = a.K / kBK / a.kparts, s0 = (int)blockIdx.z * ns;
  PW4W::Plan pl;
  PW4W::plan(pl, lane, rowbytes);
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  const uint32_t wreg = (uint32_t)(kRing * XB + rw * PW4W::kWaveLds);
  const __bf16 *xsrc[TT];
#pragma unroll
  for (int j = 0; j < TT; j++) {
    const int tl = 8 * (TT * rw + j) + (lane >> 3), q = lane & 7;
    const int oct = q ^ ((tl >> 1) & 7);
    xsrc[j] = a.x + (size_t)min(t0 + tl, a.T - 1) * a.K + 8 * oct;
  }
  auto issue = [&](int st) {
    const uint32_t xslot = sbase + (uint32_t)((st % kRing) * XB);
    const int s = s0 + st;
#pragma unroll
    for (int j = 0; j < TT; j++)
      dma16(xsrc[j] + s * kBK, __builtin_amdgcn_readfirstlane(xslot + 1024u * (uint32_t)(TT * rw + j)));
    PW4W::issue(pl, w, s, sbase + wreg + (uint32_t)((st & 1) * WSB));
  };
  for (int st = 0; st < kRing - 1 && st < ns; st++) issue(st);
#pragma unroll
  for (int r = 0; r < 2; r++)
#pragma unroll
    for (int i = 0; i < TT; i++) acc[r][i] = gq_f32x16{};
  const int h = lane >> 5, i32 = lane & 31;
  uint32_t aoff[4][TT];
#pragma unroll
  for (int kk = 0; kk < 4; kk++)
#pragma unroll
    for (int i = 0; i < TT; i++) {
      const int tl = 32 * i + i32, q = (2 * kk + h) ^ ((tl >> 1) & 7);
      aoff[kk][i] = (uint32_t)((tl * 8 + q) * 16);
    }
  auto wslot = [&](int st) { return smem + wreg + (st & 1) * WSB; };
  gq_bf16x8 b[2][4], av[2][TT];
  PW<GQ_Q4_K>::Raw raw[2];
  wait_groups<NPS, kRing - 2>(ns - 1);
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; r++) PW4W::read(raw[r], wslot(0), lane, r);
#pragma unroll
  for (int r = 0; r < 2; r++) PW<GQ_Q4_K>::dequant(raw[r], s0, b[r]);
  for (int s = 0; s < ns; s++) {
    /* this wave's copies of step s + 1 have landed once only later steps'
     * remain; the barrier extends that to every wave and frees the X slot
     * of step s - 1 and the weight slot of step s (read in iteration s - 1)
     * for step s + 2 */
    if (s + 1 < ns) wait_groups<NPS, kRing - 3>(ns - 2 - s);
    __syncthreads();
    if (s + kRing - 1 < ns) issue(s + kRing - 1);
    const GQ_LDS uint8_t *xc = smem + (s % kRing) * XB;
    /* A operands one k-slice ahead of the MFMAs that use them */
#pragma unroll
    for (int i = 0; i < TT; i++) av[0][i] = lld<gq_bf16x8>(xc, aoff[0][i]);
    const bool more = s + 1 < ns;
    if (more) {
#pragma unroll
      for (int r = 0; r < 2; r++) PW4W::read(raw[r], wslot(s + 1), lane, r);
    }
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      if (kk < 3) {
#pragma unroll
        for (int i = 0; i < TT; i++) av[(kk + 1) & 1][i] = lld<gq_bf16x8>(xc, aoff[kk + 1][i]);
      }
#pragma unroll
      for (int i = 0; i < TT; i++)
#pragma unroll
        for (int r = 0; r < 2; r++)
          acc[r][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[kk & 1][i], b[r][kk], acc[r][i], 0, 0, 0);
    }
    if (more) {
#pragma unroll
      for (int r = 0; r < 2; r++) PW<GQ_Q4_K>::dequant(raw[r], s0 + s + 1, b[r]);
    }
  }
}

/* Fused gate/up + SwiGLU over Q4_K weights on the wide tile.  Grid: x = 128
 * gate rows (with the same 128 up rows), y = token tiles of 32 TT; 256
 * threads.  Waves 0/1 take gate rows 0-63 / 64-127 of the tile, waves 2/3 the
 * same up rows.  Each output is the same sum in the same order as
 * pgemm_kernel's (MFMAs over the steps, k-slices in order), so the two agree
 * bit for bit; the epilogue is pgemm_kernel's. */
template <int TT>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void pgemm_wide_swiglu_kernel(PgArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t pg_smem[];
  GQ_LDS uint8_t *smem = (GQ_LDS uint8_t *)pg_smem;
  const int lane = threadIdx.x & 63, rw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t0 = blockIdx.y * 32 * TT;
  const PgSeg &S = a.seg[rw >> 1];
  const int r0 = blockIdx.x * 128 + 64 * (rw & 1);
  const uint32_t rowbytes = (uint32_t)(a.K / 256) * 144u;
  gq_f32x16 acc[2][TT];
  tile_loop_wide<TT>(a, S.w + (size_t)r0 * rowbytes, rowbytes, t0, smem, acc);
  __syncthreads(); /* the ring is free */
  GQ_LDS float *xch = (GQ_LDS float *)smem;
  if (rw >= 2) {
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
      for (int i = 0; i < TT; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) xch[((((rw - 2) * 2 + r) * TT + i) * 16 + e) * 64 + lane] = acc[r][i][e];
  }
  __syncthreads();
  if (rw < 2) {
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int n = r0 + 32 * r + (lane & 31);
#pragma unroll
      for (int i = 0; i < TT; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int t = t0 + tile_token(i, e, lane);
          const float g = acc[r][i][e], u = xch[(((rw * 2 + r) * TT + i) * 16 + e) * 64 + lane];
          const float sig = 1.0f / (1.0f + expf(0.0f - g));
          const __bf16 v = (__bf16)((g * sig) * u);
          if (t < a.T) gst<unsigned short>(a.act + (size_t)t * S.rows + n, __builtin_bit_cast(unsigned short, v));
        }
    }
  }
}
static_assert(wide_ring_bytes<4>() >= 2 * 2 * 4 * 16 * 64 * 4 && 2 * wide_ring_bytes<4>() <= 160 * 1024,
              "wide ring: the SwiGLU exchange fits, two workgroups per CU");

/* y = (y +) ((part 0 + part 1) + ...) elementwise over T x rows_total
 * (n4 float4s per part), scattered back to the segments' outputs */
__global__ void pg_parts_kernel(PgArgs a, size_t n4, int resid) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const size_t e = 4 * i;
  const int t = (int)(e / (size_t)a.rows_total);
  int r = (int)(e - (size_t)t * a.rows_total);
  const int n0 = a.seg[0].rows, n1 = a.seg[1].rows;
  float *yb = a.seg[0].y;
  int rows = n0;
  if (a.nseg > 1 && r >= n0) {
    r -= n0, yb = a.seg[1].y, rows = n1;
    if (a.nseg > 2 && r >= n1) r -= n1, yb = a.seg[2].y, rows = a.seg[2].rows;
  }
  float *y = yb + (size_t)t * rows + r;
  float4 s = gld<float4>(a.part + e);
  for (int k = 1; k < a.kparts; k++) {
    const float4 u = gld<float4>(a.part + (size_t)k * 4 * n4 + e);
    s.x += u.x, s.y += u.y, s.z += u.z, s.w += u.w;
  }
  if (resid) {
    const float4 q = gld<float4>(y);
    s = make_float4(q.x + s.x, q.y + s.y, q.z + s.z, q.w + s.w);
  }
  gst<float4>(y, s);
}

__global__ void to_bf16_kernel(const float *x, __bf16 *y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (__bf16)x[i];
}

/* Launch shape: token tiles of 128 (TT = 4: each dequantized weight feeds
 * four MFMAs) for launches whose grid still gives every CU a workgroup
 * (gate/up at 512 tokens) and whose weights are Q4_K or Q6_K in the step
 * layout (Q6_K 14336 x 4096 at 512 tokens: 160 -> 95 us).  Other STORE
 * and RESID launches with fewer such tiles than CUs split K over the grid
 * instead (PgArgs.part).  Otherwise tiles of 64, with 2 K-splits inside the
 * workgroup when the grid has at most one workgroup per CU (a second wave
 * per SIMD comes from the split), 1 when it has more. */
int n_cus() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev))
      return 256;
    return n > 0 ? n : 256;
  }();
  return cus;
}

template <int MODE, int KS, int TT>
int launch_shape(const PgArgs &a, int row_tiles, size_t lds, hipStream_t s) {
  static bool attr_done = false;
  if (!attr_done) {
    (void)hipFuncSetAttribute((const void *)pgemm_kernel<MODE, KS, TT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    attr_done = true;
  }
  hipLaunchKernelGGL((pgemm_kernel<MODE, KS, TT>), dim3(row_tiles, (a.T + 32 * TT - 1) / (32 * TT), a.kparts),
                     dim3(kPThreads * KS), lds, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <int MODE>
int launch_mode(const PgArgs &a0, int row_tiles, hipStream_t s) {
  PgArgs a = a0;
  a.kparts = 1;
  if (a.kparts_out) *a.kparts_out = 1;
  /* Q4_K gate/up whose 128-row tiles alone give every CU a workgroup: the
   * wide tile */
  if (MODE == MV_SWIGLU && a.seg[0].dtype == GQ_Q4_K && a.seg[0].rows % 128 == 0 &&
      (a.seg[0].rows / 128) * ((a.T + 127) / 128) >= n_cus()) {
    static bool attr = false;
    if (!attr) {
      (void)hipFuncSetAttribute((const void *)pgemm_wide_swiglu_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                wide_ring_bytes<4>());
      attr = true;
    }
    hipLaunchKernelGGL(pgemm_wide_swiglu_kernel<4>, dim3(a.seg[0].rows / 128, (a.T + 127) / 128, 1), dim3(kPThreads),
                       wide_ring_bytes<4>(), s, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
  }
  bool q4 = false, q6 = false, q6x = false, q8 = false;
  for (int i = 0; i < a.nseg; i++)
    q4 |= a.seg[i].dtype == GQ_Q4_K, q6 |= a.seg[i].dtype == GQ_Q6_K, q6x |= a.seg[i].dtype == GQ_Q6_KX,
        q8 |= a.seg[i].dtype == GQ_Q8_0;
  const int tiles4 = row_tiles * ((a.T + 127) / 128);
  a.rows_total = 0;
  for (int i = 0; i < a.nseg; i++) a.rows_total += a.seg[i].rows;
  /* as few parts as give 1.5 workgroups per CU: 2 for the fused q/k/v
   * launch at 512 tokens (forward 13.83 -> 13.62 ms against 4 parts'
   * 13.95), 4 for o, down and k/v alone */
  const int KP = 2 * tiles4 * 2 >= 3 * n_cus() ? 2 : kKParts;
  if (MODE != MV_SWIGLU && a.part && tiles4 < n_cus() && (a.K / kBK) % KP == 0 &&
      (size_t)KP * a.T * a.rows_total <= a.part_cap) {
    /* too few 128-token tiles to give every CU work: K in KP parts over
     * the grid (four-wave workgroups), then their sum.  At 512 tokens: down
     * 120 -> 91 us (Q4_K) and 145 -> 101 us (Q6_K step layout), k/v
     * 33 -> 25 us, the o projection in the model forward ~4 us faster,
     * whole forward 15.1 -> 13.6 ms.  Q6_K in the reference layout keeps
     * 64-token tiles (its stages are larger); the tile width does not
     * change the order of any sum, so both layouts still agree bit for
     * bit. */
    a.kparts = KP;
    int rc;
    if (q6) {
      rc = launch_shape<MODE, 1, 2>(
          a, row_tiles, std::max({ring_bytes<GQ_Q6_K, 1, 2>(), ring_bytes<GQ_Q4_K, 1, 2>(), ring_bytes<GQ_Q8_0, 1, 2>()}), s);
    } else {
      const size_t lds = std::max({q6x ? ring_bytes<GQ_Q6_KX, 1, 4>() : 0, q8 ? ring_bytes<GQ_Q8_0, 1, 4>() : 0,
                                   ring_bytes<GQ_Q4_K, 1, 4>()});
      rc = launch_shape<MODE, 1, 4>(a, row_tiles, lds, s);
    }
    if (rc) return rc;
    if (a.kparts_out) { /* the caller sums the parts */
      *a.kparts_out = KP;
      return 0;
    }
    const size_t n4 = (size_t)a.T * a.rows_total / 4;
    hipLaunchKernelGGL(pg_parts_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, a, n4,
                       MODE == MV_RESID ? 1 : 0);
    return hipGetLastError() == hipSuccess ? 0 : -4;
  }
  const int tt = !q6 && tiles4 >= n_cus() ? 4 : 2;
  const int wgs = row_tiles * ((a.T + 32 * tt - 1) / (32 * tt));
  int ks = wgs <= n_cus() ? 2 : 1;
  if ((a.K / kBK) % 2) ks = 1;
  if (tt == 4) {
    const size_t lds = ks == 2 ? std::max({q6x ? ring_bytes<GQ_Q6_KX, 2, 4>() : 0, q8 ? ring_bytes<GQ_Q8_0, 2, 4>() : 0,
                                           ring_bytes<GQ_Q4_K, 2, 4>()})
                               : std::max({q6x ? ring_bytes<GQ_Q6_KX, 1, 4>() : 0, q8 ? ring_bytes<GQ_Q8_0, 1, 4>() : 0,
                                           ring_bytes<GQ_Q4_K, 1, 4>()});
    return ks == 2 ? launch_shape<MODE, 2, 4>(a, row_tiles, lds, s) : launch_shape<MODE, 1, 4>(a, row_tiles, lds, s);
  }
  if (ks == 2) {
    const size_t lds = std::max({q6 ? ring_bytes<GQ_Q6_K, 2, 2>() : 0, q6x ? ring_bytes<GQ_Q6_KX, 2, 2>() : 0,
                                 q4 ? ring_bytes<GQ_Q4_K, 2, 2>() : 0, q8 ? ring_bytes<GQ_Q8_0, 2, 2>() : 0});
    return launch_shape<MODE, 2, 2>(a, row_tiles, lds, s);
  }
  const size_t lds = std::max({q6 ? ring_bytes<GQ_Q6_K, 1, 2>() : 0, q6x ? ring_bytes<GQ_Q6_KX, 1, 2>() : 0,
                               q4 ? ring_bytes<GQ_Q4_K, 1, 2>() : 0, q8 ? ring_bytes<GQ_Q8_0, 1, 2>() : 0});
  return launch_shape<MODE, 1, 2>(a, row_tiles, lds, s);
}

} // namespace

int gq_launch_pgemm(int mode, const PgArgs &a, hipStream_t s) {
  if (a.T <= 0 || a.K <= 0 || a.K % 256 || a.nseg < 1 || a.nseg > 3 || !a.x) return -1;
  int tiles = 0;
  for (int i = 0; i < a.nseg; i++) {
    const PgSeg &g = a.seg[i];
    if (!g.w || g.rows <= 0) return -1;
    if (g.dtype != GQ_Q4_K && g.dtype != GQ_Q6_K && g.dtype != GQ_Q6_KX && g.dtype != GQ_Q8_0) return -1;
    if ((g.dtype == GQ_Q6_K && a.K % 512) || (g.dtype == GQ_Q6_KX && a.K % 2048)) return -2; /* Q6_KX: 16-byte rows */
    if (mode == MV_SWIGLU) {
      if (g.rows % (kBN / 2) || g.dtype != a.seg[0].dtype || g.rows != a.seg[0].rows) return -1;
    } else {
      if (g.rows % kBN || !g.y) return -1;
      tiles += g.rows / kBN;
    }
  }
  /* the K-half exchange (4 TT tiles) and the SwiGLU exchange (2 TT tiles)
   * reuse the ring, which is larger */
  static_assert(ring_bytes<GQ_Q4_K, 1, 2>() >= 2 * 2 * 16 * 64 * 4 && ring_bytes<GQ_Q6_K, 1, 2>() >= 2 * 2 * 16 * 64 * 4 &&
                    ring_bytes<GQ_Q4_K, 1, 4>() >= 2 * 4 * 16 * 64 * 4 && ring_bytes<GQ_Q8_0, 1, 2>() >= 2 * 2 * 16 * 64 * 4,
                "exchange fits the ring");
  static_assert(ring_bytes<GQ_Q4_K, 2, 2>() >= 6 * 2 * 16 * 64 * 4 && ring_bytes<GQ_Q6_K, 2, 2>() >= 6 * 2 * 16 * 64 * 4 &&
                    ring_bytes<GQ_Q4_K, 2, 4>() >= 6 * 4 * 16 * 64 * 4 && ring_bytes<GQ_Q8_0, 2, 2>() >= 6 * 2 * 16 * 64 * 4,
                "exchanges fit the ring");
  if (mode == MV_SWIGLU) {
    if (a.nseg != 2 || !a.act) return -1;
    return launch_mode<MV_SWIGLU>(a, a.seg[0].rows / (kBN / 2), s);
  }
  if (mode == MV_RESID) return launch_mode<MV_RESID>(a, tiles, s);
  if (mode == MV_STORE) return launch_mode<MV_STORE>(a, tiles, s);
  return -1;
}

int gq_launch_to_bf16(const float *x, __bf16 *y, size_t n, hipStream_t s) {
  if (!n) return 0;
  hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
