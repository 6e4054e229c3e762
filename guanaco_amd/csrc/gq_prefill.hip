/*
 * gq_prefill.hip — the prefill chunk (many tokens at once) on gfx950: a
 * K-quant x activations GEMM on the bf16 matrix cores, with fp32
 * accumulation.
 *
 * The reference computes a prefill projection as T sequential matvecs
 * (linear_dispatch, engine.c:119-152).  Here Y[T][N] = X[T][K] . W^T for
 * all T tokens in one launch, where W is N rows of Q4_K blocks
 * (quant_matvec_q4_k.c:9-16) or Q6_K blocks (quant_matvec_q6_k.c), X fp32
 * row-major.
 *
 * Workgroup tile: 64 tokens x 128 weight rows, 4 waves in a 2 x 2 grid, each
 * wave 32 tokens x 64 rows = two 32x32 tiles of v_mfma_f32_32x32x16_bf16.
 * K advances 64 weights per step: one 32-byte quant chunk per row, i.e. two
 * Q4_K sub-blocks, or two 32-weight groups of a Q6_K half-block.  Per step
 * the workgroup converts its X tile to bf16 (round to nearest even) and
 * dequantizes its W tile into LDS (Q4_K: w = d sc q - dmin m in fp32, Q6_K:
 * w = (d sc) q, exact in fp32; then bf16); the next step's global loads are
 * in flight while the current step's MFMAs run (double-buffered LDS).
 *
 * MFMA operand layout (32x32x16, checked on the device): A[i][k] is element
 * k % 8 of lane i + 32 (k / 8); B[k][j] element k % 8 of lane j + 32 (k / 8);
 * D[i][j] element 4 (i / 8) + i % 4 of lane j + 32 ((i / 4) % 2).
 */
#include "gq_device.h"
#include "gq_internal.h"

namespace {

typedef __bf16 gq_bf16x8 __attribute__((ext_vector_type(8)));
typedef float gq_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPThreads = 256;
constexpr int kBM = 64, kBN = 128, kBK = 64;
constexpr int kLdK = kBK + 8; /* bf16 per LDS row: +8 staggers the banks */

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const __bf16 a = (__bf16)lo, b = (__bf16)hi; /* round to nearest even */
  return (uint32_t)__builtin_bit_cast(unsigned short, a) | ((uint32_t)__builtin_bit_cast(unsigned short, b) << 16);
}

/* 16 bytes from a 2-byte-aligned address: five dword loads funnel-shifted
 * (the 4 bytes past the 16 stay inside the Q6_K block for every use here) */
__device__ __forceinline__ uint4 gld16_a2(const uint8_t *p) {
  typedef unsigned int N4 __attribute__((ext_vector_type(4), aligned(4)));
  const uintptr_t a = (uintptr_t)p, b = a & ~(uintptr_t)3;
  const N4 w = *(const GQ_GLOBAL N4 *)b;
  const uint32_t e = *(const GQ_GLOBAL unsigned int *)(b + 16);
  const uint32_t sh = (uint32_t)(a & 3u);
  return make_uint4(__builtin_amdgcn_alignbyte(w.y, w.x, sh), __builtin_amdgcn_alignbyte(w.z, w.y, sh),
                    __builtin_amdgcn_alignbyte(w.w, w.z, sh), __builtin_amdgcn_alignbyte(e, w.w, sh));
}

__device__ __forceinline__ uint32_t gld_u8(const uint8_t *p) { return *(const GQ_GLOBAL uint8_t *)p; }

/* Per-thread W slice of one step: row tid / 2 of the tile, 16 weights of
 * each of the step's two 32-weight groups (half hf = tid & 1).  dequant()
 * returns them as bf16 pairs: lo[] for k = 16 hf + i, hq[] for
 * k = 32 + 16 hf + i. */
template <int DT>
struct PW;

template <>
struct PW<GQ_Q4_K> {
  static constexpr int BB = 144;
  struct Raw {
    uint4 q, h;
  };
  /* chunk cc = s % 4 of super-block s / 4: qs bytes 32 cc + 16 hf .. + 15 */
  __device__ static void load(Raw &r, const uint8_t *blk, int cc, int hf) {
    r.h = gld<uint4>(blk);
    r.q = gld<uint4>(blk + 16 + 32 * cc + 16 * hf);
  }
  /* sub-blocks 2cc (low nibbles) and 2cc+1 (high nibbles); scale/min decode
   * as in the matvec (quant_matvec_q4_k.c:47-56) */
  __device__ static void dequant(const Raw &st, int cc, uint32_t lo[8], uint32_t hq[8]) {
    const float d = gq_h2f(st.h.x), dm = gq_h2f(st.h.x >> 16);
    const uint32_t sh = 16u * (uint32_t)(cc & 1);
    const bool hi = cc >= 2;
    const uint32_t y = st.h.y >> sh, z = st.h.z >> sh, w = st.h.w >> sh;
    const uint32_t mlo = hi ? 0x0f0fu : 0x3f3fu, mhi = hi ? 0x3030u : 0u;
    const uint32_t S = ((hi ? w : y) & mlo) | ((y >> 2) & mhi);
    const uint32_t M = ((hi ? (w >> 4) : z) & mlo) | ((z >> 2) & mhi);
    const float a0 = d * (float)(S & 0xffu), m0 = dm * (float)(M & 0xffu);
    const float a1 = d * (float)((S >> 8) & 0xffu), m1 = dm * (float)((M >> 8) & 0xffu);
    const uint32_t qw[4] = {st.q.x, st.q.y, st.q.z, st.q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        v[j] = __builtin_fmaf(a0, (float)((qw[k] >> (8 * j)) & 15u), -m0);
        v[4 + j] = __builtin_fmaf(a1, (float)((qw[k] >> (8 * j + 4)) & 15u), -m1);
      }
      lo[2 * k] = pack_bf16x2(v[0], v[1]), lo[2 * k + 1] = pack_bf16x2(v[2], v[3]);
      hq[2 * k] = pack_bf16x2(v[4], v[5]), hq[2 * k + 1] = pack_bf16x2(v[6], v[7]);
    }
  }
};

/* Q6_K block (quant_matvec_q6_k.c): ql[128], qh[64], int8 scales[16], fp16
 * d.  Weight 128 n + 32 g + l (half n, group g < 4, l < 32) has
 * q = (ql[64 n + 32 (g & 1) + l] >> 4 (g >> 1)) & 15
 *     | ((qh[32 n + l] >> 2 g) & 3) << 4,  minus 32,
 * scale scales[8 n + 2 g + l / 16].  Step chunk cc = 2 n + par holds groups
 * 2 par and 2 par + 1 of half n. */
template <>
struct PW<GQ_Q6_K> {
  static constexpr int BB = 210;
  struct Raw {
    uint4 a, b, h;
    uint32_t sd; /* scale of group 2par | scale of group 2par+1 << 8 | d << 16 */
  };
  __device__ static void load(Raw &r, const uint8_t *blk, int cc, int hf) {
    const int n = cc >> 1, par = cc & 1;
    r.a = gld16_a2(blk + 64 * n + 16 * hf);
    r.b = gld16_a2(blk + 64 * n + 32 + 16 * hf);
    r.h = gld16_a2(blk + 128 + 32 * n + 16 * hf);
    const uint8_t *sc = blk + 192 + 8 * n + 4 * par + hf;
    r.sd = gld_u8(sc) | (gld_u8(sc + 2) << 8) | ((uint32_t)gld<uint16_t>(blk + 208) << 16);
  }
  __device__ static void dequant(const Raw &st, int cc, uint32_t lo[8], uint32_t hq[8]) {
    const uint32_t sa = 4u * (uint32_t)(cc & 1);
    const float d = gq_h2f(st.sd >> 16);
    const float a0 = d * (float)(int8_t)(st.sd & 0xffu), a1 = d * (float)(int8_t)((st.sd >> 8) & 0xffu);
    const uint32_t A[4] = {st.a.x, st.a.y, st.a.z, st.a.w}, B[4] = {st.b.x, st.b.y, st.b.z, st.b.w};
    const uint32_t H[4] = {st.h.x, st.h.y, st.h.z, st.h.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t u0 = ((A[k] >> sa) & 0x0f0f0f0fu) | (((H[k] >> sa) & 0x03030303u) << 4);
      const uint32_t u1 = ((B[k] >> sa) & 0x0f0f0f0fu) | (((H[k] >> (sa + 2)) & 0x03030303u) << 4);
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        v[j] = a0 * (float)((int)((u0 >> (8 * j)) & 63u) - 32);
        v[4 + j] = a1 * (float)((int)((u1 >> (8 * j)) & 63u) - 32);
      }
      lo[2 * k] = pack_bf16x2(v[0], v[1]), lo[2 * k + 1] = pack_bf16x2(v[2], v[3]);
      hq[2 * k] = pack_bf16x2(v[4], v[5]), hq[2 * k + 1] = pack_bf16x2(v[6], v[7]);
    }
  }
};

/* Per-step register staging: X (4 float4 per thread) and the W slice. */
template <int DT>
struct Stage {
  float4 x[4];
  typename PW<DT>::Raw w;
};

template <int DT>
__device__ __forceinline__ void load_stage(Stage<DT> &st, const float *X, int T, int K, const uint8_t *W,
                                           int t0, int n0, int s) {
  const int tid = threadIdx.x;
  /* X tile: 64 tokens x 64 fp32 = 1024 float4, 4 per thread */
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int f = tid + i * kPThreads, t = f >> 4, c = f & 15;
    const int tt = min(t0 + t, T - 1);
    st.x[i] = gld<float4>(X + (size_t)tt * K + s * kBK + 4 * c);
  }
  const int r = tid >> 1, hf = tid & 1;
  const size_t rowbytes = (size_t)(K / 256) * PW<DT>::BB;
  PW<DT>::load(st.w, W + (size_t)(n0 + r) * rowbytes + (size_t)(s >> 2) * PW<DT>::BB, s & 3, hf);
}

template <int DT>
__device__ __forceinline__ void store_stage(const Stage<DT> &st, GQ_LDS uint8_t *As, GQ_LDS uint8_t *Bs, int s) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int f = tid + i * kPThreads, t = f >> 4, c = f & 15;
    uint2 v;
    v.x = pack_bf16x2(st.x[i].x, st.x[i].y);
    v.y = pack_bf16x2(st.x[i].z, st.x[i].w);
    lst<uint2>(As, (uint32_t)(t * kLdK + 4 * c) * 2u, v);
  }
  const int r = tid >> 1, hf = tid & 1;
  uint32_t lo[8], hq[8];
  PW<DT>::dequant(st.w, s & 3, lo, hq);
  /* weights 16 hf + i of the first group land at k 16 hf + i, those of the
   * second at k 32 + 16 hf + i */
  const uint32_t base = (uint32_t)(r * kLdK) * 2u;
  lst<uint4>(Bs, base + (uint32_t)(16 * hf) * 2u, make_uint4(lo[0], lo[1], lo[2], lo[3]));
  lst<uint4>(Bs, base + (uint32_t)(16 * hf + 8) * 2u, make_uint4(lo[4], lo[5], lo[6], lo[7]));
  lst<uint4>(Bs, base + (uint32_t)(32 + 16 * hf) * 2u, make_uint4(hq[0], hq[1], hq[2], hq[3]));
  lst<uint4>(Bs, base + (uint32_t)(32 + 16 * hf + 8) * 2u, make_uint4(hq[4], hq[5], hq[6], hq[7]));
}

template <int DT, int MODE>
__global__ __launch_bounds__(kPThreads) void prefill_gemm_kernel(const float *X, const uint8_t *W, float *Y,
                                                                const float *R, int T, int N, int K) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][(kBM + kBN) * kLdK * 2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * kBN, t0 = blockIdx.y * kBM;
  const int nsteps = K / kBK;
  gq_f32x16 acc[2] = {};
  Stage<DT> st;
  load_stage<DT>(st, X, T, K, W, t0, n0, 0);
  for (int s = 0; s < nsteps; s++) {
    GQ_LDS uint8_t *As = (GQ_LDS uint8_t *)smem[s & 1];
    GQ_LDS uint8_t *Bs = As + kBM * kLdK * 2;
    store_stage<DT>(st, As, Bs, s);
    __syncthreads();
    if (s + 1 < nsteps) load_stage<DT>(st, X, T, K, W, t0, n0, s + 1);
#pragma unroll
    for (int kk = 0; kk < kBK / 16; kk++) {
      const uint32_t ko = (uint32_t)(16 * kk + 8 * (lane >> 5));
      const gq_bf16x8 a = lld<gq_bf16x8>(As, ((uint32_t)(32 * wm + (lane & 31)) * kLdK + ko) * 2u);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const gq_bf16x8 b = lld<gq_bf16x8>(Bs, ((uint32_t)(64 * wn + 32 * j + (lane & 31)) * kLdK + ko) * 2u);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
      }
    }
    /* the other buffer is written next step; this one only after a barrier */
  }
  /* D[i][j]: token t0 + 32 wm + i, row n0 + 64 wn + 32 jt + j */
#pragma unroll
  for (int jt = 0; jt < 2; jt++)
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int i = (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
      const int t = t0 + 32 * wm + i, n = n0 + 64 * wn + 32 * jt + (lane & 31);
      if (t < T) {
        float v = acc[jt][e];
        if (MODE == MV_RESID) v = gld<float>(R + (size_t)t * N + n) + v;
        gst<float>(Y + (size_t)t * N + n, v);
      }
    }
}

} // namespace

namespace {
template <int DT>
int launch_dt(int mode, const float *X, const void *W, float *Y, const float *R, int T, int N, int K,
              hipStream_t s) {
  const dim3 grid(N / kBN, (T + kBM - 1) / kBM), block(kPThreads);
  if (mode == MV_RESID)
    hipLaunchKernelGGL((prefill_gemm_kernel<DT, MV_RESID>), grid, block, 0, s, X, (const uint8_t *)W, Y, R, T, N,
                       K);
  else if (mode == MV_STORE)
    hipLaunchKernelGGL((prefill_gemm_kernel<DT, MV_STORE>), grid, block, 0, s, X, (const uint8_t *)W, Y, R, T, N,
                       K);
  else
    return -1;
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
} // namespace

int gq_launch_prefill_gemm(int dtype, int mode, const float *X, const void *W, float *Y, const float *R, int T,
                           int N, int K, hipStream_t s) {
  if (T <= 0 || N <= 0 || K <= 0 || N % kBN || K % 256 || (mode == MV_RESID && !R)) return -1;
  if (dtype == GQ_Q4_K) return launch_dt<GQ_Q4_K>(mode, X, W, Y, R, T, N, K, s);
  if (dtype == GQ_Q6_K) return launch_dt<GQ_Q6_K>(mode, X, W, Y, R, T, N, K, s);
  return -1;
}
