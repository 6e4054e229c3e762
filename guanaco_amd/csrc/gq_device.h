/*
 * gq_device.h — gfx950 device helpers shared by the decode kernels.
 *
 * Wave64 reductions use DPP row operations (a 16-lane row reduces with
 * row_ror:8, row_ror:4 and two quad permutes, all folded into the VALU add)
 * and two cross-row exchanges.  Block loads are 16-byte vector loads where
 * the K-quant layout is 16-byte aligned (Q4_K) and dword loads funnel-shifted
 * with v_alignbyte where it is only 2-byte aligned (Q6_K: 210-byte blocks,
 * Q8_0: 34-byte blocks).
 */
#ifndef GQ_DEVICE_H
#define GQ_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#define GQ_WAVE 64

typedef uint32_t gq_u32x3 __attribute__((ext_vector_type(3), aligned(4)));

/* Global-address-space accesses.  Pointers read out of kernel-argument
 * structs lose their address space and would otherwise compile to FLAT
 * instructions, which count against the LDS wait counter as well: every
 * s_waitcnt for an LDS read would then also wait for the in-flight HBM loads
 * and serialise the prefetching. */
#define GQ_GLOBAL __attribute__((address_space(1)))

/* Native clang vector of the same size as T (HIP's float4 / uint4 are
 * classes whose constructors cannot bind address-space-qualified
 * references). */
template <int N>
struct gq_native;
template <>
struct gq_native<2> {
  typedef unsigned short type;
};
template <>
struct gq_native<4> {
  typedef unsigned int type;
};
template <>
struct gq_native<8> {
  typedef unsigned int type __attribute__((ext_vector_type(2)));
};
template <>
struct gq_native<16> {
  typedef unsigned int type __attribute__((ext_vector_type(4)));
};

template <class T>
__device__ __forceinline__ T gld(const void *p) {
  typedef typename gq_native<sizeof(T)>::type N;
  return __builtin_bit_cast(T, *(const GQ_GLOBAL N *)p);
}

/* Non-temporal load (the `nt` cache policy): for streams read once per
 * launch, such as the K/V cache, so that they do not evict lines that other
 * waves still reuse. */
template <class T>
__device__ __forceinline__ T gld_nt(const void *p) {
  typedef typename gq_native<sizeof(T)>::type N;
  return __builtin_bit_cast(T, __builtin_nontemporal_load((const GQ_GLOBAL N *)p));
}

/* 12-byte load (three dwords, 4-byte aligned) */
__device__ __forceinline__ uint3 gld12(const void *p) {
  typedef unsigned int N __attribute__((ext_vector_type(3), aligned(4)));
  const N v = *(const GQ_GLOBAL N *)p;
  return make_uint3(v.x, v.y, v.z);
}

template <class T>
__device__ __forceinline__ void gst(void *p, T v) {
  typedef typename gq_native<sizeof(T)>::type N;
  *(GQ_GLOBAL N *)p = __builtin_bit_cast(N, v);
}

/* LDS accesses through explicit local-address-space pointers (byte offsets
 * into the workgroup's LDS allocation). */
#define GQ_LDS __attribute__((address_space(3)))

template <class T>
__device__ __forceinline__ T lld(const GQ_LDS uint8_t *base, uint32_t off) {
  typedef typename gq_native<sizeof(T)>::type N;
  return __builtin_bit_cast(T, *(const GQ_LDS N *)(base + off));
}

template <class T>
__device__ __forceinline__ void lst(GQ_LDS uint8_t *base, uint32_t off, T v) {
  typedef typename gq_native<sizeof(T)>::type N;
  *(GQ_LDS N *)(base + off) = __builtin_bit_cast(N, v);
}

/* Eight bytes at a 2-byte-aligned LDS offset: three aligned dword reads and
 * two funnel shifts (reads up to 4 bytes past the field). */
__device__ __forceinline__ uint2 lld8_a2(const GQ_LDS uint8_t *base, uint32_t off) {
  const uint32_t a = off & ~3u, sh = off & 3u;
  const uint32_t w0 = lld<uint32_t>(base, a), w1 = lld<uint32_t>(base, a + 4),
                 w2 = lld<uint32_t>(base, a + 8);
  uint2 r;
  r.x = __builtin_amdgcn_alignbyte(w1, w0, sh);
  r.y = __builtin_amdgcn_alignbyte(w2, w1, sh);
  return r;
}

__device__ __forceinline__ float gq_h2f(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h16 & 0xffffu));
}

/* DPP move helpers: compile-time control words (gfx9 encoding). */
template <int CTRL>
__device__ __forceinline__ float gq_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                0xf, 0xf, false));
}

/* Sum over each 16-lane row; every lane of the row receives the row sum. */
__device__ __forceinline__ float gq_row16_sum(float v) {
  v += gq_dpp<0x128>(v); /* row_ror:8 */
  v += gq_dpp<0x124>(v); /* row_ror:4 */
  v += gq_dpp<0x4e>(v);  /* quad_perm [2,3,0,1] */
  v += gq_dpp<0xb1>(v);  /* quad_perm [1,0,3,2] */
  return v;
}

/* Sum over groups of 8 lanes (lanes 8k..8k+7); every lane receives it. */
__device__ __forceinline__ float gq_row8_sum(float v) {
  v += gq_dpp<0x141>(v); /* row_half_mirror: lane i <-> 7-i within 8 */
  v += gq_dpp<0x4e>(v);
  v += gq_dpp<0xb1>(v);
  return v;
}

/* Full wave64 sum; every lane receives it. */
__device__ __forceinline__ float gq_wave_sum(float v) {
  v = gq_row16_sum(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

/* Full wave64 sum with DPP only (no LDS round trip): row sums, then
 * row_bcast:15 and row_bcast:31 fold rows 0-1 and 2-3 into lane 63, which is
 * returned to every lane (a scalar). */
__device__ __forceinline__ float gq_wave_total(float v) {
  v = gq_row16_sum(v);
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

/* Load of a wave-uniform value through the scalar data cache (counts against
 * lgkmcnt, not vmcnt).  Only for data written before the kernel started. */
template <class T>
__device__ __forceinline__ T gq_sld(const void *p) {
  typedef typename gq_native<sizeof(T)>::type N;
  return __builtin_bit_cast(T, *(const __attribute__((address_space(4))) N *)p);
}

__device__ __forceinline__ float gq_wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

/* Two dwords starting at a 2-byte-aligned address: one 12-byte dword-aligned
 * load and two v_alignbyte funnel shifts.  Reads at most 4 bytes past the
 * 8 requested (callers keep that inside the block). */
__device__ __forceinline__ uint2 gq_load8_a2(const uint8_t *p) {
  const uintptr_t a = (uintptr_t)p;
  const uint3 w = gld12((const void *)(a & ~(uintptr_t)3));
  const uint32_t sh = (uint32_t)(a & 3u);
  uint2 r;
  r.x = __builtin_amdgcn_alignbyte(w.y, w.x, sh);
  r.y = __builtin_amdgcn_alignbyte(w.z, w.y, sh);
  return r;
}

__device__ __forceinline__ uint32_t gq_byte(uint32_t w, int k) { return (w >> (8 * k)) & 0xffu; }

typedef float gq_f32x2 __attribute__((ext_vector_type(2)));

/* Two 4-bit integers held in bytes 0,1 (HI = false) or 2,3 (HI = true) of w
 * (each byte 0..15) to float, times 2^-9, in one v_cvt_pk_f32_fp8.  A byte
 * 0..15 read as OCP FP8 E4M3 (bias 7) is exactly v * 2^-9: 0..7 are the
 * subnormals m * 2^-3 * 2^-6, 8..15 the first normal binade
 * (1 + m/8) * 2^-6 = (8 + m) * 2^-9. */
template <bool HI>
__device__ __forceinline__ gq_f32x2 gq_nib2f(uint32_t w) {
  return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, HI);
}

/* Direct global -> LDS copies (no VGPRs): 16 or 4 bytes per lane, lane i at
 * lds_addr + 16 i (or 4 i).  They are issued from inline assembly on purpose:
 * the compiler's wait-count pass treats a visible LDS-DMA load as a write to
 * every LDS location and would put s_waitcnt vmcnt(0) in front of each LDS
 * read of a pipelined loop, draining the stages in flight.  Completion is
 * tracked by hand (wait_vmcnt + barrier).  VMEM loads retire in order, so the
 * compiler's own waits for other loads can only wait longer than needed,
 * never less.  The LDS address goes in M0 (the "{m0}" operand: the compiler
 * writes M0). */
__device__ __forceinline__ void dma16(const void *src, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(lds_addr));
}

__device__ __forceinline__ void dma4(const void *src, uint32_t lds_addr) {
  asm volatile("global_load_lds_dword %0, off" : : "v"(src), "{m0}"(lds_addr));
}

/* s_waitcnt vmcnt(n) with the other counters left alone (vmcnt(0) for n > 63). */
__device__ __forceinline__ void wait_vmcnt(int n) {
#define GQ_W(N)                                                                                   \
  case N: __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | (7 << 4) | (15 << 8)); break;
  switch (n) {
    GQ_W(0) GQ_W(1) GQ_W(2) GQ_W(3) GQ_W(4) GQ_W(5) GQ_W(6) GQ_W(7) GQ_W(8) GQ_W(9) GQ_W(10)
    GQ_W(11) GQ_W(12) GQ_W(13) GQ_W(14) GQ_W(15) GQ_W(16) GQ_W(17) GQ_W(18) GQ_W(19) GQ_W(20)
    GQ_W(21) GQ_W(22) GQ_W(23) GQ_W(24) GQ_W(25) GQ_W(26) GQ_W(27) GQ_W(28) GQ_W(29) GQ_W(30)
    GQ_W(31) GQ_W(32) GQ_W(33) GQ_W(34) GQ_W(35) GQ_W(36) GQ_W(37) GQ_W(38) GQ_W(39) GQ_W(40)
    GQ_W(41) GQ_W(42) GQ_W(43) GQ_W(44) GQ_W(45) GQ_W(46) GQ_W(47) GQ_W(48) GQ_W(49) GQ_W(50)
    GQ_W(51) GQ_W(52) GQ_W(53) GQ_W(54) GQ_W(55) GQ_W(56) GQ_W(57) GQ_W(58) GQ_W(59) GQ_W(60)
    GQ_W(61) GQ_W(62) GQ_W(63)
  default: __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); break; /* vmcnt(0) */
  }
#undef GQ_W
}

/* s_waitcnt vmcnt(N) for a compile-time N */
template <int N>
__device__ __forceinline__ void wait_vmcnt_c() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

/* vmcnt(min(ahead, A) * NPS): ahead groups of NPS loads may stay in flight */
template <int NPS, int A>
__device__ __forceinline__ void wait_groups(int ahead) {
  if constexpr (A == 0) {
    wait_vmcnt_c<0>();
  } else {
    if (ahead >= A)
      wait_vmcnt_c<A * NPS>();
    else
      wait_groups<NPS, A - 1>(ahead);
  }
}

#endif
