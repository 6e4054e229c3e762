/*
 * gq_synth.h — deterministic, libm-free synthetic input generator.
 *
 * One definition of every synthetic byte the benchmarks and parity tests use:
 * Q4_K / Q6_K / Q8_0 super-blocks, fp32 activations and the KV pre-fill.
 * The same inline functions are compiled by gcc (host oracle, fixture
 * harness) and by hipcc (device fill kernels in libgq_hip.so), so the GPU box
 * regenerates bit-identical inputs from a seed without shipping the 4.6 GB of
 * weights or the multi-GiB KV pre-fill.
 *
 * Every value is a pure function of (seed, index): a SplitMix64 finaliser
 * over a Weyl sequence.  Only integer arithmetic and exactly representable
 * float operations are used, so no libm and no rounding-mode dependence:
 *   - uniform bytes:      bytes of the hash word;
 *   - "N(0,1)" fp32:      Irwin–Hall sum of twelve 16-bit uniforms, centred
 *                         and scaled by 2^-16 (exact in fp32; support [-6,6],
 *                         unit variance);
 *   - U(0.001, 0.05) fp16: 24-bit uniform -> fp32 affine map with separate
 *                         (non-fused) multiply and add, then round-to-nearest-
 *                         even to binary16 in integer code.
 *
 * Block layouts follow the K-quant formats read by the reference
 * (quant_matvec_q4_k.c:9-16, quant_matvec_q6_k.c:5-12, quant_matvec_q8_0.c:5-10).
 */
#ifndef GQ_SYNTH_H
#define GQ_SYNTH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define GQ_HD __host__ __device__ __forceinline__
#else
#define GQ_HD static inline
#endif

#define GQ_Q4K_BLOCK_BYTES 144
#define GQ_Q6K_BLOCK_BYTES 210
#define GQ_Q8_0_BLOCK_BYTES 34

GQ_HD uint64_t gq_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

/* Word `idx` of the stream named by `seed`. */
GQ_HD uint64_t gq_hash(uint64_t seed, uint64_t idx) {
  return gq_mix64(seed + (idx + 1ULL) * 0x9e3779b97f4a7c15ULL);
}

/* Seed of a sub-stream (a tensor, a field of a block). */
GQ_HD uint64_t gq_subseed(uint64_t seed, uint64_t tag) {
  return gq_mix64(seed ^ gq_mix64(tag + 0x632be59bd9b4e019ULL));
}

GQ_HD float gq_bits_f32(uint32_t u) {
  union { uint32_t u; float f; } v;
  v.u = u;
  return v.f;
}

GQ_HD uint32_t gq_f32_bits(float f) {
  union { uint32_t u; float f; } v;
  v.f = f;
  return v.u;
}

/* fp32 -> IEEE binary16, round to nearest even, with subnormals, inf, NaN. */
GQ_HD uint16_t gq_f32_to_f16(float f) {
  uint32_t x = gq_f32_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf or NaN */
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  }
  if (ax >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
    return (uint16_t)(sign | 0x7c00u);
  }
  if (ax < 0x38800000u) { /* below the smallest normal half: subnormal or 0 */
    if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* 14..24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (ax >> 23) - 112u; /* rebias 127 -> 15 */
  uint32_t m = ax & 0x7fffffu;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

/* IEEE binary16 -> fp32, exact (subnormals, inf and NaN included). */
GQ_HD float gq_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1fu) return gq_bits_f32(sign | 0x7f800000u | (m << 13));
  if (e == 0u) { /* zero or subnormal: m * 2^-24, normalised by hand */
    if (m == 0u) return gq_bits_f32(sign);
    uint32_t ex = 113u; /* exponent field of 2^-14 */
    while (!(m & 0x400u)) m <<= 1, ex--;
    return gq_bits_f32(sign | (ex << 23) | ((m & 0x3ffu) << 13));
  }
  return gq_bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* 24-bit uniform in [0,1) from a hash word. */
GQ_HD float gq_u01(uint64_t h) {
  return (float)(uint32_t)(h >> 40) * 5.9604644775390625e-08f; /* 2^-24, exact */
}

/* fp16 bits of U(0.001, 0.05), the d / dmin distribution of every config. */
GQ_HD uint16_t gq_scale_f16(uint64_t h) {
#if defined(__clang__)
#pragma clang fp contract(off) /* multiply and add stay separate roundings */
#endif
  float p = 0.049f * gq_u01(h);
  float v = 0.001f + p;
  return gq_f32_to_f16(v);
}

/* Approximately N(0,1) fp32: Irwin–Hall(12) of 16-bit uniforms, exact. */
GQ_HD float gq_normal(uint64_t seed, uint64_t idx) {
  uint64_t h0 = gq_hash(seed, 3ULL * idx + 0ULL);
  uint64_t h1 = gq_hash(seed, 3ULL * idx + 1ULL);
  uint64_t h2 = gq_hash(seed, 3ULL * idx + 2ULL);
  int32_t s = 0;
  for (int k = 0; k < 4; k++) {
    s += (int32_t)((h0 >> (16 * k)) & 0xffffu);
    s += (int32_t)((h1 >> (16 * k)) & 0xffffu);
    s += (int32_t)((h2 >> (16 * k)) & 0xffffu);
  }
  return (float)(s - 393210) * 1.52587890625e-05f; /* 2^-16, exact */
}

/*
 * Seed of one tensor of a synthetic model.  layer = -1 for global tensors.
 * Slots: 0 wq, 1 wk, 2 wv, 3 wo, 4 w_gate, 5 w_up, 6 w_down, 7 rms_att,
 * 8 rms_ffn, 10 token_embd, 11 output, 12 output_norm, 13 K pre-fill,
 * 14 V pre-fill, 15 activations.
 */
GQ_HD uint64_t gq_tensor_seed(uint64_t model_seed, int layer, int slot) {
  return gq_subseed(model_seed, ((uint64_t)(int64_t)(layer + 1) << 8) | (uint64_t)(uint32_t)slot);
}

/* RMSNorm weight: 1 + z/64 with z ~ gq_normal (every step exact in fp32). */
GQ_HD float gq_norm_weight(uint64_t seed, uint64_t i) {
  return 1.0f + gq_normal(seed, i) * 0.015625f;
}

/*
 * Index of KV pre-fill element (layer, kv_head, pos, dim) in its gq_normal
 * stream; independent of max_seq so any cache size sees the same history.
 */
GQ_HD uint64_t gq_kv_index(int layer, int n_kv_heads, int kv_head, int pos, int head_dim, int d) {
  return (((uint64_t)layer * (uint64_t)n_kv_heads + (uint64_t)kv_head) << 32) |
         ((uint64_t)pos * (uint64_t)head_dim + (uint64_t)d);
}

/* Uniform byte `i` of stream `seed`. */
GQ_HD uint8_t gq_byte(uint64_t seed, uint64_t i) {
  return (uint8_t)(gq_hash(seed, i >> 3) >> (8u * (uint32_t)(i & 7u)));
}

/*
 * Byte `o` (0..143) of Q4_K super-block `b`: d, dmin = fp16 U(0.001,0.05);
 * scales[12] and qs[128] uniform bytes (16 independent 6-bit scales/mins and
 * 256 uniform nibbles, since the packing uses disjoint bits).
 */
GQ_HD uint8_t gq_q4k_byte(uint64_t seed, uint64_t b, uint32_t o) {
  if (o < 4u) {
    uint16_t h = gq_scale_f16(gq_hash(gq_subseed(seed, 1u + (o >> 1)), b));
    return (uint8_t)(h >> (8u * (o & 1u)));
  }
  return gq_byte(seed, b * 144ULL + o);
}

/*
 * Byte `o` (0..143) of a zero-mean Q4_K super-block `b`.  The plain rule
 * above gives w = d*sc*q - dmin*m a mean of about 5 (q averages 7.5 and
 * d, dmin, sc, m are independent and positive), which pushes every hidden
 * state along one direction.  Here each sub-block's min cancels its scale's
 * mean: m_j = sc_j and dmin = fp16(7.5 * d), so w = d*sc_j*(q - 7.5) up to
 * the rounding of dmin.  d and the quants are the plain rule's bytes; the 8
 * six-bit sc_j come from their own stream and are packed as
 * get_scale_min_k4 (quant_matvec_q4_k.c:47-56) unpacks them.
 */
GQ_HD uint8_t gq_q4k_zm_byte(uint64_t seed, uint64_t b, uint32_t o) {
  if (o < 2u) return gq_q4k_byte(seed, b, o);
  if (o < 4u) {
    uint16_t d = (uint16_t)(gq_q4k_byte(seed, b, 0u) | (gq_q4k_byte(seed, b, 1u) << 8));
    uint16_t h = gq_f32_to_f16(7.5f * gq_f16_to_f32(d)); /* the product is exact in fp32 */
    return (uint8_t)(h >> (8u * (o - 2u)));
  }
  if (o < 16u) {
    uint64_t v = gq_hash(gq_subseed(seed, 5u), b); /* sc_j = bits 6j..6j+5 */
    uint32_t i = o - 4u;
    if (i < 8u) { /* scales[i], i = j or j + 4 for j < 4: sc_j (and m_j), top bits of sc_{j+4} */
      uint32_t j = i & 3u;
      return (uint8_t)(((v >> (6u * j)) & 63u) | (((v >> (6u * (j + 4u) + 4u)) & 3u) << 6));
    }
    uint32_t lo = (uint32_t)(v >> (6u * (i - 4u))) & 15u; /* scales[8+j]: low nibbles of sc_{4+j}, m_{4+j} */
    return (uint8_t)(lo | (lo << 4));
  }
  return gq_q4k_byte(seed, b, o);
}

/*
 * Byte `o` (0..209) of Q6_K super-block `b`: ql[128], qh[64] uniform bytes,
 * scales[16] int8 uniform in -32..31, d fp16 U(0.001,0.05).
 */
GQ_HD uint8_t gq_q6k_byte(uint64_t seed, uint64_t b, uint32_t o) {
  if (o >= 208u) {
    uint16_t h = gq_scale_f16(gq_hash(gq_subseed(seed, 3u), b));
    return (uint8_t)(h >> (8u * (o - 208u)));
  }
  uint8_t r = gq_byte(seed, b * 210ULL + o);
  if (o >= 192u) return (uint8_t)(int8_t)((int)(r & 63u) - 32);
  return r;
}

/* Byte `o` (0..33) of Q8_0 block `b`: scale fp16 U(0.001,0.05), 32 int8. */
GQ_HD uint8_t gq_q8_0_byte(uint64_t seed, uint64_t b, uint32_t o) {
  if (o < 2u) {
    uint16_t h = gq_scale_f16(gq_hash(gq_subseed(seed, 4u), b));
    return (uint8_t)(h >> (8u * o));
  }
  return gq_byte(seed, b * 34ULL + o);
}

/* Generator code of the zero-mean Q4_K rule: this flag or'ed into the Q4_K
 * dtype code (the blocks are still Q4_K). */
#define GQ_SYNTH_Q4K_ZERO_MEAN 0x100

#endif /* GQ_SYNTH_H */
