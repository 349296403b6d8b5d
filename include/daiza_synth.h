/*
 * daiza_synth.h — deterministic synthetic inputs for the Q1_0 decode path.
 *
 * Header-only C.  Both the HIP library's host side and the CPU oracle include
 * this file, so a seed names the same bytes on every machine with the same
 * C library.  Everything is counter based: element i of a tensor is a pure
 * function of (tensor key, i), which lets callers generate any slice (one
 * embedding row, one row range of a matrix) without generating the rest.
 *
 * Q1_0 block layout (18 bytes per 128 weights), as the reference stores it in
 * Daiza-engine/src/tensor/quant.rs:1-27 and quant.rs:136-141:
 *   bytes 0..1  fp16 scale, little endian
 *   bytes 2..17 sign bits; bit j of sign byte b is column g*128 + 8*b + j,
 *               bit = 1 -> +scale, bit = 0 -> -scale
 *
 * Distributions (unspecified ones chosen here):
 *   sign bits           Bernoulli(0.5)  (uniform bytes)
 *   Q1_0 scale          f16_rne(|N(0,1)| * 0.02)
 *   dense activations   N(0, 1)                       (config 1 x, config 3 KV)
 *   norm weights        U(0.8, 1.2)
 *   f16 embedding       f16_rne(U(-1, 1))
 *   conv1d weights      N(0, 0.25^2)
 *   ssm_a               -exp(U(-1, 1))   (the tensor stores A = -exp(A_log))
 *   dt_bias             N(0, 0.1^2)
 * Normals come from Box-Muller in double precision (one normal per pair of
 * 53-bit uniforms), rounded once to f32.
 */
#ifndef DAIZA_SYNTH_H
#define DAIZA_SYNTH_H

#include <stdint.h>
#include <string.h>
#include <math.h>

/* The integer-exact generators also compile for the GPU (hipcc), giving the same bits there. */
#if defined(__HIPCC__) || defined(__HIP__)
#define DZ_SYNTH_HD __host__ __device__
#else
#define DZ_SYNTH_HD
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* splitmix64 output function */
static inline DZ_SYNTH_HD uint64_t dz_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

/* Key of one tensor: seed, tensor kind, layer index. */
static inline DZ_SYNTH_HD uint64_t dz_key(uint64_t seed, uint32_t kind, uint32_t layer) {
  return dz_mix64(seed ^ dz_mix64(((uint64_t)kind << 32) | (uint64_t)(layer + 1u)));
}

/* i-th 64-bit word of the stream named by key (splitmix64 at counter i). */
static inline DZ_SYNTH_HD uint64_t dz_word(uint64_t key, uint64_t i) {
  return dz_mix64(key + (i + 1ULL) * 0x9E3779B97F4A7C15ULL);
}

/* uniform double in (0, 1] and [0, 1) from one word */
static inline double dz_u01_open0(uint64_t w) { return (double)((w >> 11) + 1ULL) * (1.0 / 9007199254740992.0); }
static inline double dz_u01(uint64_t w) { return (double)(w >> 11) * (1.0 / 9007199254740992.0); }

/* i-th standard normal of the stream (Box-Muller, cosine branch). */
static inline double dz_normal(uint64_t key, uint64_t i) {
  double u1 = dz_u01_open0(dz_word(key, 2 * i));
  double u2 = dz_u01(dz_word(key, 2 * i + 1));
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
}

/* i-th uniform f32 in [lo, hi): 24-bit uniform, exact in f32, then an f32 affine map. */
static inline DZ_SYNTH_HD float dz_uniform_f32(uint64_t key, uint64_t i, float lo, float hi) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  /* two roundings on every compiler and target: no fused multiply-add */
  float u = (float)(dz_word(key, i) >> 40) * (1.0f / 16777216.0f);
  float span = hi - lo;
  float t = span * u;
  return lo + t;
}

/* f32 -> f16 bits, round to nearest even; overflow -> inf, NaN -> quiet NaN. */
static inline DZ_SYNTH_HD uint16_t dz_f32_to_f16(float v) {
  uint32_t x;
  {
    union { float f; uint32_t u; } cv;
    cv.f = v;
    x = cv.u;
  }
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7C00u); /* |v| >= 65536 */
  if (ax < 0x00800000u) return sign;                        /* f32 subnormal: far below half range */
  int e = (int)(ax >> 23) - 127;
  uint32_t m = (ax & 0x7FFFFFu) | 0x800000u; /* 24-bit significand */
  if (e >= -14) {
    uint32_t keep = m >> 13, rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (keep & 1u))) keep++;
    /* keep holds the implicit bit at bit 10; a rounding carry moves into the exponent */
    return (uint16_t)(sign | (((uint32_t)(e + 14) << 10) + keep));
  }
  int shift = -e - 1; /* value / 2^-24 = m * 2^(e+1) */
  if (shift > 24) return sign;
  uint32_t keep = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (keep & 1u))) keep++;
  return (uint16_t)(sign | keep);
}

/* ---- tensor kinds (stream names) ---- */
enum dz_synth_kind {
  DZ_K_EMBD = 1, DZ_K_OUTPUT_NORM, DZ_K_OUTPUT,
  DZ_K_ATTN_NORM = 16, DZ_K_POST_NORM, DZ_K_FFN_GATE, DZ_K_FFN_UP, DZ_K_FFN_DOWN,
  DZ_K_SSM_QKV = 32, DZ_K_SSM_ALPHA, DZ_K_SSM_BETA, DZ_K_SSM_Z, DZ_K_SSM_OUT,
  DZ_K_SSM_CONV, DZ_K_SSM_A, DZ_K_SSM_DT, DZ_K_SSM_NORM,
  DZ_K_ATT_Q = 48, DZ_K_ATT_K, DZ_K_ATT_V, DZ_K_ATT_O, DZ_K_ATT_QNORM, DZ_K_ATT_KNORM,
  /* standalone inputs */
  DZ_K_X = 64, DZ_K_SSM_STATE, DZ_K_CONV_STATE, DZ_K_KV, DZ_K_TOKENS
};

/*
 * Rows [r0, r1) of a Q1_0 matrix with `cols` columns (a multiple of 128),
 * written in the reference AoS layout: out holds (r1-r0) * (cols/128) * 18 bytes.
 */
static inline void dz_synth_q1_0_rows(uint64_t key, uint64_t cols, uint64_t r0, uint64_t r1, uint8_t* out) {
  uint64_t gpr = cols / 128;
  for (uint64_t r = r0; r < r1; ++r) {
    for (uint64_t g = 0; g < gpr; ++g) {
      uint64_t gi = r * gpr + g;
      uint8_t* blk = out + ((r - r0) * gpr + g) * 18;
      float sc = (float)(fabs(dz_normal(key, gi)) * 0.02);
      uint16_t h = dz_f32_to_f16(sc);
      blk[0] = (uint8_t)(h & 0xFF);
      blk[1] = (uint8_t)(h >> 8);
      /* sign words use counters past the normal stream's range: 2*gi and 2*gi+1 are
         taken by the normal, so signs use the key rotated into a separate stream */
      uint64_t skey = key ^ 0x5A5A5A5A5A5A5A5AULL;
      uint64_t w0 = dz_word(skey, 2 * gi), w1 = dz_word(skey, 2 * gi + 1);
      for (int b = 0; b < 8; ++b) {
        blk[2 + b] = (uint8_t)(w0 >> (8 * b));
        blk[10 + b] = (uint8_t)(w1 >> (8 * b));
      }
    }
  }
}

/* n f32 values = mean + sigma * N(0,1), element i from counter i0 + i */
static inline void dz_synth_normal_f32(uint64_t key, uint64_t i0, uint64_t n, double mean, double sigma, float* out) {
  for (uint64_t i = 0; i < n; ++i) out[i] = (float)(mean + sigma * dz_normal(key, i0 + i));
}

static inline void dz_synth_uniform_f32(uint64_t key, uint64_t i0, uint64_t n, float lo, float hi, float* out) {
  for (uint64_t i = 0; i < n; ++i) out[i] = dz_uniform_f32(key, i0 + i, lo, hi);
}

/* one row of the f16 embedding [vocab][hidden]: f16_rne(U(-1,1)) */
static inline void dz_synth_embd_row_f16(uint64_t key, uint64_t row, uint64_t hidden, uint16_t* out) {
  for (uint64_t c = 0; c < hidden; ++c) out[c] = dz_f32_to_f16(dz_uniform_f32(key, row * hidden + c, -1.0f, 1.0f));
}

/* ssm_a = -exp(A_log), A_log ~ U(-1,1); computed in f32 like a GGUF converter would store it */
static inline void dz_synth_ssm_a(uint64_t key, uint64_t n, float* out) {
  for (uint64_t i = 0; i < n; ++i) out[i] = -expf(dz_uniform_f32(key, i, -1.0f, 1.0f));
}

#ifdef __cplusplus
}
#endif
#endif /* DAIZA_SYNTH_H */
