/*
 * oracle.c — CPU restatement of the reference decode path (guang384/Daiza, Rust + AVX2).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the CPU baseline of bench.py.
 * The product never links this file.  Build: oracle/Makefile (gcc -O2 -mavx2 -mfma -mf16c
 * -ffp-contract=off), so scalar expressions round exactly like the reference's Rust code
 * (Rust never contracts a*b+c) and the vector code issues the reference's intrinsics in its order.
 *
 * Citations are to /root/reference/Daiza-engine/src/... unless the path says otherwise.
 *
 * Pinning (tests/test_oracle_cpu.py): every function is checked against known answers, closed
 * forms, float64 brute force or the independent float64 restatement tests/npref.py; or_siphash
 * against the published SipHash-2-4 vectors (tests/test_session_cpu.py).  Parity
 * unpinned (matched within tolerance only; only running the reference could fix the bits):
 * sigmoid_ps / silu_ps (vendor-specific _mm256_rcp_ps) and libm expf/logf/powf/sinf/cosf, which
 * the reference takes from its platform's libm and this file from glibc.
 */
#include "oracle.h"
#include "daiza_synth.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define Q1_GROUP 128
#define Q1_BLOCK 18

/* ------------------------------------------------------------------ f16 */

/* tensor/quant.rs:39-74 — exact binary16 -> f32 incl. subnormal, Inf and NaN payload */
float or_f16_to_f32(uint16_t bits) {
  uint32_t sign = (bits >> 15) & 1u, exp = (bits >> 10) & 0x1Fu, mant = bits & 0x3FFu;
  uint32_t s32 = sign << 31, out;
  if (exp == 0) {
    if (mant == 0) {
      out = s32;
    } else {
      uint32_t m = mant, e = 1;
      while ((m & 0x400u) == 0) { m <<= 1; e += 1; }
      m &= 0x3FFu;
      out = s32 | ((127u - 15u + e) << 23) | (m << 13);
    }
  } else if (exp == 0x1F) {
    out = s32 | 0x7F800000u | (mant << 13);
  } else {
    out = s32 | ((exp + 112u) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

/* the same conversion returned as bits (a float return through ctypes would quiet a signalling NaN) */
uint32_t or_f16_to_f32_bits(uint16_t bits) {
  float f = or_f16_to_f32(bits);
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* tensor/quant.rs:86-108 — branch-free variant that flushes subnormal scales to zero */
float or_f16_to_f32_fast(uint16_t bits) {
  uint32_t t = bits, sign = (t & 0x8000u) << 16, exp = (t >> 10) & 0x1Fu, mant = t & 0x3FFu;
  uint32_t nz = exp != 0, inf = exp == 0x1F;
  uint32_t e32 = nz * (exp + 112u) + inf * 112u;
  uint32_t out = sign | (e32 << 23) | (mant << 13);
  float f;
  memcpy(&f, &out, 4);
  return f;
}

/* tensor/quant.rs:161-194 — w = (bit*2 - 1) * scale, one row */
void or_dequant_row(const uint8_t* aos, size_t row, size_t cols, float* out) {
  size_t gpr = cols / Q1_GROUP;
  const uint8_t* rb = aos + row * gpr * Q1_BLOCK;
  size_t o = 0;
  for (size_t g = 0; g < gpr; ++g) {
    const uint8_t* blk = rb + g * Q1_BLOCK;
    float scale = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int b = 0; b < 16; ++b)
      for (int j = 0; j < 8; ++j) {
        float bit = (float)((blk[2 + b] >> j) & 1);
        out[o++] = (bit * 2.0f - 1.0f) * scale;
      }
  }
}

/* ------------------------------------------------------------------ SIMD helpers */

/* math/simd_exp.rs:354-362: ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) */
static inline float hsum_ps(__m256 v) {
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 s = _mm_add_ps(hi, lo);
  __m128 sh = _mm_movehdup_ps(s);
  __m128 ss = _mm_add_ps(s, sh);
  __m128 s2 = _mm_movehl_ps(ss, ss);
  return _mm_cvtss_f32(_mm_add_ss(ss, s2));
}

/* the same reduction order on 8 scalars */
static inline float hsum8(const float* l) { return ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7])); }

/* tensor/quant.rs:208-225: SIGN_LUT[b][j] = bit j of b ? +1 : -1 */
static float SIGN_LUT[256][8] __attribute__((aligned(32)));
static void init_sign_lut(void) {
  static int done = 0;
  if (done) return;
  for (int b = 0; b < 256; ++b)
    for (int j = 0; j < 8; ++j) SIGN_LUT[b][j] = ((b >> j) & 1) ? 1.0f : -1.0f;
  done = 1;
}

static inline __m256 cvt_scale(const uint8_t* blk) {
  return _mm256_cvtph_ps(_mm_set1_epi16((short)(uint16_t)(blk[0] | (blk[1] << 8))));
}

/* ------------------------------------------------------------------ row kernels */

/* tensor/quant.rs:614-740 dot_q1_0_row_quad_avx2 (V5 fold: two chains per row, two scale FMAs per group) */
static void dot_quad_avx2(const uint8_t* aos, size_t r0, size_t cols, const float* x, float out[4]) {
  size_t gpr = cols / Q1_GROUP, rowb = gpr * Q1_BLOCK;
  const uint8_t* R[4] = {aos + r0 * rowb, aos + (r0 + 1) * rowb, aos + (r0 + 2) * rowb, aos + (r0 + 3) * rowb};
  __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
  const __m256 zero = _mm256_setzero_ps();
  for (size_t g = 0; g < gpr; ++g) {
    __m256 sc[4];
    const uint8_t* sp[4];
    for (int r = 0; r < 4; ++r) {
      const uint8_t* blk = R[r] + g * Q1_BLOCK;
      sc[r] = cvt_scale(blk);
      sp[r] = blk + 2;
    }
    const float* xp = x + g * Q1_GROUP;
    __m256 c0[4] = {zero, zero, zero, zero}, c1[4] = {zero, zero, zero, zero};
    for (int bi = 0; bi < 16; bi += 2) {
      __m256 x0 = _mm256_loadu_ps(xp + bi * 8);
      __m256 x1 = _mm256_loadu_ps(xp + (bi + 1) * 8);
      for (int r = 0; r < 4; ++r) {
        c0[r] = _mm256_fmadd_ps(_mm256_load_ps(SIGN_LUT[sp[r][bi]]), x0, c0[r]);
        c1[r] = _mm256_fmadd_ps(_mm256_load_ps(SIGN_LUT[sp[r][bi + 1]]), x1, c1[r]);
      }
    }
    for (int r = 0; r < 4; ++r) {
      acc[r] = _mm256_fmadd_ps(sc[r], c0[r], acc[r]);
      acc[r] = _mm256_fmadd_ps(sc[r], c1[r], acc[r]);
    }
  }
  for (int r = 0; r < 4; ++r) out[r] = hsum_ps(acc[r]);
}

/*
 * Scalar statement of the same kernels, lane by lane.  fmaf(+-1, x, a) is the AVX2
 * FMA with a SIGN_LUT operand; every reference variant keeps 8 lanes per row and ends in hsum.
 *  quad   (quant.rs:614-740): chains over even / odd sign bytes; acc = fma(s, c0, acc); acc = fma(s, c1, acc)
 *  triple (quant.rs:492-600): chains over even / odd bytes;      acc = fma(s, c0 + c1, acc)
 *  dual   (quant.rs:361-490) and single (quant.rs:267-330): four chains over bytes mod 4;
 *                                                              acc = fma(s, (c0+c1)+(c2+c3), acc)
 */
float or_dot_row_scalar(const uint8_t* aos, size_t row, size_t cols, const float* x, int variant) {
  init_sign_lut();
  size_t gpr = cols / Q1_GROUP;
  const uint8_t* rb = aos + row * gpr * Q1_BLOCK;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (size_t g = 0; g < gpr; ++g) {
    const uint8_t* blk = rb + g * Q1_BLOCK;
    /* every AVX2 row kernel converts the scale with vcvtph2ps (exact IEEE, subnormals included) */
    float s = _cvtsh_ss((unsigned short)(blk[0] | (blk[1] << 8)));
    const float* xp = x + g * Q1_GROUP;
    for (int l = 0; l < 8; ++l) {
      float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      int nch = (variant >= 3) ? 2 : 4;
      for (int bi = 0; bi < 16; ++bi) {
        int ch = bi % nch;
        c[ch] = fmaf(SIGN_LUT[blk[2 + bi]][l], xp[bi * 8 + l], c[ch]);
      }
      if (variant == 4) {
        acc[l] = fmaf(s, c[0], acc[l]);
        acc[l] = fmaf(s, c[1], acc[l]);
      } else if (variant == 3) {
        acc[l] = fmaf(s, c[0] + c[1], acc[l]);
      } else {
        acc[l] = fmaf(s, (c[0] + c[1]) + (c[2] + c[3]), acc[l]);
      }
    }
  }
  return hsum8(acc);
}

/*
 * Rows [a, b) the way one work-stealing chunk runs them (weights.rs:922-953 and the serial
 * path weights.rs:170-199): quads from a, then a triple, dual or single tail.
 */
static void rows_chunk(const uint8_t* aos, size_t cols, const float* x, float* y, size_t a, size_t b, int accumulate) {
  size_t i = a;
  float r4[4];
  for (; i + 3 < b; i += 4) {
    dot_quad_avx2(aos, i, cols, x, r4);
    for (int k = 0; k < 4; ++k) y[i + k] = accumulate ? y[i + k] + r4[k] : r4[k];
  }
  size_t rem = b - i;
  int variant = rem == 3 ? 3 : (rem == 2 ? 2 : 1);
  for (; i < b; ++i) {
    float v = or_dot_row_scalar(aos, i, cols, x, variant);
    y[i] = accumulate ? y[i] + v : v;
  }
}

void or_matvec(const uint8_t* aos, size_t rows, size_t cols, const float* x, float* y, int accumulate, int nthreads) {
  init_sign_lut();
  if (nthreads <= 0) nthreads = omp_get_num_procs();
  /* weights.rs:59-69: 128-row chunks; threshold rows >= 1024 for the pool (weights.rs:159-160) */
  const size_t chunk = 128;
  if (nthreads == 1 || rows < 1024) {
    rows_chunk(aos, cols, x, y, 0, rows, accumulate);
    return;
  }
  size_t nchunks = (rows + chunk - 1) / chunk;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (size_t c = 0; c < nchunks; ++c) {
    size_t a = c * chunk, b = a + chunk < rows ? a + chunk : rows;
    rows_chunk(aos, cols, x, y, a, b, accumulate);
  }
}

void or_matvec_scalar(const uint8_t* aos, size_t rows, size_t cols, const float* x, float* y, int accumulate) {
  init_sign_lut();
  size_t i = 0, n4 = rows / 4 * 4;
  for (; i < n4; ++i) {
    /* every row of a quad group uses the quad chain structure */
    float v = or_dot_row_scalar(aos, i, cols, x, 4);
    y[i] = accumulate ? y[i] + v : v;
  }
  size_t rem = rows - i;
  int variant = rem == 3 ? 3 : (rem == 2 ? 2 : 1);
  for (; i < rows; ++i) {
    float v = or_dot_row_scalar(aos, i, cols, x, variant);
    y[i] = accumulate ? y[i] + v : v;
  }
}

/* ------------------------------------------------------------------ transcendental glue */

static const float LN2_F = 0.693147180559945309417232121458176568f; /* std::f32::consts::LN_2 */
#define LN2_INV (1.0f / LN2_F)

/* math/simd_exp.rs:44-85 exp_ps: clamp, n = round(x/ln2), degree-5 Horner, 2^n via exponent bits */
static inline __m256 exp_ps(__m256 x) {
  x = _mm256_max_ps(_mm256_min_ps(x, _mm256_set1_ps(88.0f)), _mm256_set1_ps(-88.0f));
  __m256 n_f = _mm256_mul_ps(x, _mm256_set1_ps(LN2_INV));
  n_f = _mm256_round_ps(n_f, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m256 r = _mm256_fnmadd_ps(n_f, _mm256_set1_ps(LN2_F), x);
  __m256 p = _mm256_set1_ps(1.0f / 120.0f);
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 24.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 6.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  __m256 nc = _mm256_max_ps(_mm256_min_ps(n_f, _mm256_set1_ps(129.0f)), _mm256_set1_ps(-126.0f));
  __m256i ni = _mm256_cvtps_epi32(nc);
  __m256i eb = _mm256_slli_epi32(_mm256_add_epi32(ni, _mm256_set1_epi32(127)), 23);
  return _mm256_mul_ps(_mm256_castsi256_ps(eb), p);
}

/* math/simd_exp.rs:101-111: 1 / (1 + exp(-x)) with rcp + one Newton step */
static inline __m256 sigmoid_ps(__m256 x) {
  __m256 nx = _mm256_xor_ps(x, _mm256_set1_ps(-0.0f));
  __m256 e = exp_ps(nx);
  __m256 d = _mm256_add_ps(_mm256_set1_ps(1.0f), e);
  __m256 y0 = _mm256_rcp_ps(d);
  return _mm256_mul_ps(y0, _mm256_fnmadd_ps(d, y0, _mm256_set1_ps(2.0f)));
}

/* math/simd_exp.rs:119-123 */
static inline __m256 silu_ps(__m256 x) { return _mm256_mul_ps(x, sigmoid_ps(x)); }

void or_exp_ps(const float* x, float* y, size_t n) {
  for (size_t i = 0; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, exp_ps(_mm256_loadu_ps(x + i)));
}
void or_sigmoid_ps(const float* x, float* y, size_t n) {
  for (size_t i = 0; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, sigmoid_ps(_mm256_loadu_ps(x + i)));
}
void or_silu_ps(const float* x, float* y, size_t n) {
  for (size_t i = 0; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, silu_ps(_mm256_loadu_ps(x + i)));
}
/* math/simd_exp.rs:156-167 / 140-151: broadcast, vector op, lane 0 */
float or_exp_fast(float x) { return _mm256_cvtss_f32(exp_ps(_mm256_set1_ps(x))); }
float or_sigmoid_fast(float x) { return _mm256_cvtss_f32(sigmoid_ps(_mm256_set1_ps(x))); }

/* math/simd_exp.rs:213-238 silu_inplace_simd (scalar tail x / (1 + exp(-x))) */
static void silu_inplace(float* x, size_t n) {
  size_t n8 = n / 8 * 8;
  for (size_t i = 0; i < n8; i += 8) _mm256_storeu_ps(x + i, silu_ps(_mm256_loadu_ps(x + i)));
  for (size_t i = n8; i < n; ++i) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* math/simd_exp.rs:187-211 sigmoid_inplace_simd */
static void sigmoid_inplace(float* x, size_t n) {
  size_t n8 = n / 8 * 8;
  for (size_t i = 0; i < n8; i += 8) _mm256_storeu_ps(x + i, sigmoid_ps(_mm256_loadu_ps(x + i)));
  for (size_t i = n8; i < n; ++i) x[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* math/simd_exp.rs:247-271 mul_inplace_simd */
static void mul_inplace(float* d, const float* s, size_t n) {
  size_t n8 = n / 8 * 8;
  for (size_t i = 0; i < n8; i += 8) _mm256_storeu_ps(d + i, _mm256_mul_ps(_mm256_loadu_ps(d + i), _mm256_loadu_ps(s + i)));
  for (size_t i = n8; i < n; ++i) d[i] *= s[i];
}

/* math/simd_exp.rs:273-296 swiglu_inplace_simd: gate = silu(gate) * up */
void or_swiglu(float* g, const float* u, size_t n) {
  size_t n8 = n / 8 * 8;
  for (size_t i = 0; i < n8; i += 8)
    _mm256_storeu_ps(g + i, _mm256_mul_ps(silu_ps(_mm256_loadu_ps(g + i)), _mm256_loadu_ps(u + i)));
  for (size_t i = n8; i < n; ++i) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* math/simd_exp.rs:488-507 scale_inplace_avx2 */
static void scale_inplace(float* x, size_t n, float s) {
  size_t i = 0;
  __m256 sv = _mm256_set1_ps(s);
  for (; i + 8 <= n; i += 8) _mm256_storeu_ps(x + i, _mm256_mul_ps(sv, _mm256_loadu_ps(x + i)));
  for (; i < n; ++i) x[i] *= s;
}

/* math/simd_exp.rs:551-598: first index of the maximum (strict >), NaN never wins, -inf start */
int or_argmax(const float* x, size_t n) {
  int best = 0;
  float bv = -INFINITY;
  for (size_t i = 0; i < n; ++i)
    if (x[i] > bv) { bv = x[i]; best = (int)i; }
  return best;
}

/* ------------------------------------------------------------------ norms */

/* math/rmsnorm.rs:82-145 rmsnorm_into_avx2 (rmsnorm_inplace_avx2 17-80 has the same arithmetic) */
void or_rmsnorm_into(const float* x, float* y, const float* w, size_t n, float eps) {
  float nf = (float)n;
  __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps(), s2 = _mm256_setzero_ps(), s3 = _mm256_setzero_ps();
  size_t i = 0, n32 = n / 32 * 32, n8 = n / 8 * 8;
  for (; i < n32; i += 32) {
    __m256 v0 = _mm256_loadu_ps(x + i), v1 = _mm256_loadu_ps(x + i + 8);
    __m256 v2 = _mm256_loadu_ps(x + i + 16), v3 = _mm256_loadu_ps(x + i + 24);
    s0 = _mm256_fmadd_ps(v0, v0, s0);
    s1 = _mm256_fmadd_ps(v1, v1, s1);
    s2 = _mm256_fmadd_ps(v2, v2, s2);
    s3 = _mm256_fmadd_ps(v3, v3, s3);
  }
  for (; i < n8; i += 8) {
    __m256 v = _mm256_loadu_ps(x + i);
    s0 = _mm256_fmadd_ps(v, v, s0);
  }
  s0 = _mm256_add_ps(_mm256_add_ps(s0, s1), _mm256_add_ps(s2, s3));
  float ss = hsum_ps(s0);
  for (size_t j = n8; j < n; ++j) ss += x[j] * x[j];
  float inv = 1.0f / sqrtf(ss / nf + eps);
  __m256 iv = _mm256_set1_ps(inv);
  i = 0;
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(y + i, _mm256_mul_ps(_mm256_mul_ps(_mm256_loadu_ps(x + i), iv), _mm256_loadu_ps(w + i)));
  for (; i < n; ++i) y[i] = x[i] * inv * w[i];
}

/* model/ssm.rs:106-135 l2norm_inplace_avx2 */
void or_l2norm_inplace(float* x, size_t n, float eps) {
  __m256 sv = _mm256_setzero_ps();
  size_t i = 0, n8 = n / 8 * 8;
  for (; i < n8; i += 8) {
    __m256 v = _mm256_loadu_ps(x + i);
    sv = _mm256_fmadd_ps(v, v, sv);
  }
  float ss = hsum_ps(sv);
  for (size_t j = n8; j < n; ++j) ss += x[j] * x[j];
  float inv = 1.0f / sqrtf(ss + eps);
  __m256 iv = _mm256_set1_ps(inv);
  for (i = 0; i < n8; i += 8) _mm256_storeu_ps(x + i, _mm256_mul_ps(_mm256_loadu_ps(x + i), iv));
  for (size_t j = n8; j < n; ++j) x[j] *= inv;
}

/* ------------------------------------------------------------------ rope */

/* math/rope.rs:27-38 (first half of cat([freqs, freqs])) */
void or_rope_freqs(int rope_dim, float base, float* freqs) {
  int half = rope_dim / 2;
  for (int i = 0; i < half; ++i) freqs[i] = 1.0f / powf(base, (float)(2 * i) / (float)rope_dim);
}

/* math/rope.rs:82-101 text M-RoPE: every pair uses position t; cos/sin duplicated for both halves */
void or_rope_cos_sin(int pos, const float* freqs, int rope_dim, float* co, float* si) {
  int half = rope_dim / 2;
  for (int i = 0; i < half; ++i) {
    float th = (float)pos * freqs[i];
    float c = cosf(th), s = sinf(th);
    co[i] = c; si[i] = s; co[i + half] = c; si[i + half] = s;
  }
}

/* math/rope.rs:187-231 AVX2 path: out1 = x1*c + x2*s, out2 = x2*c + x1*s (both '+', as the reference) */
void or_rope_partial(float* x, int rope_dim, const float* co, const float* si) {
  int half = rope_dim / 2, i = 0;
  if (half >= 8) {
    for (; i + 8 <= half; i += 8) {
      __m256 x1 = _mm256_loadu_ps(x + i), x2 = _mm256_loadu_ps(x + i + half);
      __m256 c = _mm256_loadu_ps(co + i), s = _mm256_loadu_ps(si + i);
      __m256 o1 = _mm256_fmadd_ps(x1, c, _mm256_mul_ps(x2, s));
      __m256 o2 = _mm256_fmadd_ps(x2, c, _mm256_mul_ps(x1, s));
      _mm256_storeu_ps(x + i, o1);
      _mm256_storeu_ps(x + i + half, o2);
    }
    for (; i < half; ++i) {
      float x1 = x[i], x2 = x[i + half];
      x[i] = x1 * co[i] + x2 * si[i];
      x[i + half] = x2 * co[i] + x1 * si[i];
    }
  } else {
    for (; i < half; ++i) {
      float x1 = x[i], x2 = x[i + half];
      x[i] = x1 * co[i] + x2 * si[i];
      x[i + half] = x2 * co[i] + x1 * si[i];
    }
  }
}

/* ------------------------------------------------------------------ DeltaNet */

/* model/ssm.rs:61-67 */
static inline float softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

/* model/ssm.rs:153-180 ssm_scan_vhead + 378-418 ssm_scan_fused_avx2 (row-major S[i][j]) */
void or_ssm_scan_vhead(float* s, float* y, const float* q, const float* k, const float* v, float a_vh,
                       float alpha_vh, float beta_vh, float dt_bias_vh, int hd) {
  float g = a_vh * softplus(alpha_vh + dt_bias_vh);
  float decay = expf(g);
  float beta = or_sigmoid_fast(beta_vh);
  __m256 dv = _mm256_set1_ps(decay);
  for (int i = 0; i < hd; ++i) {
    float* row = s + (size_t)i * hd;
    __m256 kv = _mm256_setzero_ps();
    for (int j = 0; j < hd; j += 8) {
      __m256 sn = _mm256_mul_ps(_mm256_loadu_ps(row + j), dv);
      _mm256_storeu_ps(row + j, sn);
      kv = _mm256_fmadd_ps(sn, _mm256_loadu_ps(k + j), kv);
    }
    float kvm = hsum_ps(kv);
    float di = (v[i] - kvm) * beta;
    __m256 div = _mm256_set1_ps(di);
    __m256 ya = _mm256_setzero_ps();
    for (int j = 0; j < hd; j += 8) {
      __m256 sn = _mm256_fmadd_ps(div, _mm256_loadu_ps(k + j), _mm256_loadu_ps(row + j));
      _mm256_storeu_ps(row + j, sn);
      ya = _mm256_fmadd_ps(sn, _mm256_loadu_ps(q + j), ya);
    }
    y[i] = hsum_ps(ya);
  }
}

/* model/ssm.rs:246-286 ssm_output_gate_avx2: y = ((y * inv_rms) * w) * z per v-head */
static void ssm_output_gate(float* y, const float* z, const float* w, int nvh, int hd, float eps) {
  float inv_hd = 1.0f / (float)hd;
  for (int h = 0; h < nvh; ++h) {
    float* yh = y + (size_t)h * hd;
    const float* zh = z + (size_t)h * hd;
    __m256 sv = _mm256_setzero_ps();
    for (int i = 0; i < hd; i += 8) {
      __m256 v = _mm256_loadu_ps(yh + i);
      sv = _mm256_fmadd_ps(v, v, sv);
    }
    float ss = hsum_ps(sv);
    float inv = 1.0f / sqrtf(ss * inv_hd + eps);
    __m256 iv = _mm256_set1_ps(inv);
    for (int i = 0; i < hd; i += 8) {
      __m256 r = _mm256_mul_ps(_mm256_mul_ps(_mm256_mul_ps(_mm256_loadu_ps(yh + i), iv), _mm256_loadu_ps(w + i)),
                               _mm256_loadu_ps(zh + i));
      _mm256_storeu_ps(yh + i, r);
    }
  }
}

/* ------------------------------------------------------------------ attention helpers */

/* math/simd_exp.rs:306-331 dot_product_avx2 (two accumulators over 16-wide steps) */
static float dot_avx2(const float* a, const float* b, int len) {
  __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
  int i = 0;
  for (; i + 16 <= len; i += 16) {
    s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
    s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), s1);
  }
  for (; i + 8 <= len; i += 8) s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
  s0 = _mm256_add_ps(s0, s1);
  return hsum_ps(s0);
}

/* math/simd_exp.rs:416-455: y = y*alpha + beta*x */
static void online_v_update(float* y, float alpha, float beta, const float* x, int len) {
  __m256 av = _mm256_set1_ps(alpha), bv = _mm256_set1_ps(beta);
  int i = 0;
  for (; i + 16 <= len; i += 16) {
    __m256 y0 = _mm256_loadu_ps(y + i), x0 = _mm256_loadu_ps(x + i);
    __m256 y1 = _mm256_loadu_ps(y + i + 8), x1 = _mm256_loadu_ps(x + i + 8);
    _mm256_storeu_ps(y + i, _mm256_fmadd_ps(bv, x0, _mm256_mul_ps(av, y0)));
    _mm256_storeu_ps(y + i + 8, _mm256_fmadd_ps(bv, x1, _mm256_mul_ps(av, y1)));
  }
  for (; i + 8 <= len; i += 8) {
    __m256 y0 = _mm256_loadu_ps(y + i), x0 = _mm256_loadu_ps(x + i);
    _mm256_storeu_ps(y + i, _mm256_fmadd_ps(bv, x0, _mm256_mul_ps(av, y0)));
  }
}

/* ------------------------------------------------------------------ LcgRng */

/* math/sampling.rs:9-19 */
float or_lcg_next(uint64_t* state) {
  *state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
  uint32_t bits = (uint32_t)((*state >> 40) & 0xFFFFFFu);
  return (float)bits / (float)0x1000000;
}

/* ------------------------------------------------------------------ sampling (speculative verify) */

/* hmax_ps (simd_exp.rs:375-383) */
static inline float hmax_ps(__m256 v) {
  __m128 m = _mm_max_ps(_mm256_extractf128_ps(v, 1), _mm256_castps256_ps128(v));
  __m128 s = _mm_max_ps(m, _mm_movehdup_ps(m));
  return _mm_cvtss_f32(_mm_max_ss(s, _mm_movehl_ps(s, s)));
}

/* softmax_inplace (math/softmax.rs:15-80): AVX2 max, exp_ps + sum, multiply by 1/sum */
void or_softmax_inplace(float* x, size_t n) {
  size_t n8 = n / 8 * 8, i;
  __m256 mv = _mm256_set1_ps(x[0]);
  for (i = 0; i < n8; i += 8) mv = _mm256_max_ps(mv, _mm256_loadu_ps(x + i));
  float mx = hmax_ps(mv);
  for (; i < n; ++i)
    if (x[i] > mx) mx = x[i];
  __m256 mxv = _mm256_set1_ps(mx), sv = _mm256_setzero_ps();
  for (i = 0; i < n8; i += 8) {
    __m256 e = exp_ps(_mm256_sub_ps(_mm256_loadu_ps(x + i), mxv));
    _mm256_storeu_ps(x + i, e);
    sv = _mm256_add_ps(sv, e);
  }
  float sum = hsum_ps(sv);
  for (i = n8; i < n; ++i) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  float inv = 1.0f / sum;
  __m256 iv = _mm256_set1_ps(inv);
  for (i = 0; i < n8; i += 8) _mm256_storeu_ps(x + i, _mm256_mul_ps(_mm256_loadu_ps(x + i), iv));
  for (i = n8; i < n; ++i) x[i] *= inv;
}

/* softmax_pair_single_avx2 (simd_exp.rs:656-767) */
void or_softmax_pair_single(const float* t, const float* d, size_t n, size_t idx, float* p, float* q) {
  size_t n8 = n / 8 * 8, i;
  __m256 tm = _mm256_set1_ps(t[0]), dm = _mm256_set1_ps(d[0]);
  for (i = 0; i < n8; i += 8) {
    tm = _mm256_max_ps(tm, _mm256_loadu_ps(t + i));
    dm = _mm256_max_ps(dm, _mm256_loadu_ps(d + i));
  }
  float tmax = hmax_ps(tm), dmax = hmax_ps(dm);
  for (; i < n; ++i) {
    if (t[i] > tmax) tmax = t[i];
    if (d[i] > dmax) dmax = d[i];
  }
  __m256 tmv = _mm256_set1_ps(tmax), dmv = _mm256_set1_ps(dmax), ts = _mm256_setzero_ps(), ds = _mm256_setzero_ps();
  float ti = 0.f, di = 0.f;
  for (i = 0; i < n8; i += 8) {
    __m256 te = exp_ps(_mm256_sub_ps(_mm256_loadu_ps(t + i), tmv));
    __m256 de = exp_ps(_mm256_sub_ps(_mm256_loadu_ps(d + i), dmv));
    ts = _mm256_add_ps(ts, te);
    ds = _mm256_add_ps(ds, de);
    if (idx >= i && idx < i + 8) {
      float bt[8], bd[8];
      _mm256_storeu_ps(bt, te);
      _mm256_storeu_ps(bd, de);
      ti = bt[idx - i];
      di = bd[idx - i];
    }
  }
  float tsum = hsum_ps(ts), dsum = hsum_ps(ds);
  for (i = n8; i < n; ++i) {
    float te = expf(t[i] - tmax), de = expf(d[i] - dmax);
    tsum += te;
    dsum += de;
    if (i == idx) {
      ti = te;
      di = de;
    }
  }
  if (tsum <= 0.f) tsum = 1.f;
  if (dsum <= 0.f) dsum = 1.f;
  *p = ti / tsum;
  *q = di / dsum;
}

/* sample_top_k_top_p_into (math/sampling.rs:144-247).  The reference orders the top k with
 * select_nth_unstable + sort (tie order unspecified); ties here go to the lower index. */
uint32_t or_sample_top_k_top_p(const float* logits, size_t n, float temperature, int top_k, float top_p,
                               uint64_t* rng) {
  if (temperature <= 0.f) return (uint32_t)or_argmax(logits, n);
  float inv_t = 1.0f / temperature;
  size_t k = (size_t)top_k < n ? (size_t)top_k : n;
  uint32_t* top = (uint32_t*)malloc(k * sizeof(uint32_t));
  float* val = (float*)malloc(k * sizeof(float));
  size_t have = 0;
  for (size_t i = 0; i < n; ++i) {
    float v = logits[i] * inv_t;  /* scale_avx2: one multiply per element */
    if (have == k && !(v > val[k - 1])) continue;
    size_t j = have < k ? have++ : k - 1;
    while (j > 0 && v > val[j - 1]) {
      val[j] = val[j - 1];
      top[j] = top[j - 1];
      --j;
    }
    val[j] = v;
    top[j] = (uint32_t)i;
  }
  float mx = -INFINITY;
  for (size_t j = 0; j < k; ++j)
    if (val[j] > mx) mx = val[j];
  float* pr = (float*)malloc(k * sizeof(float));
  float sum = 0.f;
  for (size_t j = 0; j < k; ++j) pr[j] = expf(val[j] - mx);
  for (size_t j = 0; j < k; ++j) sum += pr[j];
  float inv = 1.0f / sum;
  for (size_t j = 0; j < k; ++j) pr[j] *= inv;
  float cum = 0.f;
  size_t cut = k;
  for (size_t j = 0; j < k; ++j) {
    cum += pr[j];
    if (cum >= top_p) {
      cut = j + 1;
      break;
    }
  }
  float ns = 0.f;
  for (size_t j = 0; j < cut; ++j) ns += pr[j];
  float ninv = 1.0f / ns;
  for (size_t j = 0; j < cut; ++j) pr[j] *= ninv;
  float r = or_lcg_next(rng), acc = 0.f;
  uint32_t chosen = top[0];
  for (size_t j = 0; j < cut; ++j) {
    acc += pr[j];
    if (r <= acc) {
      chosen = top[j];
      break;
    }
  }
  free(top);
  free(val);
  free(pr);
  return chosen;
}

/* sample_bonus (Daiza-runtime/src/engine.rs:1833-1866) with residual_max_zero_sum_avx2
 * (simd_exp.rs:605-642) */
uint32_t or_sample_bonus(const float* target, const float* draft, size_t n, float temperature, int top_k,
                         float top_p, uint64_t* rng) {
  float* p = (float*)malloc(n * sizeof(float));
  float* q = (float*)malloc(n * sizeof(float));
  memcpy(p, target, n * sizeof(float));
  memcpy(q, draft, n * sizeof(float));
  or_softmax_inplace(p, n);
  or_softmax_inplace(q, n);
  size_t n8 = n / 8 * 8, i;
  __m256 sv = _mm256_setzero_ps(), z = _mm256_setzero_ps();
  for (i = 0; i < n8; i += 8) {
    __m256 r = _mm256_max_ps(_mm256_sub_ps(_mm256_loadu_ps(p + i), _mm256_loadu_ps(q + i)), z);
    _mm256_storeu_ps(p + i, r);
    sv = _mm256_add_ps(sv, r);
  }
  float sum = hsum_ps(sv);
  for (i = n8; i < n; ++i) {
    float r = fmaxf(p[i] - q[i], 0.f);
    p[i] = r;
    sum += r;
  }
  uint32_t out;
  if (sum <= 1e-12f) {
    out = or_sample_top_k_top_p(target, n, temperature, top_k, top_p, rng);
  } else {
    float inv = 1.0f / sum;
    for (i = 0; i < n; ++i) p[i] = logf(p[i] * inv);
    out = or_sample_top_k_top_p(p, n, temperature, top_k, top_p, rng);
  }
  free(p);
  free(q);
  return out;
}

/* leviathan_check (Daiza-runtime/src/engine.rs:1791-1819) */
int or_leviathan_check(const float* target, const float* draft, size_t n, uint32_t token, float temperature,
                       uint64_t* rng) {
  if (temperature <= 0.f) return (uint32_t)or_argmax(target, n) == token;
  float p, q;
  or_softmax_pair_single(target, draft, n, token, &p, &q);
  float r = q > 1e-12f ? p / q : 0.f;
  return or_lcg_next(rng) < r;
}

/* ------------------------------------------------------------------ model */

typedef struct {
  uint8_t* q;
  size_t rows, cols;
} qmat;

typedef struct {
  int is_attn;
  float *attn_norm, *post_norm;
  qmat gate, up, down;
  /* DeltaNet */
  qmat qkv, alpha, beta, z, out;
  float* conv_w_t; /* [conv_k][qkv_dim] (transposed at load, weights.rs:1339-1356) */
  float *ssm_a, *dt_bias, *ssm_norm;
  /* attention */
  qmat wq, wk, wv, wo;
  float *q_norm, *k_norm;
} or_layer;

struct or_model {
  dz_config cfg;
  uint64_t seed;
  int nthreads;
  or_layer* L;
  float* output_norm;
  qmat output;
  qmat embd_q;
  uint64_t embd_key;
  float freqs[128];
};

struct or_ctx {
  or_model* m;
  int pos;
  float** ssm;      /* per layer [vh][hd][hd] */
  float** conv;     /* per layer [conv_k][qkv_dim], NULL until first use (ssm.rs:467-470) */
  int* conv_head;
  float** kk;       /* per layer [kvh][cap][hd] */
  float** vv;
  int* kv_len;
  /* workspace */
  float *h, *normed, *qkv, *al, *be, *z, *cout, *q, *k, *v, *y;
  float *qt, *aq, *ag, *ak, *av, *ao, *mg, *mu, *logits;
  float co[128], si[128];
};

static int is_attn_layer(const dz_config* c, int i) {
  if (c->full_attn_interval == 0) return 1;
  return i % c->full_attn_interval == c->full_attn_interval - 1;
}

static qmat gen_q(uint64_t seed, int kind, int layer, size_t rows, size_t cols, int nthreads) {
  qmat m;
  m.rows = rows;
  m.cols = cols;
  m.q = (uint8_t*)malloc(rows * (cols / Q1_GROUP) * Q1_BLOCK);
  uint64_t key = dz_key(seed, (uint32_t)kind, (uint32_t)layer);
  size_t rb = (cols / Q1_GROUP) * Q1_BLOCK;
  size_t chunk = 64, nch = (rows + chunk - 1) / chunk;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (size_t c = 0; c < nch; ++c) {
    size_t a = c * chunk, b = a + chunk < rows ? a + chunk : rows;
    dz_synth_q1_0_rows(key, cols, a, b, m.q + a * rb);
  }
  return m;
}

static float* gen_uniform(uint64_t seed, int kind, int layer, size_t n, float lo, float hi) {
  float* p = (float*)malloc(n * sizeof(float));
  dz_synth_uniform_f32(dz_key(seed, (uint32_t)kind, (uint32_t)layer), 0, n, lo, hi, p);
  return p;
}
static float* gen_normal(uint64_t seed, int kind, int layer, size_t n, double sigma) {
  float* p = (float*)malloc(n * sizeof(float));
  dz_synth_normal_f32(dz_key(seed, (uint32_t)kind, (uint32_t)layer), 0, n, 0.0, sigma, p);
  return p;
}

or_model* or_model_synth(const dz_config* cfg, uint64_t seed, int nthreads) {
  init_sign_lut();
  or_model* m = (or_model*)calloc(1, sizeof(or_model));
  m->cfg = *cfg;
  m->seed = seed;
  m->nthreads = nthreads > 0 ? nthreads : omp_get_num_procs();
  const dz_config* c = cfg;
  size_t H = (size_t)c->hidden, F = (size_t)c->ffn;
  size_t hd = (size_t)c->ssm_state;
  size_t kdim = (size_t)c->ssm_k_heads * hd, inner = (size_t)c->ssm_v_heads * hd, qkvd = 2 * kdim + inner;
  size_t qdim = (size_t)c->n_head * c->head_dim, kvdim = (size_t)c->n_head_kv * c->head_dim;
  m->L = (or_layer*)calloc((size_t)c->n_layers, sizeof(or_layer));
  for (int i = 0; i < c->n_layers; ++i) {
    or_layer* l = &m->L[i];
    l->is_attn = is_attn_layer(c, i);
    l->attn_norm = gen_uniform(seed, DZ_K_ATTN_NORM, i, H, 0.8f, 1.2f);
    l->post_norm = gen_uniform(seed, DZ_K_POST_NORM, i, H, 0.8f, 1.2f);
    l->gate = gen_q(seed, DZ_K_FFN_GATE, i, F, H, m->nthreads);
    l->up = gen_q(seed, DZ_K_FFN_UP, i, F, H, m->nthreads);
    l->down = gen_q(seed, DZ_K_FFN_DOWN, i, H, F, m->nthreads);
    if (!l->is_attn) {
      l->qkv = gen_q(seed, DZ_K_SSM_QKV, i, qkvd, H, m->nthreads);
      l->alpha = gen_q(seed, DZ_K_SSM_ALPHA, i, (size_t)c->ssm_v_heads, H, m->nthreads);
      l->beta = gen_q(seed, DZ_K_SSM_BETA, i, (size_t)c->ssm_v_heads, H, m->nthreads);
      l->z = gen_q(seed, DZ_K_SSM_Z, i, inner, H, m->nthreads);
      l->out = gen_q(seed, DZ_K_SSM_OUT, i, H, inner, m->nthreads);
      /* GGUF stores conv1d as [qkv_dim][conv_k]; generated in that order then transposed */
      size_t ck = (size_t)c->ssm_conv_kernel;
      float* raw = gen_normal(seed, DZ_K_SSM_CONV, i, qkvd * ck, 0.25);
      l->conv_w_t = (float*)malloc(qkvd * ck * sizeof(float));
      for (size_t ch = 0; ch < qkvd; ++ch)
        for (size_t t = 0; t < ck; ++t) l->conv_w_t[t * qkvd + ch] = raw[ch * ck + t];
      free(raw);
      l->ssm_a = (float*)malloc((size_t)c->ssm_v_heads * sizeof(float));
      dz_synth_ssm_a(dz_key(seed, DZ_K_SSM_A, (uint32_t)i), (uint64_t)c->ssm_v_heads, l->ssm_a);
      l->dt_bias = gen_normal(seed, DZ_K_SSM_DT, i, (size_t)c->ssm_v_heads, 0.1);
      l->ssm_norm = gen_uniform(seed, DZ_K_SSM_NORM, i, hd, 0.8f, 1.2f);
    } else {
      l->wq = gen_q(seed, DZ_K_ATT_Q, i, 2 * qdim, H, m->nthreads);
      l->wk = gen_q(seed, DZ_K_ATT_K, i, kvdim, H, m->nthreads);
      l->wv = gen_q(seed, DZ_K_ATT_V, i, kvdim, H, m->nthreads);
      l->wo = gen_q(seed, DZ_K_ATT_O, i, H, qdim, m->nthreads);
      l->q_norm = gen_uniform(seed, DZ_K_ATT_QNORM, i, (size_t)c->head_dim, 0.8f, 1.2f);
      l->k_norm = gen_uniform(seed, DZ_K_ATT_KNORM, i, (size_t)c->head_dim, 0.8f, 1.2f);
    }
  }
  m->output_norm = gen_uniform(seed, DZ_K_OUTPUT_NORM, -1, H, 0.8f, 1.2f);
  m->output = gen_q(seed, DZ_K_OUTPUT, -1, (size_t)c->vocab, H, m->nthreads);
  m->embd_key = dz_key(seed, DZ_K_EMBD, (uint32_t)-1);
  if (!c->embd_f16) m->embd_q = gen_q(seed, DZ_K_EMBD, -1, (size_t)c->vocab, H, m->nthreads);
  or_rope_freqs(c->rope_dim, c->rope_base, m->freqs);
  return m;
}

static void free_q(qmat* q) { free(q->q); }

void or_model_free(or_model* m) {
  if (!m) return;
  for (int i = 0; i < m->cfg.n_layers; ++i) {
    or_layer* l = &m->L[i];
    free(l->attn_norm); free(l->post_norm);
    free_q(&l->gate); free_q(&l->up); free_q(&l->down);
    if (!l->is_attn) {
      free_q(&l->qkv); free_q(&l->alpha); free_q(&l->beta); free_q(&l->z); free_q(&l->out);
      free(l->conv_w_t); free(l->ssm_a); free(l->dt_bias); free(l->ssm_norm);
    } else {
      free_q(&l->wq); free_q(&l->wk); free_q(&l->wv); free_q(&l->wo);
      free(l->q_norm); free(l->k_norm);
    }
  }
  free(m->L);
  free(m->output_norm);
  free_q(&m->output);
  if (m->embd_q.q) free_q(&m->embd_q);
  free(m);
}

const uint8_t* or_model_q1(or_model* m, int kind, int layer, size_t* rows, size_t* cols) {
  qmat* q = NULL;
  if (layer < 0) {
    if (kind == DZ_K_OUTPUT) q = &m->output;
    else if (kind == DZ_K_EMBD) q = &m->embd_q;
  } else if (layer < m->cfg.n_layers) {
    or_layer* l = &m->L[layer];
    switch (kind) {
      case DZ_K_FFN_GATE: q = &l->gate; break;
      case DZ_K_FFN_UP: q = &l->up; break;
      case DZ_K_FFN_DOWN: q = &l->down; break;
      case DZ_K_SSM_QKV: q = &l->qkv; break;
      case DZ_K_SSM_ALPHA: q = &l->alpha; break;
      case DZ_K_SSM_BETA: q = &l->beta; break;
      case DZ_K_SSM_Z: q = &l->z; break;
      case DZ_K_SSM_OUT: q = &l->out; break;
      case DZ_K_ATT_Q: q = &l->wq; break;
      case DZ_K_ATT_K: q = &l->wk; break;
      case DZ_K_ATT_V: q = &l->wv; break;
      case DZ_K_ATT_O: q = &l->wo; break;
      default: break;
    }
  }
  if (!q || !q->q) return NULL;
  if (rows) *rows = q->rows;
  if (cols) *cols = q->cols;
  return q->q;
}

const float* or_model_f32(or_model* m, int kind, int layer, size_t* n) {
  const dz_config* c = &m->cfg;
  if (layer < 0) {
    if (kind == DZ_K_OUTPUT_NORM) { if (n) *n = (size_t)c->hidden; return m->output_norm; }
    return NULL;
  }
  or_layer* l = &m->L[layer];
  size_t qkvd = (size_t)(2 * c->ssm_k_heads + c->ssm_v_heads) * c->ssm_state;
  switch (kind) {
    case DZ_K_ATTN_NORM: if (n) *n = (size_t)c->hidden; return l->attn_norm;
    case DZ_K_POST_NORM: if (n) *n = (size_t)c->hidden; return l->post_norm;
    case DZ_K_SSM_CONV: if (n) *n = qkvd * (size_t)c->ssm_conv_kernel; return l->conv_w_t;
    case DZ_K_SSM_A: if (n) *n = (size_t)c->ssm_v_heads; return l->ssm_a;
    case DZ_K_SSM_DT: if (n) *n = (size_t)c->ssm_v_heads; return l->dt_bias;
    case DZ_K_SSM_NORM: if (n) *n = (size_t)c->ssm_state; return l->ssm_norm;
    case DZ_K_ATT_QNORM: if (n) *n = (size_t)c->head_dim; return l->q_norm;
    case DZ_K_ATT_KNORM: if (n) *n = (size_t)c->head_dim; return l->k_norm;
    default: return NULL;
  }
}

or_ctx* or_ctx_new(or_model* m) {
  const dz_config* c = &m->cfg;
  or_ctx* x = (or_ctx*)calloc(1, sizeof(or_ctx));
  x->m = m;
  int nl = c->n_layers;
  size_t hd = (size_t)c->ssm_state, H = (size_t)c->hidden, F = (size_t)c->ffn;
  size_t kdim = (size_t)c->ssm_k_heads * hd, inner = (size_t)c->ssm_v_heads * hd, qkvd = 2 * kdim + inner;
  size_t qdim = (size_t)c->n_head * c->head_dim, kvdim = (size_t)c->n_head_kv * c->head_dim;
  x->ssm = (float**)calloc((size_t)nl, sizeof(float*));
  x->conv = (float**)calloc((size_t)nl, sizeof(float*));
  x->conv_head = (int*)calloc((size_t)nl, sizeof(int));
  x->kk = (float**)calloc((size_t)nl, sizeof(float*));
  x->vv = (float**)calloc((size_t)nl, sizeof(float*));
  x->kv_len = (int*)calloc((size_t)nl, sizeof(int));
  for (int i = 0; i < nl; ++i) {
    if (m->L[i].is_attn) {
      size_t n = (size_t)c->n_head_kv * (size_t)c->max_ctx * (size_t)c->head_dim;
      x->kk[i] = (float*)calloc(n, sizeof(float));
      x->vv[i] = (float*)calloc(n, sizeof(float));
    } else {
      x->ssm[i] = (float*)calloc((size_t)c->ssm_v_heads * hd * hd, sizeof(float));
    }
  }
  x->h = (float*)calloc(H, 4); x->normed = (float*)calloc(H, 4);
  x->qkv = (float*)calloc(qkvd, 4); x->al = (float*)calloc((size_t)c->ssm_v_heads, 4);
  x->be = (float*)calloc((size_t)c->ssm_v_heads, 4); x->z = (float*)calloc(inner, 4);
  x->cout = (float*)calloc(qkvd, 4); x->q = (float*)calloc(kdim, 4); x->k = (float*)calloc(kdim, 4);
  x->v = (float*)calloc(inner, 4); x->y = (float*)calloc(inner, 4);
  x->qt = (float*)calloc(2 * qdim, 4); x->aq = (float*)calloc(qdim, 4); x->ag = (float*)calloc(qdim, 4);
  x->ak = (float*)calloc(kvdim, 4); x->av = (float*)calloc(kvdim, 4); x->ao = (float*)calloc(qdim, 4);
  x->mg = (float*)calloc(F, 4); x->mu = (float*)calloc(F, 4);
  x->logits = (float*)calloc((size_t)c->vocab, 4);
  return x;
}

void or_ctx_free(or_ctx* x) {
  if (!x) return;
  for (int i = 0; i < x->m->cfg.n_layers; ++i) { free(x->ssm[i]); free(x->conv[i]); free(x->kk[i]); free(x->vv[i]); }
  free(x->ssm); free(x->conv); free(x->conv_head); free(x->kk); free(x->vv); free(x->kv_len);
  free(x->h); free(x->normed); free(x->qkv); free(x->al); free(x->be); free(x->z); free(x->cout);
  free(x->q); free(x->k); free(x->v); free(x->y); free(x->qt); free(x->aq); free(x->ag); free(x->ak);
  free(x->av); free(x->ao); free(x->mg); free(x->mu); free(x->logits);
  free(x);
}

int or_ctx_pos(or_ctx* x) { return x->pos; }
void or_ctx_set_pos(or_ctx* x, int pos) { x->pos = pos; }

/* KvCache::truncate (kv_cache.rs:119-130) on every attention layer, then pos = len: a longer len
 * leaves a cache as it is; the DeltaNet states and conv rings (SsmState) are not touched. */
void or_kv_truncate(or_ctx* x, int len) {
  for (int i = 0; i < x->m->cfg.n_layers; ++i)
    if (x->m->L[i].is_attn && len < x->kv_len[i]) x->kv_len[i] = len;
  x->pos = len;
}

static void mv(or_ctx* x, const qmat* w, const float* in, float* out, int acc) {
  or_matvec(w->q, w->rows, w->cols, in, out, acc, x->m->nthreads);
}

/* model/ssm.rs:425-616 ssm_forward_into */
static void ssm_forward(or_ctx* x, int li, float* h) {
  const dz_config* c = &x->m->cfg;
  or_layer* l = &x->m->L[li];
  int hd = c->ssm_state, nkh = c->ssm_k_heads, nvh = c->ssm_v_heads, ck = c->ssm_conv_kernel;
  size_t kdim = (size_t)nkh * hd, inner = (size_t)nvh * hd, qkvd = 2 * kdim + inner;
  or_rmsnorm_into(h, x->normed, l->attn_norm, (size_t)c->hidden, c->rms_eps);
  /* matvec_multi: each row is the quad kernel of its own matrix */
  mv(x, &l->qkv, x->normed, x->qkv, 0);
  mv(x, &l->alpha, x->normed, x->al, 0);
  mv(x, &l->beta, x->normed, x->be, 0);
  mv(x, &l->z, x->normed, x->z, 0);
  if (!x->conv[li]) {
    x->conv[li] = (float*)calloc((size_t)ck * qkvd, sizeof(float));
    x->conv_head[li] = 0;
  }
  float* hist = x->conv[li];
  memcpy(hist + (size_t)x->conv_head[li] * qkvd, x->qkv, qkvd * sizeof(float));
  x->conv_head[li] = (x->conv_head[li] + 1) % ck;
  memset(x->cout, 0, qkvd * sizeof(float));
  for (int t = 0; t < ck; ++t) {
    const float* hr = hist + (size_t)((x->conv_head[li] + t) % ck) * qkvd;
    const float* wt = l->conv_w_t + (size_t)t * qkvd;
    size_t i = 0;
    for (; i + 8 <= qkvd; i += 8)
      _mm256_storeu_ps(x->cout + i, _mm256_fmadd_ps(_mm256_loadu_ps(hr + i), _mm256_loadu_ps(wt + i), _mm256_loadu_ps(x->cout + i)));
    for (; i < qkvd; ++i) x->cout[i] += hr[i] * wt[i];
  }
  silu_inplace(x->cout, qkvd);
  memcpy(x->q, x->cout, kdim * 4);
  memcpy(x->k, x->cout + kdim, kdim * 4);
  memcpy(x->v, x->cout + 2 * kdim, inner * 4);
  for (int hh = 0; hh < nkh; ++hh) {
    or_l2norm_inplace(x->q + (size_t)hh * hd, (size_t)hd, 1e-6f);
    or_l2norm_inplace(x->k + (size_t)hh * hd, (size_t)hd, 1e-6f);
  }
  scale_inplace(x->q, kdim, 1.0f / sqrtf((float)hd));
  float* st = x->ssm[li];
  for (int vh = 0; vh < nvh; ++vh) {
    int kh = vh % nkh; /* tiled k-head -> v-head mapping (ssm.rs:558-561) */
    or_ssm_scan_vhead(st + (size_t)vh * hd * hd, x->y + (size_t)vh * hd, x->q + (size_t)kh * hd, x->k + (size_t)kh * hd,
                      x->v + (size_t)vh * hd, l->ssm_a[vh], x->al[vh], x->be[vh], l->dt_bias[vh], hd);
  }
  silu_inplace(x->z, inner);
  ssm_output_gate(x->y, x->z, l->ssm_norm, nvh, hd, 1e-6f);
  mv(x, &l->out, x->y, h, 1);
}

/* model/attention.rs:56-208 attention_forward_into */
static void attn_forward(or_ctx* x, int li, float* h) {
  const dz_config* c = &x->m->cfg;
  or_layer* l = &x->m->L[li];
  int hd = c->head_dim, nq = c->n_head, nkv = c->n_head_kv, grp = nq / nkv;
  or_rmsnorm_into(h, x->normed, l->attn_norm, (size_t)c->hidden, c->rms_eps);
  mv(x, &l->wq, x->normed, x->qt, 0);
  mv(x, &l->wk, x->normed, x->ak, 0);
  mv(x, &l->wv, x->normed, x->av, 0);
  for (int hh = 0; hh < nq; ++hh) {
    memcpy(x->aq + (size_t)hh * hd, x->qt + (size_t)hh * 2 * hd, (size_t)hd * 4);
    memcpy(x->ag + (size_t)hh * hd, x->qt + (size_t)hh * 2 * hd + hd, (size_t)hd * 4);
  }
  for (int hh = 0; hh < nq; ++hh) {
    float* qh = x->aq + (size_t)hh * hd;
    or_rmsnorm_into(qh, qh, l->q_norm, (size_t)hd, c->rms_eps);
    or_rope_partial(qh, c->rope_dim, x->co, x->si);
  }
  scale_inplace(x->aq, (size_t)nq * hd, 1.0f / sqrtf((float)hd));
  for (int hh = 0; hh < nkv; ++hh) {
    float* kh = x->ak + (size_t)hh * hd;
    or_rmsnorm_into(kh, kh, l->k_norm, (size_t)hd, c->rms_eps);
    or_rope_partial(kh, c->rope_dim, x->co, x->si);
  }
  /* KvCache::append (kv_cache.rs:79-88) */
  int len = x->kv_len[li];
  size_t cap = (size_t)c->max_ctx;
  for (int kv = 0; kv < nkv; ++kv) {
    memcpy(x->kk[li] + ((size_t)kv * cap + (size_t)len) * hd, x->ak + (size_t)kv * hd, (size_t)hd * 4);
    memcpy(x->vv[li] + ((size_t)kv * cap + (size_t)len) * hd, x->av + (size_t)kv * hd, (size_t)hd * 4);
  }
  x->kv_len[li] = len + 1;
  int n_cached = len + 1;
  float* outb = (float*)malloc((size_t)grp * hd * sizeof(float));
  float mm[16], ss[16];
  for (int kv = 0; kv < nkv; ++kv) {
    for (int g = 0; g < grp; ++g) { mm[g] = -INFINITY; ss[g] = 0.0f; }
    memset(outb, 0, (size_t)grp * hd * sizeof(float));
    const float* kb = x->kk[li] + (size_t)kv * cap * hd;
    const float* vb = x->vv[li] + (size_t)kv * cap * hd;
    for (int p = 0; p < n_cached; ++p) {
      const float* kp = kb + (size_t)p * hd;
      const float* vp = vb + (size_t)p * hd;
      for (int g = 0; g < grp; ++g) {
        int qh = kv * grp + g; /* grouped GQA mapping (attention.rs:163-165) */
        float score = dot_avx2(x->aq + (size_t)qh * hd, kp, hd);
        float mo = mm[g];
        float mn = fmaxf(mo, score);
        float al = or_exp_fast(mo - mn);
        float bt = or_exp_fast(score - mn);
        ss[g] = ss[g] * al + bt;
        online_v_update(outb + (size_t)g * hd, al, bt, vp, hd);
        mm[g] = mn;
      }
    }
    for (int g = 0; g < grp; ++g) {
      int qh = kv * grp + g;
      float inv = 1.0f / ss[g];
      const float* src = outb + (size_t)g * hd;
      float* dst = x->ao + (size_t)qh * hd;
      int i = 0;
      __m256 iv = _mm256_set1_ps(inv);
      for (; i + 8 <= hd; i += 8) _mm256_storeu_ps(dst + i, _mm256_mul_ps(iv, _mm256_loadu_ps(src + i)));
      for (; i < hd; ++i) dst[i] = src[i] * inv;
    }
  }
  free(outb);
  sigmoid_inplace(x->ag, (size_t)nq * hd);
  mul_inplace(x->ao, x->ag, (size_t)nq * hd);
  mv(x, &l->wo, x->ao, h, 1);
}

/* model/mlp.rs:28-47 */
static void mlp_forward(or_ctx* x, int li, float* h) {
  const dz_config* c = &x->m->cfg;
  or_layer* l = &x->m->L[li];
  or_rmsnorm_into(h, x->normed, l->post_norm, (size_t)c->hidden, c->rms_eps);
  mv(x, &l->gate, x->normed, x->mg, 0);
  mv(x, &l->up, x->normed, x->mu, 0);
  or_swiglu(x->mg, x->mu, (size_t)c->ffn);
  mv(x, &l->down, x->mg, h, 1);
}

void or_mixer_step(or_ctx* x, int li, float* h) {
  or_rope_cos_sin(x->pos, x->m->freqs, x->m->cfg.rope_dim, x->co, x->si);
  if (x->m->L[li].is_attn) attn_forward(x, li, h);
  else ssm_forward(x, li, h);
  x->pos += 1; /* the step consumed one position (its KV entry / conv slot) */
}

/* forward.rs:212 token embedding row.  An F16 token_embd converts element-wise with f16_to_f32
 * (Tensor::to_f32, tensor/tensor.rs:68-80); a Q1_0 one is dequantize_q1_0_row_into. */
void or_model_embd_row(or_model* m, uint32_t token, float* out) {
  size_t H = (size_t)m->cfg.hidden;
  if (m->cfg.embd_f16) {
    uint16_t* row = (uint16_t*)malloc(H * 2);
    dz_synth_embd_row_f16(m->embd_key, token, H, row);
    for (size_t i = 0; i < H; ++i) out[i] = or_f16_to_f32(row[i]);
    free(row);
  } else {
    or_dequant_row(m->embd_q.q, token, H, out);
  }
}

/* model/forward.rs:204-375 forward_single_token */
int or_forward_token(or_ctx* x, uint32_t token, float* logits) {
  or_model* m = x->m;
  const dz_config* c = &m->cfg;
  size_t H = (size_t)c->hidden;
  or_model_embd_row(m, token, x->h);
  or_rope_cos_sin(x->pos, m->freqs, c->rope_dim, x->co, x->si);
  for (int li = 0; li < c->n_layers; ++li) {
    if (m->L[li].is_attn) attn_forward(x, li, x->h);
    else ssm_forward(x, li, x->h);
    mlp_forward(x, li, x->h);
  }
  or_rmsnorm_into(x->h, x->h, m->output_norm, H, c->rms_eps);
  mv(x, &m->output, x->h, x->logits, 0);
  x->pos += 1;
  if (logits) memcpy(logits, x->logits, (size_t)c->vocab * 4);
  return or_argmax(x->logits, (size_t)c->vocab);
}

void or_set_ssm_state(or_ctx* x, int li, const float* state, const float* conv_hist, int conv_head) {
  const dz_config* c = &x->m->cfg;
  size_t hd = (size_t)c->ssm_state;
  size_t qkvd = (size_t)(2 * c->ssm_k_heads + c->ssm_v_heads) * hd;
  memcpy(x->ssm[li], state, (size_t)c->ssm_v_heads * hd * hd * 4);
  if (!x->conv[li]) x->conv[li] = (float*)calloc((size_t)c->ssm_conv_kernel * qkvd, sizeof(float));
  memcpy(x->conv[li], conv_hist, (size_t)c->ssm_conv_kernel * qkvd * 4);
  x->conv_head[li] = conv_head;
}

void or_get_ssm_state(or_ctx* x, int li, float* state, float* conv_hist, int* conv_head) {
  const dz_config* c = &x->m->cfg;
  size_t hd = (size_t)c->ssm_state;
  size_t qkvd = (size_t)(2 * c->ssm_k_heads + c->ssm_v_heads) * hd;
  memcpy(state, x->ssm[li], (size_t)c->ssm_v_heads * hd * hd * 4);
  if (x->conv[li]) memcpy(conv_hist, x->conv[li], (size_t)c->ssm_conv_kernel * qkvd * 4);
  else memset(conv_hist, 0, (size_t)c->ssm_conv_kernel * qkvd * 4);
  *conv_head = x->conv_head[li];
}

void or_set_kv(or_ctx* x, int li, const float* k, const float* v, int len) {
  const dz_config* c = &x->m->cfg;
  size_t hd = (size_t)c->head_dim, cap = (size_t)c->max_ctx;
  for (int kv = 0; kv < c->n_head_kv; ++kv) {
    memcpy(x->kk[li] + (size_t)kv * cap * hd, k + (size_t)kv * len * hd, (size_t)len * hd * 4);
    memcpy(x->vv[li] + (size_t)kv * cap * hd, v + (size_t)kv * len * hd, (size_t)len * hd * 4);
  }
  x->kv_len[li] = len;
}

int or_kv_len(or_ctx* x, int li) { return x->kv_len[li]; }

void or_get_kv(or_ctx* x, int li, float* k, float* v, int len) {
  const dz_config* c = &x->m->cfg;
  size_t hd = (size_t)c->head_dim, cap = (size_t)c->max_ctx;
  for (int kv = 0; kv < c->n_head_kv; ++kv) {
    memcpy(k + (size_t)kv * len * hd, x->kk[li] + (size_t)kv * cap * hd, (size_t)len * hd * 4);
    memcpy(v + (size_t)kv * len * hd, x->vv[li] + (size_t)kv * cap * hd, (size_t)len * hd * 4);
  }
}

/* ------------------------------------------------------------------ synthetic inputs (daiza_synth.h) */
void or_synth_q1_0_rows(uint64_t seed, int kind, int layer, uint64_t cols, uint64_t r0, uint64_t r1, uint8_t* out) {
  dz_synth_q1_0_rows(dz_key(seed, (uint32_t)kind, (uint32_t)layer), cols, r0, r1, out);
}
void or_synth_normal_f32(uint64_t seed, int kind, int layer, uint64_t i0, uint64_t n, double mean, double sigma, float* out) {
  dz_synth_normal_f32(dz_key(seed, (uint32_t)kind, (uint32_t)layer), i0, n, mean, sigma, out);
}
uint16_t or_f32_to_f16(float v) { return dz_f32_to_f16(v); }
void or_synth_embd_row_f16(uint64_t seed, uint32_t token, uint64_t hidden, uint16_t* out) {
  dz_synth_embd_row_f16(dz_key(seed, DZ_K_EMBD, (uint32_t)-1), token, hidden, out);
}

/* ---- SipHash (Aumasson and Bernstein, "SipHash: a fast short-input PRF", 2012) ----
 * c compression rounds per 8-byte word, d finalisation rounds; little-endian words; the last word
 * carries the message length mod 256 in its top byte.  SipHash-2-4 is the published function (pinned
 * by its test vectors); the reference's cfg_hash (Daiza-runtime/src/session_persist.rs:52-66) is
 * Rust's DefaultHasher, SipHash-1-3 with keys 0 and 0, over ten usize fields as 8-byte LE words. */
static uint64_t or_rotl(uint64_t x, int b) { return (x << b) | (x >> (64 - b)); }
#define OR_SIPROUND                                                                  \
  do {                                                                               \
    v0 += v1; v1 = or_rotl(v1, 13); v1 ^= v0; v0 = or_rotl(v0, 32);                  \
    v2 += v3; v3 = or_rotl(v3, 16); v3 ^= v2;                                        \
    v0 += v3; v3 = or_rotl(v3, 21); v3 ^= v0;                                        \
    v2 += v1; v1 = or_rotl(v1, 17); v1 ^= v2; v2 = or_rotl(v2, 32);                  \
  } while (0)
uint64_t or_siphash(int c, int d, uint64_t k0, uint64_t k1, const uint8_t* m, size_t n) {
  uint64_t v0 = 0x736f6d6570736575ull ^ k0, v1 = 0x646f72616e646f6dull ^ k1;
  uint64_t v2 = 0x6c7967656e657261ull ^ k0, v3 = 0x7465646279746573ull ^ k1;
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t w = 0;
    for (int b = 0; b < 8; ++b) w |= (uint64_t)m[i + b] << (8 * b);
    v3 ^= w;
    for (int r = 0; r < c; ++r) OR_SIPROUND;
    v0 ^= w;
  }
  uint64_t w = ((uint64_t)n & 0xFF) << 56;
  for (int b = 0; i + b < n; ++b) w |= (uint64_t)m[i + b] << (8 * b);
  v3 ^= w;
  for (int r = 0; r < c; ++r) OR_SIPROUND;
  v0 ^= w;
  v2 ^= 0xFF;
  for (int r = 0; r < d; ++r) OR_SIPROUND;
  return v0 ^ v1 ^ v2 ^ v3;
}
