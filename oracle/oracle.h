/*
 * oracle.h — CPU restatement of the reference (guang384/Daiza) batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (daiza_amd/, include/) may link or call
 * this code: it is the checker for the HIP kernels (tests/, __graft_entry__.smoke()) and the
 * CPU baseline timed by bench.py.  The reference is Rust and cannot be built in this image
 * (no rustc/cargo), so each function restates the reference's instruction sequence in C with
 * the same AVX2/FMA/F16C intrinsics and operation order, citing the file:line it follows.
 */
#ifndef DAIZA_ORACLE_H
#define DAIZA_ORACLE_H

#include <stddef.h>
#include <stdint.h>
#include "daiza_hip.h" /* dz_config */

#ifdef __cplusplus
extern "C" {
#endif

/* quant.rs:39-74 */
float or_f16_to_f32(uint16_t bits);
uint32_t or_f16_to_f32_bits(uint16_t bits);
/* quant.rs:86-108 (scalar fallback only; flushes subnormals) */
float or_f16_to_f32_fast(uint16_t bits);
/* quant.rs:161-194 */
void or_dequant_row(const uint8_t* aos, size_t row, size_t cols, float* out);

/* Row kernels.  variant: 4 = quad (quant.rs:614-740), 3 = triple (492-600), 2 = dual (361-490),
 * 1 = single (267-330).  Scalar C with fmaf in the AVX2 lane order: bit-exact with the AVX2 kernels. */
float or_dot_row_scalar(const uint8_t* aos, size_t row, size_t cols, const float* x, int variant);

/* y = W x / y += W x over all rows, with the reference's row grouping (quads, then a triple/dual/
 * single tail) and 128-row work-stealing chunks (weights.rs:123-465, workspace.rs:522-632).
 * nthreads <= 0 means all cores.  AVX2 quad kernel. */
void or_matvec(const uint8_t* aos, size_t rows, size_t cols, const float* x, float* y, int accumulate, int nthreads);
/* same result from the scalar restatement, single thread */
void or_matvec_scalar(const uint8_t* aos, size_t rows, size_t cols, const float* x, float* y, int accumulate);

/* math glue on arrays (n multiple of 8 where the reference has no tail) */
void or_exp_ps(const float* x, float* y, size_t n);      /* simd_exp.rs:44-85 */
void or_sigmoid_ps(const float* x, float* y, size_t n);  /* simd_exp.rs:101-111 */
void or_silu_ps(const float* x, float* y, size_t n);     /* simd_exp.rs:119-123 */
float or_exp_fast(float x);                              /* simd_exp.rs:156-167 */
float or_sigmoid_fast(float x);                          /* simd_exp.rs:140-151 */
void or_rmsnorm_into(const float* x, float* y, const float* w, size_t n, float eps); /* rmsnorm.rs:82-200 */
void or_l2norm_inplace(float* x, size_t n, float eps);   /* ssm.rs:76-135 */
void or_rope_freqs(int rope_dim, float base, float* freqs); /* rope.rs:27-38 */
void or_rope_cos_sin(int pos, const float* freqs, int rope_dim, float* cos_out, float* sin_out); /* rope.rs:82-101 */
void or_rope_partial(float* x, int rope_dim, const float* cos_t, const float* sin_t); /* rope.rs:187-231 */
void or_swiglu(float* gate, const float* up, size_t n);  /* simd_exp.rs:273-296 */
int or_argmax(const float* x, size_t n);                 /* simd_exp.rs:551-598 */
/* one v-head of the gated delta rule, state row-major S[i][j] (ssm.rs:153-180, 378-418) */
void or_ssm_scan_vhead(float* s, float* y, const float* q, const float* k, const float* v, float a_vh,
                       float alpha_vh, float beta_vh, float dt_bias_vh, int head_dim);
/* LcgRng::next_f32 (sampling.rs:9-19); returns the value and advances *state */
float or_lcg_next(uint64_t* state);
/* speculative-verify sampling (math/softmax.rs:15-80, simd_exp.rs:605-767, sampling.rs:144-247,
 * Daiza-runtime/src/engine.rs:1791-1866) */
void or_softmax_inplace(float* x, size_t n);
void or_softmax_pair_single(const float* t, const float* d, size_t n, size_t idx, float* p, float* q);
uint32_t or_sample_top_k_top_p(const float* logits, size_t n, float temperature, int top_k, float top_p, uint64_t* rng);
uint32_t or_sample_bonus(const float* target, const float* draft, size_t n, float temperature, int top_k,
                         float top_p, uint64_t* rng);
int or_leviathan_check(const float* target, const float* draft, size_t n, uint32_t token, float temperature,
                       uint64_t* rng);

/* synthetic inputs of daiza_synth.h, exported for tests */
void or_synth_q1_0_rows(uint64_t seed, int kind, int layer, uint64_t cols, uint64_t r0, uint64_t r1, uint8_t* out);
void or_synth_normal_f32(uint64_t seed, int kind, int layer, uint64_t i0, uint64_t n, double mean, double sigma, float* out);
uint16_t or_f32_to_f16(float v);
void or_synth_embd_row_f16(uint64_t seed, uint32_t token, uint64_t hidden, uint16_t* out);

/* ------------------------------ model ------------------------------ */
typedef struct or_model or_model;
typedef struct or_ctx or_ctx;

/* Synthetic model, same bytes as dz_model_create_synth (daiza_synth.h). */
or_model* or_model_synth(const dz_config* cfg, uint64_t seed, int nthreads);
void or_model_free(or_model* m);
/* AoS bytes of a Q1_0 weight: kind = DZ_K_* of daiza_synth.h, layer = -1 for globals */
const uint8_t* or_model_q1(or_model* m, int kind, int layer, size_t* rows, size_t* cols);
const float* or_model_f32(or_model* m, int kind, int layer, size_t* n);

or_ctx* or_ctx_new(or_model* m);
void or_ctx_free(or_ctx* c);
int or_ctx_pos(or_ctx* c);
void or_ctx_set_pos(or_ctx* c, int pos);
/* KvCache::truncate (kv_cache.rs:119-130) on every attention layer, pos = len; SSM state untouched. */
void or_kv_truncate(or_ctx* c, int len);
/* forward_single_token (forward.rs:204-375); logits may be NULL; returns argmax */
void or_model_embd_row(or_model* m, uint32_t token, float* out);
int or_forward_token(or_ctx* c, uint32_t token, float* logits);
/* h += mixer(rmsnorm(h)) of one layer (ssm_forward_into / attention_forward_into); pos += 1 */
void or_mixer_step(or_ctx* c, int layer, float* h);
void or_set_ssm_state(or_ctx* c, int layer, const float* state, const float* conv_hist, int conv_head);
void or_get_ssm_state(or_ctx* c, int layer, float* state, float* conv_hist, int* conv_head);
void or_set_kv(or_ctx* c, int layer, const float* k, const float* v, int len);
int or_kv_len(or_ctx* c, int layer);
void or_get_kv(or_ctx* c, int layer, float* k, float* v, int len);

/* SipHash with c compression and d finalisation rounds (session_persist.rs:52-66 uses c=1, d=3). */
uint64_t or_siphash(int c, int d, uint64_t k0, uint64_t k1, const uint8_t* m, size_t n);

#ifdef __cplusplus
}
#endif
#endif
