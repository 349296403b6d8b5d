// q1_gemm.h — the N-column Q1_0 product Y[n][rows] (=|+=) X[n][cols] · Wᵀ on gfx950's matrix
// cores, for prefill and speculative verify: matvec_batch_into_slice / matvec_add_batch_into_slice
// (Daiza-engine/src/model/weights.rs:475-682, 976-980) and the batched GEMM it dispatches to
// (tensor/gemm.rs:336-439).
//
// Numerics.  A weight is ±scale with scale an f16 value, so it is exact as an f16 matrix-core
// operand (f16 subnormal scales included).  Each token's activations are divided by a power of two
// sig (exact) that puts their largest magnitude in [2^13, 2^14), and split into three f16 values
// hi = f16(v), mid = f16(v - hi), lo = f16(v - hi - mid) (v = x/sig; each difference is exact in
// f32): 33 significant bits, so hi + mid + lo = v exactly for every f32 activation whose residuals
// stay in f16's normal range (those below max|x| · 2^-24 lose bits only beneath f32's own precision
// relative to the row's largest term).  The products of the f16 operands are exact in the f32
// accumulator, so y = sig·(W·hi + W·mid + W·lo) carries the activations at f32 width and differs
// from an f32 dot product only by the f32 accumulation order (the reference's GEMM reorders its
// sums too, gemm.rs:153-225).
//
// Layout.  The weights stay in the GEMV layout (common.h): unit (row-block rb, tile t) holds 64
// rows × 512 columns, each row's 64 sign bytes as four 16-byte chunks, chunk c of row L holding
// group (L >> 4) ^ c with its bytes permuted by position ^ L.  A workgroup owns RB row-blocks
// RB·blockIdx.x .. +RB-1 (RB = 4: two waves each, taking two 16-row blocks; RB = 8, the wide form
// only: one wave each, taking all four) and walks the tiles; in a 16-row block sb of a unit, lane (r, q)
// (r = lane & 15, q = lane >> 4) takes the chunk of row 16·sb + r that holds group q, restores the
// byte order in registers, and feeds the 32 sign bits of dword j of that group as the A operands
// of steps 4j .. 4j+3 of v_mfma_f32_16x16x32_f16 (columns 128q + 32j .. +31).  The B operand, token
// (lane & 15)'s activations at the same columns, is read from a tile staged in LDS.
//
// Column order inside a 32-column block.  Step 4j + s' takes the sign bits 15 - k and 31 - k of
// dword j, k = 4s' + p for its f16 pairs p = 0..3, so that one shift of the whole dword serves a
// pair: ((w << k) & 0x80008000).  The staged activations follow the same order: the 16-byte slot
// s' of a 32-column block holds, as f16 elements 2p and 2p + 1, the columns 15 - 4s' - p and
// 31 - 4s' - p of the block (pack_slot).  The order is a permutation of the K sum only.
#pragma once
#include "common.h"

namespace dz {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kGemmNB = 2;                     // 16-token column blocks per workgroup (wide form)
constexpr int kGemmTok = 16 * kGemmNB;         // tokens per workgroup of the wide form, the padding of n
constexpr int kGemmRowPad = 2 * kTileCols + 16;  // LDS bytes per staged token row (16 B pad: no bank conflicts)
constexpr int kGemmParts = 3;                  // hi, mid and lo f16 parts of every activation
// Waves per workgroup: the workgroup owns 4 row-blocks, and two waves share a row-block, each taking
// two of its four 16-row blocks, so the per-tile chain of a wave (operand expansion and matrix
// instructions) is half as long and the packing of the activations is shared by twice as many waves.
__host__ __device__ constexpr int gemm_waves(int) { return 8; }
// LDS of a workgroup: the hi, mid and lo tiles of NB token blocks (two buffers of them for NB = 1);
// the paired form (hl) stages one tile of eight tokens per buffer as 32 rows: hi 0..7, mid 8..15,
// lo 16..23 (rows 24..31 are read as the unused columns 8..15 of the lo operand).
__host__ __device__ constexpr size_t gemm_buf(int nb, bool hl) {
  return hl ? (size_t)2 * 16 * kGemmRowPad : (size_t)kGemmParts * 16 * nb * kGemmRowPad;
}
__host__ __device__ constexpr size_t gemm_shmem(int nb, bool hl = false) {
  return (size_t)(nb == 1 ? 2 : 1) * gemm_buf(nb, hl);
}

// Activations packed for the matrix cores.
struct GemmX {
  const uint16_t* xh;  // [Np][Kp] f16 bits of v = x/sig
  const uint16_t* xm;  // [Np][Kp] f16 bits of v - hi
  const uint16_t* xl;  // [Np][Kp] f16 bits of v - hi - mid
  const float* sig;    // [Np] power-of-two scale of each token
  int64_t Kp;          // columns padded to the tile (ntiles * 512)
  // raw form (q1_gemm_kernel<NB, true>): x[n][K] f32 with row stride ldx, packed per tile in LDS
  const float* xf;
  int64_t ldx, K;
  // raw form with RMSNorm (rmsnorm_into, rmsnorm.rs:17-200): the tiles are packed from x·nw, the
  // sums of squares of x gathered on the way, and y = inv · W (x·nw) with inv = 1/sqrt(ss/K + eps):
  // by the kernel itself when it sees every tile, else by the consumer of the split partials, from
  // the per-split sums ssq[z][ssq_ld] that the workgroups of row-block group 0 write
  const float* nw;
  float* ssq;
  int ssq_ld;
  float eps;
};

// The power of two that brings max|x| into [2^13, 2^14) (1 for an all-zero or non-finite row).
__device__ __forceinline__ float pack_sig(float amax) {
  if (!(amax > 0.f) || !(amax <= 3.0e38f)) return 1.0f;
  int e;
  (void)frexpf(amax, &e);  // amax = f * 2^e, f in [0.5, 1)
  return ldexpf(1.0f, e - 14 < -100 ? -100 : e - 14);
}

// max(|v.x|, |v.y|, |v.z|, |v.w|) over the 64 lanes of the wave, in every lane: the 16 lanes of each
// DPP row (xor 1, xor 2, half-row mirror, row mirror), then the four rows' lanes 0, 16, 32, 48.
__device__ __forceinline__ float wave_max_abs4(float4 v) {
  float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0xB1, 0xF, 0xF, false)));
  m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0x4E, 0xF, 0xF, false)));
  m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0x141, 0xF, 0xF, false)));
  m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0x140, 0xF, 0xF, false)));
  const int mi = __builtin_bit_cast(int, m);
  const float m0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(mi, 0));
  const float m1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(mi, 16));
  const float m2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(mi, 32));
  const float m3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(mi, 48));
  return fmaxf(fmaxf(m0, m1), fmaxf(m2, m3));
}

// v.x² + v.y² + v.z² + v.w² summed over the 64 lanes of the wave, in every lane, in a fixed order
// (the DPP row sums as in wave_max_abs4, then rows 0..3).
__device__ __forceinline__ float wave_sumsq4(float4 v) {
  float q = v.x * v.x;
  q = __builtin_fmaf(v.y, v.y, q);
  q = __builtin_fmaf(v.z, v.z, q);
  q = __builtin_fmaf(v.w, v.w, q);
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0xB1, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x4E, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x141, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x140, 0xF, 0xF, false));
  const int qi = __builtin_bit_cast(int, q);
  const float q0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 0));
  const float q1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 16));
  const float q2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 32));
  const float q3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 48));
  return (q0 + q1) + (q2 + q3);
}

// The exponent e of the power of two sig = 2^e that pack_sig returns (0 for an all-zero or
// non-finite row): x / sig = ldexp(x, -e), exact.
__device__ __forceinline__ int pack_exp(float amax) {
  if (!(amax > 0.f) || !(amax <= 3.0e38f)) return 0;
  int e;
  (void)frexpf(amax, &e);
  return e - 14 < -100 ? -100 : e - 14;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Eight values of a 32-column block, already divided by the token's power of two — a = columns
// 4m .. 4m+3 and b = columns 16+4m .. 16+4m+3 (m = 0..3) — split into f16 hi, mid and lo (round to
// nearest even; the residuals v - hi and v - hi - mid are exact in f32) and laid out as the block's
// 16-byte B-operand slot 3 - m: dword p = {a[3-p], b[3-p]} (columns 15 - 4s' - p and 31 - 4s' - p
// of slot s' = 3 - m).
__device__ __forceinline__ void pack_slot(float4 a, float4 b, u32x4& h, u32x4& md, u32x4& l) {
  const f32x2 p[4] = {{a.w, b.w}, {a.z, b.z}, {a.y, b.y}, {a.x, b.x}};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 hi = __builtin_convertvector(p[i], f16x2);
    const f32x2 r1 = p[i] - __builtin_convertvector(hi, f32x2);
    const f16x2 mi = __builtin_convertvector(r1, f16x2);
    const f16x2 lo = __builtin_convertvector(r1 - __builtin_convertvector(mi, f32x2), f16x2);
    h[i] = __builtin_bit_cast(unsigned, hi);
    md[i] = __builtin_bit_cast(unsigned, mi);
    l[i] = __builtin_bit_cast(unsigned, lo);
  }
}

// max |v| over the 8 values of every lane of the wave, in every lane (as wave_max_abs4).
__device__ __forceinline__ float wave_max_abs8(float4 a, float4 b) {
  const float4 m = make_float4(fmaxf(fabsf(a.x), fabsf(b.x)), fmaxf(fabsf(a.y), fabsf(b.y)), fmaxf(fabsf(a.z), fabsf(b.z)),
                               fmaxf(fabsf(a.w), fabsf(b.w)));
  return wave_max_abs4(m);
}

// Sum of the squares over the wave of a lane partial q (in every lane, in a fixed order).
__device__ __forceinline__ float wave_sum_lanes(float q) {
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0xB1, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x4E, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x141, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x140, 0xF, 0xF, false));
  const int qi = __builtin_bit_cast(int, q);
  const float q0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 0));
  const float q1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 16));
  const float q2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 32));
  const float q3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 48));
  return (q0 + q1) + (q2 + q3);
}

// Sum of the squares of the 16 values of every lane over the wave, in every lane, in a fixed order.
__device__ __forceinline__ float wave_sumsq16(float4 a, float4 b, float4 c, float4 d) {
  float q = a.x * a.x;
  const float4 v[4] = {a, b, c, d};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (k > 0) q = __builtin_fmaf(v[k].x, v[k].x, q);
    q = __builtin_fmaf(v[k].y, v[k].y, q);
    q = __builtin_fmaf(v[k].z, v[k].z, q);
    q = __builtin_fmaf(v[k].w, v[k].w, q);
  }
  return wave_sum_lanes(q);
}

// Sum of the squares of the 8 values of every lane over the wave, in every lane, in a fixed order.
__device__ __forceinline__ float wave_sumsq8(float4 a, float4 b) {
  float q = a.x * a.x;
  q = __builtin_fmaf(a.y, a.y, q);
  q = __builtin_fmaf(a.z, a.z, q);
  q = __builtin_fmaf(a.w, a.w, q);
  q = __builtin_fmaf(b.x, b.x, q);
  q = __builtin_fmaf(b.y, b.y, q);
  q = __builtin_fmaf(b.z, b.z, q);
  q = __builtin_fmaf(b.w, b.w, q);
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0xB1, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x4E, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x141, 0xF, 0xF, false));
  q += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, q), 0x140, 0xF, 0xF, false));
  const int qi = __builtin_bit_cast(int, q);
  const float q0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 0));
  const float q1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 16));
  const float q2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 32));
  const float q3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(qi, 48));
  return (q0 + q1) + (q2 + q3);
}

// One workgroup (256 threads) per token row n < Np: x[n][0..K) -> xh/xm/xl[n][0..Kp), sig[n]; rows
// n >= n_tok and columns k >= K are zero.  When w is given the row is first RMS-normalised with
// weight w (rmsnorm_into, Daiza-engine/src/math/rmsnorm.rs:17-200: x·(1/sqrt(ss/K + eps))·w).
// One pass gathers Σx² and max|x·w| (the norm's scale is positive, so the normalised row's
// maximum is the scale times that), the second writes.  K is a multiple of 4 (of 128 for Q1_0).
__global__ __launch_bounds__(256) void x_pack_kernel(const float* __restrict__ x, int64_t ldx, int64_t K, int n_tok,
                                                     const float* __restrict__ w, float eps, uint16_t* __restrict__ xh,
                                                     uint16_t* __restrict__ xm, uint16_t* __restrict__ xl,
                                                     float* __restrict__ sig, int64_t Kp) {
  __shared__ float red[8];
  const int n = blockIdx.x;
  const unsigned tid = threadIdx.x;
  const bool live = n < n_tok;
  const float4* row = reinterpret_cast<const float4*>(x + (size_t)(live ? n : 0) * ldx);
  const float4* w4 = reinterpret_cast<const float4*>(w);
  const int64_t K4 = live ? K / 4 : 0;
  float ss = 0.f, amax = 0.f;
  for (int64_t k = tid; k < K4; k += 256) {
    const float4 v = row[k];
    ss = __builtin_fmaf(v.x, v.x, ss);
    ss = __builtin_fmaf(v.y, v.y, ss);
    ss = __builtin_fmaf(v.z, v.z, ss);
    ss = __builtin_fmaf(v.w, v.w, ss);
    const float4 u = w ? make_float4(v.x * w4[k].x, v.y * w4[k].y, v.z * w4[k].z, v.w * w4[k].w) : v;
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
  }
  for (int o = 32; o > 0; o >>= 1) {
    ss += __shfl_xor(ss, o);
    amax = fmaxf(amax, __shfl_xor(amax, o));
  }
  if ((tid & 63u) == 0) {
    red[tid >> 6] = ss;
    red[4 + (tid >> 6)] = amax;
  }
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  amax = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
  const float inv = w ? 1.0f / sqrtf(ss / (float)K + eps) : 1.0f;
  const float s = live ? pack_sig(amax * inv) : 1.0f;
  const float rs = 1.0f / s;  // exact: s is a power of two
  u32x4* oh = reinterpret_cast<u32x4*>(xh + (size_t)n * Kp);
  u32x4* om = reinterpret_cast<u32x4*>(xm + (size_t)n * Kp);
  u32x4* ol = reinterpret_cast<u32x4*>(xl + (size_t)n * Kp);
  // slot k8 = 4J + m of the row: the float4 pair at columns 32J + 4m and 32J + 16 + 4m, written as
  // slot 3 - m of block J (pack_slot); K is a multiple of 128, so a pair is wholly in or out
  auto scaled = [&](int64_t k) {
    const float4 v = row[k];
    float4 u = v;
    if (w) u = make_float4((v.x * inv) * w4[k].x, (v.y * inv) * w4[k].y, (v.z * inv) * w4[k].z, (v.w * inv) * w4[k].w);
    return make_float4(u.x * rs, u.y * rs, u.z * rs, u.w * rs);
  };
  for (int64_t k8 = tid; k8 < Kp / 8; k8 += 256) {
    const int64_t J = k8 >> 2, m = k8 & 3, ka = 8 * J + m;
    u32x4 h = {0u, 0u, 0u, 0u}, md = h, l = h;
    if (ka < K4) pack_slot(scaled(ka), scaled(ka + 4), h, md, l);
    oh[4 * J + 3 - m] = h;
    om[4 * J + 3 - m] = md;
    ol[4 * J + 3 - m] = l;
  }
  if (tid == 0) sig[n] = live ? s : 0.f;
}

// Step S's eight f16 operand values from dword j = S >> 2 of a restored chunk (32 sign bits in
// column order): pair p takes bits 15 - k and 31 - k, k = 4·(S & 3) + p, to the sign positions 15
// and 31 with one shift; an element is +scale where its bit is set, else -scale.  s2x is the
// scale's f16 bits in both halves with both sign bits flipped, so a pair costs a shift and one
// and-xor: ((w << k) & 0x80008000) ^ s2x (no shift for k = 0).
template <int S>
__device__ __forceinline__ f16x8 expand_signs(const unsigned (&wn)[4], unsigned s2x) {
  const unsigned w = wn[S >> 2];
  unsigned d[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) d[p] = ((w << (4 * (S & 3) + p)) & 0x80008000u) ^ s2x;
  u32x4 v = {d[0], d[1], d[2], d[3]};
  return __builtin_bit_cast(f16x8, v);
}

// v_cndmask_b32 with a constant lane mask: mask bit of this lane set ? b : a.
template <unsigned long long M>
__device__ __forceinline__ unsigned lane_select(unsigned a, unsigned b) {
  unsigned d;
  asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "s"(M));
  return d;
}

// Chunk of row L = 16·sb + r holding group q, bytes restored to position order: stored byte i holds
// position i ^ r, so within each dword the bytes move by r & 3 (one v_perm with the lane's
// selector sel), and the dwords by r >> 2, in two stages of lane selects whose masks are constants
// (bits 2 and 3 of the lane index are those of r).  s2x: see expand_signs.
__device__ __forceinline__ void restore_chunk(const u32x4 v, unsigned sc_bits, unsigned sel, unsigned (&wn)[4],
                                              unsigned& s2x) {
  unsigned u[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) u[k] = __builtin_amdgcn_perm(v[k], v[k], sel);
  unsigned t[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) t[k] = lane_select<0xF0F0F0F0F0F0F0F0ull>(u[k], u[k ^ 1]);
#pragma unroll
  for (int k = 0; k < 4; ++k) wn[k] = lane_select<0xFF00FF00FF00FF00ull>(t[k], t[k ^ 2]);
  s2x = ((sc_bits & 0xFFFFu) * 0x00010001u) ^ 0x80008000u;
}

// Grid (ceil(nrb / RB), Np / (16·NB), splits), 64·gemm_waves(NB) threads, gemm_shmem(NB, HL) bytes of
// LDS.  Workgroup z of a split product takes K tiles [z·tps, min(ntiles, (z+1)·tps)) and writes its
// partial to y + z·zstride; an unsplit product (gridDim.z = 1) writes
// y[n][row] = (accumulate ? y : 0) + sig[n] · Σ_k W[row][k] (xh + xm + xl)[n][k] for n < n_tok,
// row < rows.
//
// Raw form (RAW): the workgroup reads x[n][K] as f32 and packs each tile itself, with a power of two
// sig(n, t) per token and tile (max |x| of the tile's 512 columns in [2^13, 2^14), as pack_sig); a
// tile's products are scaled by it as they are added: y = Σ_t sig(n, t) · W_t (hi + mid + lo)(n, t).
// That skips the separate packing pass for inputs that need no RMSNorm.
//
// Paired form (HL, raw form with n ≤ 8 tokens): one B operand carries two parts, columns 0..7 the
// hi rows and columns 8..15 the mid rows of the eight tokens, and a second the lo rows in columns
// 0..7, so each (step, block) takes two matrix instructions instead of three; lanes r and r + 8 of
// the first D layout hold the hi and mid sums of token r & 7, lane r of the second its lo sum (all
// scaled by that token's sig(n, t)), added once after the last tile.
template <int NB, bool RAW = false, bool HL = false, int RB = 4>
__global__ __launch_bounds__(64 * gemm_waves(NB), NB == 1 ? 4 : (RB == 4 ? 2 : 1)) void q1_gemm_kernel(const uint8_t* __restrict__ W, int64_t rows, int64_t nrb,
                                                         int ntiles, int tps, const GemmX x, int n_tok,
                                                         float* __restrict__ y, int64_t ldy, int64_t zstride,
                                                         int accumulate) {
  static_assert(!HL || (NB == 1 && RAW), "the paired form is a raw form of one token block");
  constexpr int TOK = 16 * NB;
  constexpr int NT = 64 * gemm_waves(NB);  // threads
  static_assert(RB == 4 || (RB == 8 && NB > 1), "row-blocks per workgroup: 4, or 8 for the wide form");
  constexpr int HALVES = gemm_waves(NB) / RB;  // waves per row-block
  constexpr int SBW = 4 / HALVES;             // 16-row blocks per wave
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int WV = gemm_waves(NB);
  constexpr int TPW = TOK / WV;        // raw form: token rows packed by each wave
  constexpr size_t BUF = gemm_buf(NB, HL);  // bytes of one activation buffer
  __shared__ float tile_sig[2][TOK];   // raw form: sig(n, t) of each activation buffer
  __shared__ float tok_inv[TOK];       // raw form with RMSNorm: 1/rms of each token (unsplit product)
  float ss_acc[TPW];                   // raw form with RMSNorm: sum of x^2 of the wave's token rows over
#pragma unroll                         // this workgroup's tiles (the same value in every lane)
  for (int jt = 0; jt < TPW; ++jt) ss_acc[jt] = 0.f;
  const unsigned tid = threadIdx.x, lane = tid & 63u;
  const int64_t rb = (int64_t)blockIdx.x * RB + (tid >> 6) / HALVES;
  const int sb0 = (int)((tid >> 6) % HALVES) * SBW;  // first 16-row block of this wave
  const bool live = rb < nrb;
  const int tok0 = (int)blockIdx.y * TOK;
  const unsigned r = lane & 15u, q = lane >> 4;
  const unsigned psel = 0x03020100u ^ (0x01010101u * (r & 3u));  // restore_chunk's byte selector
  const int t_begin = (int)blockIdx.z * tps, t_end = min(ntiles, t_begin + tps);
  y += (size_t)blockIdx.z * zstride;
  if (gridDim.z > 1) accumulate = 0;
  f32x4 acc[SBW][NB];
  f32x4 acc2[HL ? SBW : 1];  // paired form: the lo sums
#pragma unroll
  for (int sb = 0; sb < SBW; ++sb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[sb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sb = 0; sb < (HL ? SBW : 1); ++sb) acc2[sb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Tile t's operands are requested one tile ahead: the wave's unit (four 16-byte chunks and their
  // scale slots) into registers, the activations (hi, mid and lo rows of the TOK tokens) into
  // registers that are written to the other of two LDS buffers after the current tile's products
  // (one buffer when NB > 1).  A tile past the range reloads the last one (never used), so that no
  // loaded value becomes a phi.
  constexpr int NBUF = NB == 1 ? 2 : 1;
  // 16-byte activation chunks per thread and tile: the paired form's wave row (two per lane), the
  // raw form's TPW rows (two per lane each), or the packed form's three parts
  constexpr int XV = HL ? 2 : RAW ? 2 * TPW : kGemmParts * TOK * 64 / NT;
  auto load_unit = [&](int t, u32x4 (&cv)[SBW], unsigned (&cs)[SBW]) {
    const int tc = t < t_end ? t : t_end - 1;
    const uint8_t* unit = W + ((size_t)(live ? rb : 0) * ntiles + tc) * kUnitBytes;
#pragma unroll
    for (int sb = 0; sb < SBW; ++sb) {
      const unsigned L = 16u * (sb0 + sb) + r, c = (unsigned)(sb0 + sb) ^ q;
      cv[sb] = *reinterpret_cast<const u32x4*>(unit + ((size_t)c * 64 + L) * 16);
      const unsigned short* scp = reinterpret_cast<const unsigned short*>(unit + kUnitSignBytes + (size_t)L * 8);
      cs[sb] = scp[c];
    }
  };
  // Raw form: token row n = w + WV·jt of the tile is loaded and packed by wave w alone (its own
  // maxima and sums, no exchange between waves); chunks 2jt and 2jt + 1 of a lane are the float4 at
  // columns 32J + 4m and 32J + 16 + 4m of that row (J = lane >> 2, m = lane & 3): the two halves
  // of the lane's B-operand slot (pack_slot).
  const int64_t xcol = 32 * (lane >> 2) + 4 * (lane & 3u);
  auto load_x = [&](int t, u32x4 (&xv)[XV]) {
    const int tc = t < t_end ? t : t_end - 1;
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      if constexpr (HL) {  // the wave's token row in tile t (zeros past the range)
        const int n = tok0 + (int)(tid >> 6);
        const int64_t col = (int64_t)t * kTileCols + xcol + 16 * (j & 1);
        xv[j] = n < n_tok && t < t_end && col < x.K ? *reinterpret_cast<const u32x4*>(x.xf + (size_t)n * x.ldx + col)
                                                    : u32x4{0u, 0u, 0u, 0u};
      } else if constexpr (RAW) {
        const int n = tok0 + (int)(tid >> 6) + WV * (j >> 1);
        const int64_t col = (int64_t)tc * kTileCols + xcol + 16 * (j & 1);
        xv[j] = n < n_tok && col < x.K ? *reinterpret_cast<const u32x4*>(x.xf + (size_t)n * x.ldx + col)
                                       : u32x4{0u, 0u, 0u, 0u};
      } else {
        const int i = (int)tid + NT * j;
        const int part = i / (TOK * 64), rem = i % (TOK * 64), n = rem >> 6, c = rem & 63;
        const uint16_t* src = part == 0 ? x.xh : part == 1 ? x.xm : x.xl;
        xv[j] = *reinterpret_cast<const u32x4*>(src + (size_t)(tok0 + n) * x.Kp + (size_t)tc * kTileCols + 8 * c);
      }
    }
  };
  auto put_x = [&](int b, u32x4 (&xv)[XV], int t_x) {
    if constexpr (HL) {
      // the wave's token row n of tile t_x: hi in row n, mid in row 8 + n, lo in row 16 + n
      const int n = (int)(tid >> 6);
      if (tok0 + n >= n_tok) return;  // wave-uniform; these product columns are never stored
      float4 v0 = __builtin_bit_cast(float4, xv[0]), v1 = __builtin_bit_cast(float4, xv[1]);
      if (x.nw != nullptr) {
        ss_acc[0] += wave_sumsq8(v0, v1);  // a tile past the range holds zeros
        const int64_t col = (int64_t)t_x * kTileCols + xcol;
        float4 w0 = make_float4(1.f, 1.f, 1.f, 1.f), w1 = w0;
        if (t_x < t_end && col < x.K) {
          w0 = *reinterpret_cast<const float4*>(x.nw + col);
          w1 = *reinterpret_cast<const float4*>(x.nw + col + 16);
        }
        v0 = make_float4(v0.x * w0.x, v0.y * w0.y, v0.z * w0.z, v0.w * w0.w);
        v1 = make_float4(v1.x * w1.x, v1.y * w1.y, v1.z * w1.z, v1.w * w1.w);
      }
      const int e = pack_exp(wave_max_abs8(v0, v1));
      u32x4 h, md, l;
      pack_slot(make_float4(ldexpf(v0.x, -e), ldexpf(v0.y, -e), ldexpf(v0.z, -e), ldexpf(v0.w, -e)),
                make_float4(ldexpf(v1.x, -e), ldexpf(v1.y, -e), ldexpf(v1.z, -e), ldexpf(v1.w, -e)), h, md, l);
      unsigned char* row = smem + (size_t)b * BUF + (size_t)n * kGemmRowPad + 64 * (lane >> 2) + 16 * (3u - (lane & 3u));
      *reinterpret_cast<u32x4*>(row) = h;
      *reinterpret_cast<u32x4*>(row + (size_t)8 * kGemmRowPad) = md;
      *reinterpret_cast<u32x4*>(row + (size_t)16 * kGemmRowPad) = l;
      if (lane == 0) tile_sig[b][n] = ldexpf(1.0f, e);
    } else if constexpr (RAW) {
      // token rows past n_tok are skipped (wave-uniform; their product columns are never stored)
      const unsigned wave = tid >> 6;
      const bool normed = x.nw != nullptr;
      float4 nw0 = make_float4(1.f, 1.f, 1.f, 1.f), nw1 = nw0;
      if (normed) {
        const int64_t col = (int64_t)t_x * kTileCols + xcol;
        if (col < x.K) {  // both halves of a 32-column block lie on the same side of K
          nw0 = *reinterpret_cast<const float4*>(x.nw + col);
          nw1 = *reinterpret_cast<const float4*>(x.nw + col + 16);
        }
      }
#pragma unroll
      for (int jt = 0; jt < TPW; ++jt) {
        const int n = (int)wave + WV * jt;
        if (tok0 + n >= n_tok) continue;
        float4 v0 = __builtin_bit_cast(float4, xv[2 * jt]), v1 = __builtin_bit_cast(float4, xv[2 * jt + 1]);
        if (normed) {
          const float q = wave_sumsq8(v0, v1);
          if (t_x < t_end) ss_acc[jt] += q;
          v0 = make_float4(v0.x * nw0.x, v0.y * nw0.y, v0.z * nw0.z, v0.w * nw0.w);
          v1 = make_float4(v1.x * nw1.x, v1.y * nw1.y, v1.z * nw1.z, v1.w * nw1.w);
        }
        const int e = pack_exp(wave_max_abs8(v0, v1));
        u32x4 h, md, l;
        pack_slot(make_float4(ldexpf(v0.x, -e), ldexpf(v0.y, -e), ldexpf(v0.z, -e), ldexpf(v0.w, -e)),
                  make_float4(ldexpf(v1.x, -e), ldexpf(v1.y, -e), ldexpf(v1.z, -e), ldexpf(v1.w, -e)), h, md, l);
        unsigned char* row = smem + (size_t)b * BUF + (size_t)n * kGemmRowPad + 64 * (lane >> 2) + 16 * (3u - (lane & 3u));
        *reinterpret_cast<u32x4*>(row) = h;
        *reinterpret_cast<u32x4*>(row + (size_t)TOK * kGemmRowPad) = md;
        *reinterpret_cast<u32x4*>(row + (size_t)2 * TOK * kGemmRowPad) = l;
        if (lane == 0) tile_sig[b][n] = ldexpf(1.0f, e);
      }
    } else {
#pragma unroll
      for (int j = 0; j < XV; ++j) {
        const int i = (int)tid + NT * j;
        const int part = i / (TOK * 64), rem = i % (TOK * 64), n = rem >> 6, c = rem & 63;
        *reinterpret_cast<u32x4*>(smem + (size_t)b * BUF + ((size_t)part * TOK + n) * kGemmRowPad + 16 * c) = xv[j];
      }
    }
  };
  u32x4 cv[SBW];
  unsigned cs[SBW];
  u32x4 xv[XV];
  // Tiles are staged one per buffer and barrier; the weights stay one tile ahead.
  constexpr int PT = 1;
  load_unit(t_begin, cv, cs);
  load_x(t_begin, xv);
  put_x(0, xv, t_begin);
  __syncthreads();
  for (int g0 = t_begin; g0 < t_end; g0 += PT) {
    const int g1 = min(t_end, g0 + PT);
    const int b = NBUF == 2 ? ((g0 - t_begin) / PT) & 1 : 0;
    const bool more = g1 < t_end;  // uniform: the activations of a next group are loaded and packed
    if (NBUF == 2 && more) load_x(g1, xv);
    f32x4 at[SBW][NB];  // raw form: this group's products, scaled by sig(n, group) after it
    f32x4 at2[HL ? SBW : 1];
#pragma unroll
    for (int sb = 0; sb < SBW; ++sb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) at[sb][nb] = RAW ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[sb][nb];
#pragma unroll
    for (int sb = 0; sb < (HL ? SBW : 1); ++sb) at2[sb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int t = g0; t < g1; ++t) {
      u32x4 cvn[SBW];
      unsigned csn[SBW];
      load_unit(t + 1, cvn, csn);
      if (live) {
        unsigned wn[SBW][4], s2[SBW];
#pragma unroll
        for (int sb = 0; sb < SBW; ++sb) restore_chunk(cv[sb], cs[sb], psel, wn[sb], s2[sb]);
        // B operand of step s for token block nb: token 16·nb + r, columns 128q + 8s .. +7, of the hi,
        // mid and lo rows (paired form: row r holds hi of token r for r < 8, else mid of token r - 8;
        // row 16 + r holds lo of token r for r < 8)
        const unsigned char* bh = smem + (size_t)b * BUF + (size_t)r * kGemmRowPad + 256u * q;
        const unsigned char* bm = bh + (size_t)(HL ? 16 : TOK) * kGemmRowPad;
        const unsigned char* bl = bh + (size_t)2 * TOK * kGemmRowPad;
#define DZ_GEMM_STEP(S)                                                                               \
  if constexpr (HL) {                                                                                 \
    const f16x8 xb_ = *reinterpret_cast<const f16x8*>(bh + 16 * (S));                                 \
    const f16x8 xc_ = *reinterpret_cast<const f16x8*>(bm + 16 * (S));                                 \
    _Pragma("unroll") for (int sb = 0; sb < SBW; ++sb) {                                              \
      const f16x8 a = expand_signs<S>(wn[sb], s2[sb]);                                                \
      at[sb][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xb_, at[sb][0], 0, 0, 0);                 \
      at2[sb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xc_, at2[sb], 0, 0, 0);                     \
    }                                                                                                 \
  } else {                                                                                            \
    f16x8 xh_[NB], xm_[NB], xl_[NB];                                                                  \
    _Pragma("unroll") for (int nb = 0; nb < NB; ++nb) {                                               \
      xh_[nb] = *reinterpret_cast<const f16x8*>(bh + (size_t)nb * 16 * kGemmRowPad + 16 * (S));       \
      xm_[nb] = *reinterpret_cast<const f16x8*>(bm + (size_t)nb * 16 * kGemmRowPad + 16 * (S));       \
      xl_[nb] = *reinterpret_cast<const f16x8*>(bl + (size_t)nb * 16 * kGemmRowPad + 16 * (S));       \
    }                                                                                                 \
    _Pragma("unroll") for (int sb = 0; sb < SBW; ++sb) {                                              \
      const f16x8 a = expand_signs<S>(wn[sb], s2[sb]);                                                \
      _Pragma("unroll") for (int nb = 0; nb < NB; ++nb) {                                             \
        at[sb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xh_[nb], at[sb][nb], 0, 0, 0);         \
        at[sb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xm_[nb], at[sb][nb], 0, 0, 0);         \
        at[sb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xl_[nb], at[sb][nb], 0, 0, 0);         \
      }                                                                                               \
    }                                                                                                 \
  }
        DZ_GEMM_STEP(0) DZ_GEMM_STEP(1) DZ_GEMM_STEP(2) DZ_GEMM_STEP(3)
        DZ_GEMM_STEP(4) DZ_GEMM_STEP(5) DZ_GEMM_STEP(6) DZ_GEMM_STEP(7)
        DZ_GEMM_STEP(8) DZ_GEMM_STEP(9) DZ_GEMM_STEP(10) DZ_GEMM_STEP(11)
        DZ_GEMM_STEP(12) DZ_GEMM_STEP(13) DZ_GEMM_STEP(14) DZ_GEMM_STEP(15)
#undef DZ_GEMM_STEP
      }
#pragma unroll
      for (int sb = 0; sb < SBW; ++sb) {
        cv[sb] = cvn[sb];
        cs[sb] = csn[sb];
      }
    }
    if (live) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const float sg = RAW ? tile_sig[b][16 * nb + (int)(HL ? r & 7u : r)] : 1.0f;
#pragma unroll
        for (int sb = 0; sb < SBW; ++sb) {
          if constexpr (RAW) {
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[sb][nb][v] = __builtin_fmaf(sg, at[sb][nb][v], acc[sb][nb][v]);
            if constexpr (HL) {
#pragma unroll
              for (int v = 0; v < 4; ++v) acc2[sb][v] = __builtin_fmaf(sg, at2[sb][v], acc2[sb][v]);
            }
          } else {
            acc[sb][nb] = at[sb][nb];
          }
        }
      }
    }
    if (!more) break;  // the epilogue reads no LDS that another wave still writes
    if (NBUF == 2) {
      put_x(b ^ 1, xv, g1);  // the other buffer: its last reads (group before this) finished before the previous barrier
    } else {
      __syncthreads();  // every wave is done with this group's activations
      load_x(g1, xv);
      put_x(0, xv, g1);
    }
    __syncthreads();
  }
  // raw form with RMSNorm: each token's 1/rms (every tile seen) or this split's sums of squares
  if (RAW && x.nw != nullptr) {
#pragma unroll
    for (int jt = 0; jt < TPW; ++jt) {
      const int n = (int)(tid >> 6) + WV * jt;
      if (lane != 0 || tok0 + n >= n_tok) continue;
      if (gridDim.z == 1)
        tok_inv[n] = 1.0f / sqrtf(ss_acc[jt] / (float)x.K + x.eps);
      else if (blockIdx.x == 0)
        x.ssq[(size_t)blockIdx.z * x.ssq_ld + tok0 + n] = ss_acc[jt];
    }
    if (gridDim.z == 1) __syncthreads();
  }
  if (!live) return;
  if constexpr (HL) {  // lane r < 8 adds the mid sums of its token from lane r + 8, then its lo sums
#pragma unroll
    for (int sb = 0; sb < SBW; ++sb)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[sb][0][v] = (acc[sb][0][v] + __shfl_xor(acc[sb][0][v], 8, 16)) + acc2[sb][v];
  }
  // D layout: lane holds rows 4q .. 4q+3 of block sb for token 16·nb + r
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = tok0 + 16 * nb + (int)r;
    if (n >= n_tok || (HL && r >= 8u)) continue;
    const float sg = RAW ? (x.nw != nullptr && gridDim.z == 1 ? tok_inv[16 * nb + (int)r] : 1.0f) : x.sig[n];
    float* yr = y + (size_t)n * ldy;
#pragma unroll
    for (int sb = 0; sb < SBW; ++sb) {
      const int64_t row0 = rb * kRowBlock + 16 * (sb0 + sb) + 4 * (int)q;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t row = row0 + v;
        if (row < rows) {
          const float val = acc[sb][nb][v] * sg;
          yr[row] = accumulate ? yr[row] + val : val;
        }
      }
    }
  }
}

// y[n][row] (=|+=) Σ_z part[z][n][row] for z < splits in order (the partials of a split product),
// times token n's 1/rms when ssq is given (a normed raw product: sums of squares [z][ssq_ld], K).
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float* __restrict__ part, int splits,
                                                                int64_t zstride, int64_t rows, int n_tok,
                                                                float* __restrict__ y, int64_t ldy, int accumulate,
                                                                const float* __restrict__ ssq, int ssq_ld, int64_t K,
                                                                float eps) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int n = blockIdx.y;
  if (row >= rows || n >= n_tok) return;
  const size_t off = (size_t)n * rows + row;
  float v = ordered_sum(part + off, zstride, splits);
  if (ssq) v *= split_inv_rms(ssq, ssq_ld, splits, n, K, eps);
  float* yr = y + (size_t)n * ldy + row;
  *yr = accumulate ? *yr + v : v;
}

}  // namespace dz
