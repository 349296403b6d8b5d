// q1_gemv.h — the Q1_0 GEMV as a sign-byte lookup table in LDS (gfx950).
//
// y_r = sum_g scale_{r,g} * sum_{k in g} (bit ? +x_k : -x_k)   (Daiza-engine/src/tensor/quant.rs:15-17)
//
// A workgroup owns one 512-column K tile at a time.  It writes the table
//   LUT[v][p] = sum_{j<8} (bit j of v ? +x[8p+j] : -x[8p+j])      v = 0..255, p = 0..63
// to LDS (64 KiB), after which one sign byte of weights costs one v_perm (byte -> LDS address),
// one ds_read_b32 and one FMA with the group scale: 8 weights per 2 VALU ops, well under the
// ~0.7 VALU/weight that 8 TB/s of 18-byte blocks allows on 256 CUs.  No MFMA is involved.
//
// Lane L of a wave owns row 64*rb + L.  At step s (0..63) it reads tile position p = L ^ s, so
// within each half-wave the 32 lanes hit 32 distinct LDS banks (bank = p mod 32): conflict free.
// The matrix is stored pre-permuted (see Q1Dev) so that "byte s of my row data" is position L ^ s
// and "scale slot s >> 4" is that position's group; both indices are wave-uniform.
#pragma once
#include "common.h"

namespace dz {

// c[m] byte k = (L ^ (4m + k)) << 2 : LDS byte offset of position L ^ s inside a 256-byte LUT row.
__device__ __forceinline__ void make_pos_consts(unsigned lane, unsigned c[16]) {
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    unsigned v = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) v |= ((lane ^ (4u * m + k)) << 2) << (8 * k);
    c[m] = v;
  }
}

struct UnitRegs {
  u32x4 s[4];  // 64 stored sign bytes of this lane's row
  u32x2 sc;    // 4 f16 scale slots
};

__device__ __forceinline__ void load_unit(const uint8_t* __restrict__ unit, unsigned lane, UnitRegs& r) {
  const u32x4* sp = reinterpret_cast<const u32x4*>(unit);
#pragma unroll
  for (int c = 0; c < 4; ++c) r.s[c] = __builtin_nontemporal_load(sp + c * 64 + lane);
  const u32x2* scp = reinterpret_cast<const u32x2*>(unit + kUnitSignBytes);
  r.sc = __builtin_nontemporal_load(scp + lane);
}

__device__ __forceinline__ float half_lo(unsigned v) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(v & 0xFFFFu)); }
__device__ __forceinline__ float half_hi(unsigned v) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(v >> 16)); }

// Dot product of one lane's 512-weight row slice with the tile whose table sits at LDS address 0
// (kernels using it allocate no static LDS, so their dynamic LDS, the table, starts at address 0
// and a v_perm result is the LDS address itself):
//   a_k = +0;  for m = 0..15:  a_k = fma(scale[m >> 2], LUT[byte k of word m][position], a_k)
//   result = (a0 + a1) + (a2 + a3)
// where word m holds stored bytes 4m..4m+3, byte k's LDS address is v_perm(word, c[m]) (byte0 =
// c[m].byte k, the position offset; byte1 = the sign byte; bytes 2,3 = 0) and scale slot m >> 2
// is the f16 group scale of those positions, converted exactly to f32.
// It is one software-pipelined block: the table reads of word m are issued three words ahead of
// their FMAs (12 reads in flight, within the 4-bit LDS counter), so LDS latency is hidden by the
// wave itself rather than by the compiler's scheduling, which serializes the reads (one in
// flight) when the surrounding kernel is short of registers.  Per sign byte: one v_perm_b32, one
// ds_read_b32, one v_fmac_f32.
#define DZ_Q1_ISSUE(M, T)                                   \
  "v_perm_b32 %[" #T "0], %[w" #M "], %[c" #M "], %[k0]\n" \
  "v_perm_b32 %[" #T "1], %[w" #M "], %[c" #M "], %[k1]\n" \
  "v_perm_b32 %[" #T "2], %[w" #M "], %[c" #M "], %[k2]\n" \
  "v_perm_b32 %[" #T "3], %[w" #M "], %[c" #M "], %[k3]\n" \
  "ds_read_b32 %[" #T "0], %[" #T "0]\n"                   \
  "ds_read_b32 %[" #T "1], %[" #T "1]\n"                   \
  "ds_read_b32 %[" #T "2], %[" #T "2]\n"                   \
  "ds_read_b32 %[" #T "3], %[" #T "3]\n"
#define DZ_Q1_ACC(T, F)                        \
  "v_fmac_f32 %[a0], %[" #F "], %[" #T "0]\n" \
  "v_fmac_f32 %[a1], %[" #F "], %[" #T "1]\n" \
  "v_fmac_f32 %[a2], %[" #F "], %[" #T "2]\n" \
  "v_fmac_f32 %[a3], %[" #F "], %[" #T "3]\n"
#define DZ_Q1_STEP(MA, TA, F, MI, TI) "s_waitcnt lgkmcnt(8)\n" DZ_Q1_ACC(TA, F) DZ_Q1_ISSUE(MI, TI)

__device__ __forceinline__ float unit_dot(const UnitRegs& r, const unsigned c[16]) {
  const float f0 = half_lo(r.sc.x), f1 = half_hi(r.sc.x), f2 = half_lo(r.sc.y), f3 = half_hi(r.sc.y);
  float a0, a1, a2, a3;
  unsigned p0, p1, p2, p3, q0, q1, q2, q3, u0, u1, u2, u3, v0, v1, v2, v3;
  asm volatile(
      "v_mov_b32 %[a0], 0\n"
      "v_mov_b32 %[a1], 0\n"
      "v_mov_b32 %[a2], 0\n"
      "v_mov_b32 %[a3], 0\n"
      DZ_Q1_ISSUE(0, p) DZ_Q1_ISSUE(1, q) DZ_Q1_ISSUE(2, u)
      DZ_Q1_STEP(0, p, f0, 3, v)
      DZ_Q1_STEP(1, q, f0, 4, p)
      DZ_Q1_STEP(2, u, f0, 5, q)
      DZ_Q1_STEP(3, v, f0, 6, u)
      DZ_Q1_STEP(4, p, f1, 7, v)
      DZ_Q1_STEP(5, q, f1, 8, p)
      DZ_Q1_STEP(6, u, f1, 9, q)
      DZ_Q1_STEP(7, v, f1, 10, u)
      DZ_Q1_STEP(8, p, f2, 11, v)
      DZ_Q1_STEP(9, q, f2, 12, p)
      DZ_Q1_STEP(10, u, f2, 13, q)
      DZ_Q1_STEP(11, v, f2, 14, u)
      DZ_Q1_STEP(12, p, f3, 15, v)
      "s_waitcnt lgkmcnt(8)\n" DZ_Q1_ACC(q, f3)
      "s_waitcnt lgkmcnt(4)\n" DZ_Q1_ACC(u, f3)
      "s_waitcnt lgkmcnt(0)\n" DZ_Q1_ACC(v, f3)
      : [a0] "=&v"(a0), [a1] "=&v"(a1), [a2] "=&v"(a2), [a3] "=&v"(a3),
        [p0] "=&v"(p0), [p1] "=&v"(p1), [p2] "=&v"(p2), [p3] "=&v"(p3),
        [q0] "=&v"(q0), [q1] "=&v"(q1), [q2] "=&v"(q2), [q3] "=&v"(q3),
        [u0] "=&v"(u0), [u1] "=&v"(u1), [u2] "=&v"(u2), [u3] "=&v"(u3),
        [v0] "=&v"(v0), [v1] "=&v"(v1), [v2] "=&v"(v2), [v3] "=&v"(v3)
      : [w0] "v"(r.s[0].x), [w1] "v"(r.s[0].y), [w2] "v"(r.s[0].z), [w3] "v"(r.s[0].w),
        [w4] "v"(r.s[1].x), [w5] "v"(r.s[1].y), [w6] "v"(r.s[1].z), [w7] "v"(r.s[1].w),
        [w8] "v"(r.s[2].x), [w9] "v"(r.s[2].y), [w10] "v"(r.s[2].z), [w11] "v"(r.s[2].w),
        [w12] "v"(r.s[3].x), [w13] "v"(r.s[3].y), [w14] "v"(r.s[3].z), [w15] "v"(r.s[3].w),
        [c0] "v"(c[0]), [c1] "v"(c[1]), [c2] "v"(c[2]), [c3] "v"(c[3]), [c4] "v"(c[4]), [c5] "v"(c[5]),
        [c6] "v"(c[6]), [c7] "v"(c[7]), [c8] "v"(c[8]), [c9] "v"(c[9]), [c10] "v"(c[10]), [c11] "v"(c[11]),
        [c12] "v"(c[12]), [c13] "v"(c[13]), [c14] "v"(c[14]), [c15] "v"(c[15]),
        [f0] "v"(f0), [f1] "v"(f1), [f2] "v"(f2), [f3] "v"(f3),
        [k0] "s"(0x0C0C0400u), [k1] "s"(0x0C0C0501u), [k2] "s"(0x0C0C0602u), [k3] "s"(0x0C0C0703u)
      : "memory");
  return (a0 + a1) + (a2 + a3);
}
#undef DZ_Q1_STEP
#undef DZ_Q1_ACC
#undef DZ_Q1_ISSUE

// Builds LUT[v][p] from xs[0..511] (LDS).  NT threads; NT/64 threads share one position.
template <int NT>
__device__ __forceinline__ void build_lut(float* __restrict__ lut, const float* __restrict__ xs, unsigned tid) {
  constexpr int NGRP = NT / 64;
  constexpr int PER = 256 / NGRP;  // table entries per thread
  constexpr int KB = (PER == 64) ? 6 : (PER == 32) ? 5 : (PER == 16) ? 4 : 7;
  static_assert(PER == (1 << KB), "threads per workgroup must be 128, 256, 512 or 1024");
  const unsigned p = tid & 63, hi = tid >> 6;
  // the position's 8 inputs as two 16-byte reads: eight 4-byte reads xs[8p + j] would put the 64
  // lanes on 4 of the 32 banks (a 16-way conflict per read, serialised across the workgroup's waves)
  const float4 xa = *reinterpret_cast<const float4*>(xs + 8 * p);
  const float4 xb = *reinterpret_cast<const float4*>(xs + 8 * p + 4);
  const float x[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  float C = 0.f;
#pragma unroll
  for (int j = KB; j < 8; ++j) C += ((hi >> (j - KB)) & 1u) ? x[j] : -x[j];
  float A[8];
#pragma unroll
  for (int lo = 0; lo < 8; ++lo) A[lo] = ((lo & 1) ? x[0] : -x[0]) + ((lo & 2) ? x[1] : -x[1]) + ((lo & 4) ? x[2] : -x[2]);
  constexpr int NB = PER / 8;
#pragma unroll
  for (int mid = 0; mid < NB; ++mid) {
    float cb = C;
#pragma unroll
    for (int j = 3; j < KB; ++j) cb += ((mid >> (j - 3)) & 1) ? x[j] : -x[j];
#pragma unroll
    for (int lo = 0; lo < 8; ++lo) lut[(hi * PER + mid * 8 + lo) * 64 + p] = cb + A[lo];
  }
}

// LDS barrier that does not wait for outstanding global loads (weight prefetches stay in flight).
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt/expcnt left at max
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Row-block segments: up to 8 matrices stacked in one virtual row space (matvec_multi).
struct GemvSeg {
  const uint8_t* data;  // Q1Dev::data
  int64_t rb_begin;     // first virtual row-block of this segment
  int64_t nrb;
};

struct GemvGrid {
  GemvSeg seg[8];
  int nseg;
  int64_t total_rb;
  int ntiles;   // K tiles (all segments share K)
  int tpw;      // tiles per workgroup (consecutive)
  int n_tg;     // tile groups = ceil(ntiles / tpw)
  int rbw;      // row-blocks per workgroup = NWAVES * M
};

__device__ __forceinline__ const uint8_t* unit_ptr(const GemvGrid& g, int64_t rb, int t) {
  int s = 0;
#pragma unroll 1
  while (s + 1 < g.nseg && rb >= g.seg[s + 1].rb_begin) ++s;
  const int64_t lrb = rb - g.seg[s].rb_begin;
  return g.seg[s].data + ((size_t)lrb * g.ntiles + t) * kUnitBytes;
}

// Src: stage(xs, red, tile, tid, nthreads, chunk) writes the 512 LUT inputs of `tile` into LDS xs,
//      one column per thread (nthreads == kTileCols);
//      `red` is 16 floats of LDS scratch for reductions; chunk is the workgroup's row-block chunk
//      (sources that also publish per-tile values do so from chunk 0 only).
// Dst: store(tg, rb, lane, acc) consumes the row result (a partial when ntiles > tpw).
template <int NWAVES, int M, class Src, class Dst>
__global__ __launch_bounds__(NWAVES * 64) void gemv_lut_kernel(const GemvGrid g, const Src src, const Dst dst) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* lut = reinterpret_cast<float*>(smem);
  float* red = reinterpret_cast<float*>(smem + kLutBytes);
  float* xs = red + 16;
  constexpr int NT = NWAVES * 64;
  static_assert(NT == kTileCols, "staging runs one thread per tile column");
  const unsigned tid = threadIdx.x, lane = tid & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar row-block math
  const int tg = (int)(blockIdx.x % (unsigned)g.n_tg);
  const int64_t chunk = blockIdx.x / (unsigned)g.n_tg;
  const int t0 = tg * g.tpw;
  const int t1 = min(t0 + g.tpw, g.ntiles);

  // stage all LUT inputs of this tile group first: their loads are older than the weight prefetch
  for (int t = t0; t < t1; ++t) src.stage(xs + (t - t0) * kTileCols, red, t, tid, NT, chunk);

  int64_t rb[M];
  bool ok[M];
  UnitRegs cur[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    rb[m] = chunk * (NWAVES * M) + wave + NWAVES * m;
    ok[m] = rb[m] < g.total_rb;
    if (ok[m]) load_unit(unit_ptr(g, rb[m], t0), lane, cur[m]);
  }
  unsigned c[16];
  make_pos_consts(lane, c);
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;

  for (int t = t0; t < t1; ++t) {
    lds_barrier();  // xs staged (or previous tile's LUT reads finished)
    build_lut<NT>(lut, xs + (t - t0) * kTileCols, tid);
    lds_barrier();
    UnitRegs nxt[M];
    const bool more = t + 1 < t1;
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (more && ok[m]) load_unit(unit_ptr(g, rb[m], t + 1), lane, nxt[m]);
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (ok[m]) acc[m] += unit_dot(cur[m], c);
#pragma unroll
    for (int m = 0; m < M; ++m) cur[m] = nxt[m];
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
    if (ok[m]) dst.store(tg, rb[m], lane, acc[m]);
}

// Output of one stacked matrix: rows [vrow_begin, vrow_begin + rows) of the virtual row space.
struct ReduceSeg {
  float* y;
  int64_t vrow_begin;  // first virtual row of the segment
  int64_t rows;        // logical rows
};

// ---- one-launch y = W x: split-K partials and their tile sum in the same kernel ----
//
// Workgroup (chunk, tile t) of the grid above with one tile per workgroup and one row-block per
// wave: the same staging, table and lookups as gemv_lut_kernel.  The tile's partial of every row
// goes out as a 64-bit word {f32 value, 32-bit call tag}, written through to the device coherence
// point.  The workgroup of the chunk's last tile then forms the chunk's rows (thread = row, the row
// whose partial it computed itself), y[row] = [y[row] +] sum_t part[t][row] in tile order (the
// order of partial_reduce_kernel), polling each word until it carries this call's tag: readiness
// travels with the data, so no fence, counter or barrier is involved.  The summing workgroup waits
// only for workgroups of lower index; the host launches this kernel only when the whole grid is
// resident at once, so all of them run.  A poll that never completes (bounded by spin_limit rounds;
// 0 gives up before the first check, for tests of the failure path) leaves NaN in the row and sets
// *err, which the host turns into DZ_ERR_DEVICE.
struct FusedGemvArgs {
  GemvGrid g;                  // tpw == 1, rbw == NWAVES
  const float* x;
  int64_t K;
  unsigned long long* part;    // [n_tg][ld] tagged words
  int64_t ld;
  unsigned tag;                // this call's tag (never 0: the buffer starts zeroed)
  int accumulate;
  int spin_limit;
  int* err;                    // set to 1 by a summing thread whose wait gave up
  ReduceSeg seg[8];            // output of each stacked matrix
};

template <int NWAVES>
__global__ __launch_bounds__(NWAVES * 64) void gemv_fused_kernel(const FusedGemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* lut = reinterpret_cast<float*>(smem);
  float* xs = reinterpret_cast<float*>(smem + kLutBytes + 64);
  constexpr int NT = NWAVES * 64;
  static_assert(NT == kTileCols, "staging runs one thread per tile column");
  typedef __attribute__((address_space(1))) unsigned long long gu64;
  const GemvGrid& g = a.g;
  const unsigned tid = threadIdx.x, lane = tid & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = (int)(blockIdx.x % (unsigned)g.n_tg);
  const int64_t chunk = blockIdx.x / (unsigned)g.n_tg;
  // the tile's inputs are staged before the weights are requested: the CU returns loads in issue
  // order, and inputs queued behind the weights would hold the table back until the weights arrive
  const int64_t col = (int64_t)t * kTileCols + tid;
  xs[tid] = col < a.K ? a.x[col] : 0.f;
  lds_barrier();
  const int64_t rb = chunk * NWAVES + wave;
  const bool ok = rb < g.total_rb;
  UnitRegs cur;
  if (ok) load_unit(unit_ptr(g, rb, t), lane, cur);
  unsigned c[16];
  make_pos_consts(lane, c);
  build_lut<NT>(lut, xs, tid);
  lds_barrier();
  const float acc = ok ? unit_dot(cur, c) : 0.f;
  if (ok)
    __hip_atomic_store((gu64*)(a.part + (size_t)t * a.ld + rb * kRowBlock + lane),
                       ((unsigned long long)a.tag << 32) | (unsigned long long)__float_as_uint(acc), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  if (t != g.n_tg - 1) return;
  // the chunk's rows: thread tid sums row chunk*NT + tid over the tiles
  const int64_t v = chunk * NT + tid;
  if (v >= g.total_rb * kRowBlock) return;
  const gu64* p = (const gu64*)(a.part + v);
  float sum = 0.f;
  bool good = true;
  for (int b = 0; b < g.n_tg && good; b += 16) {
    unsigned long long w[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int tt = b + k;
      // this thread's own partial (the last tile) is in a register
      w[k] = tt < g.n_tg - 1 ? __hip_atomic_load(p + (size_t)tt * a.ld, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : ((unsigned long long)a.tag << 32) | (unsigned long long)__float_as_uint(acc);
    }
    for (int spin = 0;; ++spin) {
      if (spin >= a.spin_limit) {
        good = false;
        break;
      }
      bool all = true;
#pragma unroll
      for (int k = 0; k < 16; ++k) all &= (unsigned)(w[k] >> 32) == a.tag;
      if (all) break;
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if ((unsigned)(w[k] >> 32) != a.tag)
          w[k] = __hip_atomic_load(p + (size_t)(b + k) * a.ld, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float pv = __uint_as_float((unsigned)w[k]);
      if (b + k == 0) sum = pv;
      else if (b + k < g.n_tg) sum += pv;
    }
  }
  int s = 0;
  while (s + 1 < g.nseg && v >= a.seg[s + 1].vrow_begin) ++s;
  const int64_t r = v - a.seg[s].vrow_begin;
  if (r >= a.seg[s].rows) return;
  float* y = a.seg[s].y + r;
  if (!good) __hip_atomic_store((__attribute__((address_space(1))) int*)a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  *y = !good ? __builtin_nanf("") : (a.accumulate ? *y + sum : sum);
}

// ---- common sources / destinations ----

struct PlainSrc {  // x[K] in device memory, zero beyond K
  const float* x;
  int64_t K;
  __device__ __forceinline__ void stage(float* xs, float*, int t, unsigned tid, int nt, int64_t) const {
    {  // one thread per tile column (nt == kTileCols)
      const int i = (int)tid;
      const int64_t col = (int64_t)t * kTileCols + i;
      xs[i] = col < K ? x[col] : 0.f;
    }
  }
};

struct PartialDst {  // part[tg][virtual row]
  float* part;
  int64_t ld;
  __device__ __forceinline__ void store(int tg, int64_t rb, unsigned lane, float v) const {
    part[(size_t)tg * ld + rb * kRowBlock + lane] = v;
  }
};

}  // namespace dz
