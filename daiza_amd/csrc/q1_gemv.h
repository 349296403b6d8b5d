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

typedef __attribute__((address_space(3))) const float lds_cfloat;

// LDS load at an absolute LDS byte address.  The GEMV kernel allocates no static LDS, so its
// dynamic LDS (the table) starts at address 0 and the v_perm result is the address itself.
__device__ __forceinline__ float lds_at(unsigned byte_addr) { return *(lds_cfloat*)(uintptr_t)byte_addr; }

// Dot product of one lane's 512-weight row slice with the tile whose table sits at LDS address 0.
__device__ __forceinline__ float unit_dot(const UnitRegs& r, const unsigned c[16]) {
  const float sc[4] = {half_lo(r.sc.x), half_hi(r.sc.x), half_lo(r.sc.y), half_hi(r.sc.y)};
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const unsigned w = r.s[m >> 2][m & 3];  // stored bytes 4m..4m+3
    const float s = sc[m >> 2];             // slot (4m+k) >> 4
    // byte0 <- c[m].byte k (position offset), byte1 <- w.byte k (sign byte), bytes 2,3 <- 0
    const unsigned ad0 = __builtin_amdgcn_perm(w, c[m], 0x0C0C0400u);
    const unsigned ad1 = __builtin_amdgcn_perm(w, c[m], 0x0C0C0501u);
    const unsigned ad2 = __builtin_amdgcn_perm(w, c[m], 0x0C0C0602u);
    const unsigned ad3 = __builtin_amdgcn_perm(w, c[m], 0x0C0C0703u);
    a0 = __builtin_fmaf(s, lds_at(ad0), a0);
    a1 = __builtin_fmaf(s, lds_at(ad1), a1);
    a2 = __builtin_fmaf(s, lds_at(ad2), a2);
    a3 = __builtin_fmaf(s, lds_at(ad3), a3);
  }
  return (a0 + a1) + (a2 + a3);
}

// Builds LUT[v][p] from xs[0..511] (LDS).  NT threads; NT/64 threads share one position.
template <int NT>
__device__ __forceinline__ void build_lut(float* __restrict__ lut, const float* __restrict__ xs, unsigned tid) {
  constexpr int NGRP = NT / 64;
  constexpr int PER = 256 / NGRP;  // table entries per thread
  constexpr int KB = (PER == 64) ? 6 : (PER == 32) ? 5 : (PER == 16) ? 4 : 7;
  static_assert(PER == (1 << KB), "threads per workgroup must be 128, 256, 512 or 1024");
  const unsigned p = tid & 63, hi = tid >> 6;
  float x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = xs[8 * p + j];
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
