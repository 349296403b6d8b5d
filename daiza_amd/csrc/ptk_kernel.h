// ptk_kernel.h — device code of the persistent token kernel (declarations in ptk.h).
#pragma once
#include "ptk.h"

namespace dz {

// LDS map of the kernel (dynamic LDS only, so that the LUT sits at LDS address 0 as unit_dot needs).
constexpr int kLdsXs = kLutBytes;                          // 512 floats: staged LUT input
constexpr int kLdsRed = kLdsXs + kTileCols * 4;            // 64 floats: reductions
constexpr int kLdsFlag = kLdsRed + 64 * 4;                 // 4 ints: abort flag
constexpr int kLdsAsg = kLdsFlag + 16;                     // 8 x {t, rb0, rb1, lead}: GEMV assignments
constexpr int kLdsRing = kLdsAsg + 8 * 16;                 // kPtkMaxLayers ints: conv ring bases
constexpr int kLdsScratch = kLdsRing + kPtkMaxLayers * 4;  // phase scratch
constexpr int kLdsScratchBytes = 28 * 1024;
// > 80 KiB so that a CU never holds two workgroups of this kernel
constexpr size_t kPtkLds = (size_t)kLdsScratch + kLdsScratchBytes;

template <class T>
__device__ __forceinline__ T* lds_ptr(unsigned char* smem, int off) { return reinterpret_cast<T*>(smem + off); }

// Workgroup-wide agreement on failure (the flag only ever goes 0 -> 1; a set flag ends the kernel).
__device__ __forceinline__ bool wg_ok(unsigned char* smem, bool ok) {
  int* f = lds_ptr<int>(smem, kLdsFlag);
  if (!ok) __hip_atomic_fetch_or(f, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  lds_barrier();
  return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0;
}

__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Deterministic block sum over 512 threads; every thread gets the result.
__device__ __forceinline__ float block_sum512(float v, float* red, unsigned tid) {
  v = wave_sum(v);
  if ((tid & 63u) == 0) red[tid >> 6] = v;
  lds_barrier();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kPtkWaves; ++w) s += red[w];
  lds_barrier();
  return s;
}

// 1 / rms of a length-n vector from its per-tile sums of squares sst[0..nt) (nt <= 64), read by
// wave 0 only and shared through LDS.
__device__ __forceinline__ bool inv_rms_tiles(unsigned char* smem, const u64* sst, unsigned tag, int nt, int n,
                                              float eps, unsigned tid, const PtkErr& e, float& inv) {
  float* red = lds_ptr<float>(smem, kLdsRed);
  bool ok = true;
  if (tid < 64) {
    float v = 0.f;
    if ((int)tid < nt) ok = ll_wait1(sst + tid, v, tag, e);
    const float s = wave_sum(v);
    if (tid == 0) red[32] = 1.0f / sqrtf(s / (float)n + eps);
  }
  if (!wg_ok(smem, ok)) return false;
  inv = red[32];
  return true;
}

constexpr int kPtkColQ = 4;  // terms per thread in ll_colsum (checked on the host)

// Column sums of LL words spread over the workgroup: for each of nc columns j, the terms
// k = 0..K-1 at ptr(j, k), each carrying tag tagf(k), are summed.  Thread (j, q) sums terms
// [q*Q, (q+1)*Q) in order (Q <= QMAX, checked on the host) into LDS, then thread j adds the slices
// in order: deterministic, and at most QMAX words in flight per thread.  Thread j < nc receives its
// column's sum in `out`.
template <int QMAX, class Ptr, class Tag>
__device__ __forceinline__ bool ll_colsum(unsigned char* smem, int nc, int K, const Ptr& ptr, const Tag& tagf,
                                          unsigned tid, const PtkErr& e, float& out) {
  float* slice = lds_ptr<float>(smem, kLdsScratch + 16 * 1024);  // up to 512 floats
  bool ok = true;
  int nq = 1, Q = K;
  if (nc > 0) {
    nq = min(kPtkThreads / nc, K);
    if (nq < 1) nq = 1;
    Q = (K + nq - 1) / nq;
    if ((int)tid < nq * nc) {
      const int j = (int)tid % nc, q = (int)tid / nc;
      const int k0 = q * Q, k1 = min(K, k0 + Q);
      u64 w[QMAX];
      unsigned tg[QMAX];
#pragma unroll
      for (int i = 0; i < QMAX; ++i) {
        tg[i] = tagf(k0 + i);
        w[i] = k0 + i < k1 ? ll_ld(ptr(j, k0 + i)) : ((u64)tg[i] << 32);
      }
      for (int spin = 0;; ++spin) {
        bool all = true;
#pragma unroll
        for (int i = 0; i < QMAX; ++i) all &= ll_tag(w[i]) == tg[i];
        if (all) break;
        if (spin >= e.spin_limit) {
          ptk_fail(e, 3, tg[0]);
          ok = false;
          break;
        }
        if ((spin & 31) == 31 && flag_ld(e.flag)) {
          ok = false;
          break;
        }
#pragma unroll
        for (int i = 0; i < QMAX; ++i)
          if (ll_tag(w[i]) != tg[i]) w[i] = ll_ld(ptr(j, k0 + i));
      }
      float sv = 0.f;
#pragma unroll
      for (int i = 0; i < QMAX; ++i) sv += k0 + i < k1 ? ll_val(w[i]) : 0.f;
      slice[q * nc + j] = sv;
    }
  }
  if (!wg_ok(smem, ok)) return false;
  if ((int)tid < nc) {
    float sv = 0.f;
    for (int q = 0; q < nq; ++q) sv += slice[q * nc + (int)tid];
    out = sv;
  }
  lds_barrier();  // slices are reused by the next call
  return true;
}

struct NoPrefetch {
  __device__ __forceinline__ void operator()() const {}
};

// ------------------------------------------------------------------ GEMV phase pieces

// Weights of one GEMV phase held by a wave: U row-blocks of the phase's tile (a kernel instance
// sizes U per matrix kind, so that only the next phase's weights stay live across a wait).
template <int U>
struct WRegs {
  UnitRegs u[U];
};

template <int U>
__device__ __forceinline__ void gemv_prefetch(const uint8_t* W, int ntiles, const Assign& a, unsigned wave, unsigned lane,
                                              WRegs<U>& r) {
#pragma unroll
  for (int m = 0; m < U; ++m) {
    const int rb = a.rb0 + (int)wave + kPtkWaves * m;
    if (rb < a.rb1) {
      load_unit(W + ((size_t)rb * ntiles + a.t) * kUnitBytes, lane, r.u[m]);
    } else {  // define every slot, so that the previous phase's registers are dead from here on
      r.u[m].s[0] = r.u[m].s[1] = r.u[m].s[2] = r.u[m].s[3] = u32x4{0u, 0u, 0u, 0u};
      r.u[m].sc = u32x2{0u, 0u};
    }
  }
}

template <int U>
__device__ __forceinline__ void gemv_compute_ll(const Assign& a, const WRegs<U>& r, const unsigned c[16], u64* out,
                                                int64_t ld, unsigned tag, unsigned wave, unsigned lane) {
#pragma unroll
  for (int m = 0; m < U; ++m) {
    const int rb = a.rb0 + (int)wave + kPtkWaves * m;
    if (rb < a.rb1) ll_st(out + (size_t)a.t * ld + (size_t)rb * kRowBlock + lane, unit_dot(r.u[m], c), tag);
  }
}

// LUT input sources: write xs[tid] for tile t (one column per thread) after waiting for their words.
// The tile's sum of v^2 goes to sq (the GEMV phase publishes it from one workgroup per tile when
// sst is set: the RMSNorm statistics of v, applied to the GEMV result by the consumer).
struct SrcNormedLL {  // v[col] * w[col]
  const u64* v;
  unsigned tag;
  const float* w;
  int K;
  u64* sst;
  __device__ __forceinline__ bool stage(float* xs, int t, unsigned tid, const PtkErr& e, float& sq) const {
    const int col = t * kTileCols + (int)tid;
    float x = 0.f;
    bool ok = true;
    sq = 0.f;
    if (col < K) {
      float hv;
      ok = ll_wait1(v + col, hv, tag, e);
      x = hv * w[col];
      sq = hv * hv;
    }
    xs[tid] = x;
    return ok;
  }
};

struct SrcPlainLL {
  const u64* v;
  unsigned tag;
  int K;
  static constexpr u64* sst = nullptr;
  __device__ __forceinline__ bool stage(float* xs, int t, unsigned tid, const PtkErr& e, float& sq) const {
    sq = 0.f;
    const int col = t * kTileCols + (int)tid;
    float x = 0.f;
    bool ok = true;
    if (col < K) ok = ll_wait1(v + col, x, tag, e);
    xs[tid] = x;
    return ok;
  }
};

// DeltaNet out-projection input: per v-head RMSNorm of y (from the quarters' sums of squares) times
// ssm_norm times silu(z) (ssm_output_gate_avx2, model/ssm.rs:246-286).
struct SrcGatedYLL {
  const u64* y;
  const u64* zs;
  const u64* yss;  // [nvh][4]
  unsigned tag;
  const float* nw;
  int K;
  static constexpr u64* sst = nullptr;
  __device__ __forceinline__ bool stage(float* xs, int t, unsigned tid, const PtkErr& e, float& sq) const {
    sq = 0.f;
    const int col = t * kTileCols + (int)tid;
    float x = 0.f;
    bool ok = true;
    if (col < K) {
      const int head = col >> 7;
      const u64* a[6] = {y + col, zs + col, yss + head * 4, yss + head * 4 + 1, yss + head * 4 + 2, yss + head * 4 + 3};
      u64 w[6];
      ok = ll_wait<6>(a, w, tag, e);
      const float s = (ll_val(w[2]) + ll_val(w[3])) + (ll_val(w[4]) + ll_val(w[5]));
      const float inv = 1.0f / sqrtf(s * (1.0f / 128.0f) + 1e-6f);
      x = ((ll_val(w[0]) * inv) * nw[col & 127]) * ll_val(w[1]);
    }
    xs[tid] = x;
    return ok;
  }
};

// One split-K GEMV phase on weights already requested (by the previous phase, right after its own
// polls: vector loads complete in issue order, so weights in flight delay any later poll): stage +
// LUT + units -> LL partials [t][row].  The first workgroup of each tile publishes the tile's sum
// of squares when the source provides one.
template <int U, class Src>
__device__ __forceinline__ bool gemv_phase(unsigned char* smem, const Src& src, const WRegs<U>& r, const Assign& a,
                                           bool lead, u64* out, int64_t ld, unsigned tag, unsigned tid,
                                           const PtkErr& e) {
  float* lut = lds_ptr<float>(smem, 0);
  float* xs = lds_ptr<float>(smem, kLdsXs);
  float sq;
  const bool ok = src.stage(xs, a.t, tid, e, sq);
  if (!wg_ok(smem, ok)) return false;
  if (src.sst != nullptr && lead) {
    const float s = block_sum512(sq, lds_ptr<float>(smem, kLdsRed), tid);
    if (tid == 0) ll_st(src.sst + a.t, s, tag);
  }
  build_lut<kPtkThreads>(lut, xs, tid);
  lds_barrier();
  unsigned c[16];
  make_pos_consts(tid & 63u, c);
  gemv_compute_ll(a, r, c, out, ld, tag, tid >> 6, tid & 63u);
  lds_barrier();  // every wave is done with the LUT before anyone rebuilds it
  return true;
}

// ------------------------------------------------------------------ phase S: token + embedding

template <class Pf>
__device__ __forceinline__ bool phase_select(unsigned char* smem, const PtkPlan& P, const PtkRun& r, int i, int w,
                                             unsigned tid, u64* tokreg, const u64* prev_cand_v, const u64* prev_cand_i,
                                             unsigned tag_prev_l, unsigned tag, int pos, int& tok_out, const Pf& pf) {
  const PtkErr& e = r.err;
  int* tok_s = lds_ptr<int>(smem, kLdsScratch);
  if (i < r.n_feed) {
    if (tid == 0) *tok_s = glb(r.feed)[i];
  } else {
    // greedy: first maximum over the previous lm_head's per-workgroup candidates (simd_exp.rs:551-598)
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    bool ok = true;
    if ((int)tid < P.G) {
      const u64* a[2] = {prev_cand_v + tid, prev_cand_i + tid};
      u64 wv[2];
      ok = ll_wait<2>(a, wv, tag_prev_l, e);
      bv = ll_val(wv[0]);
      bi = __float_as_int(ll_val(wv[1]));
    }
    if (!wg_ok(smem, ok)) return false;
    wave_argmax(bv, bi);
    float* sv = lds_ptr<float>(smem, kLdsScratch + 64);
    int* si = lds_ptr<int>(smem, kLdsScratch + 128);
    if ((tid & 63u) == 0) {
      sv[tid >> 6] = bv;
      si[tid >> 6] = bi;
    }
    lds_barrier();
    if (tid == 0) {
      for (int wv = 1; wv < kPtkWaves; ++wv)
        if (am_better(sv[wv], si[wv], bv, bi)) {
          bv = sv[wv];
          bi = si[wv];
        }
      *tok_s = bi == 0x7FFFFFFF ? 0 : bi;
    }
  }
  lds_barrier();
  const int tok = *tok_s;
  tok_out = tok;
  if (w == 0 && tid == 0) P.toklog[pos] = tok;
  // embedding columns [c0, c1) of this workgroup (forward.rs:212-213)
  int c0, c1;
  even_split(w, P.G, P.H, &c0, &c1);
  u64* hemb = tokreg;
  for (int col = c0 + (int)tid; col < c1; col += kPtkThreads) {
    float v;
    if (P.embd_f16) {
      v = ref_f16_to_f32_dev(P.emb_f16[(size_t)tok * P.H + col]);
    } else {
      const int64_t rb = tok / kRowBlock;
      const unsigned L = (unsigned)(tok % kRowBlock);
      const int t = col / kTileCols;
      const unsigned p = (unsigned)((col % kTileCols) / 8), j = (unsigned)(col % 8), s = L ^ p;
      const uint8_t* u = P.emb_q1 + ((size_t)rb * P.emb_ntiles + t) * kUnitBytes;
      const unsigned byte = u[((s >> 4) * 64 + L) * 16 + (s & 15)];
      const uint16_t* scp = reinterpret_cast<const uint16_t*>(u + kUnitSignBytes);
      const float scale = ref_f16_to_f32_dev(scp[L * 4 + ((p >> 4) ^ (L >> 4))]);
      v = ((float)((byte >> j) & 1u) * 2.0f - 1.0f) * scale;
    }
    ll_st(hemb + col, v, tag);
  }
  pf();
  return true;
}

// ------------------------------------------------------------------ R phases (tile sums)

// h_out = h_in + sum_t part[t][col] for this workgroup's columns (term 0 is h_in, then the tiles in
// order), all polled together; pf() runs after the result is stored.  Columns per workgroup <= 512.
template <int NT, class Pf>
__device__ __forceinline__ bool phase_resid(unsigned char* smem, const PtkPlan& P, int w, unsigned tid, const u64* h_in,
                                            unsigned tag_h, const u64* part, int np, int64_t ldp, unsigned tag_p,
                                            u64* h_out, unsigned tag, const PtkErr& e, const Pf& pf) {
  int c0, c1;
  even_split(w, P.G, P.H, &c0, &c1);
  const int nc = c1 - c0;
  auto ptr = [&](int j, int k) { return k == 0 ? h_in + c0 + j : part + (size_t)(k - 1) * ldp + c0 + j; };
  auto tagf = [&](int k) { return k == 0 ? tag_h : tag_p; };
  float v = 0.f;
  if (!ll_colsum<kPtkColQ>(smem, nc, np + 1, ptr, tagf, tid, e, v)) return false;
  if ((int)tid < nc) ll_st(h_out + c0 + tid, v, tag);
  pf();  // after the store: issuing a whole phase of weights can stall until part of it has landed
  return true;
}

// sw[f] = silu(inv * sum_t g) * (inv * sum_t u) for this workgroup's ffn channels (mlp.rs:28-47):
// columns 0..nf-1 are the gate rows, nf..2nf-1 the up rows, column 2nf the tile sums of squares of
// h_mid (all written by the gate/up phase); pf() runs after the results are stored.
template <int NT, class Pf>
__device__ __forceinline__ bool phase_swiglu(unsigned char* smem, const PtkPlan& P, int w, unsigned tid, const u64* sstm,
                                             const u64* pgu, unsigned tag_p, u64* sw, unsigned tag, const PtkErr& e,
                                             const Pf& pf) {
  int f0, f1;
  even_split(w, P.G, P.F, &f0, &f1);
  const int nf = f1 - f0;
  const int64_t ldp = (int64_t)P.nrb_gu * kRowBlock;
  auto ptr = [&](int j, int k) {
    return j == 2 * nf ? sstm + k : pgu + (size_t)k * ldp + (j < nf ? f0 + j : P.F + f0 + (j - nf));
  };
  auto tagf = [&](int) { return tag_p; };
  float v = 0.f;
  if (!ll_colsum<kPtkColQ>(smem, 2 * nf + 1, P.nT_h, ptr, tagf, tid, e, v)) return false;
  float* gu = lds_ptr<float>(smem, kLdsScratch);
  if ((int)tid <= 2 * nf) gu[tid] = v;
  lds_barrier();
  const float inv = 1.0f / sqrtf(gu[2 * nf] / (float)P.H + P.eps);
  if ((int)tid < nf) ll_st(sw + f0 + tid, siluf_(gu[tid] * inv) * (gu[nf + tid] * inv), tag);
  pf();
  lds_barrier();
  return true;
}

// ------------------------------------------------------------------ phase B: Gated DeltaNet step

// Workgroup w < 4*nvh: v-head w/4, state rows (w%4)*32 .. +32; threads 0..255 as in deltanet_kernel.
template <int NTH, class Pf>
__device__ __forceinline__ bool phase_deltanet(unsigned char* smem, const PtkPlan& P, const PtkLayer& Ly, int ring_base,
                                               int w, unsigned tid, int pos, const u64* sst_in, const u64* pin,
                                               unsigned tag_in, u64* y, u64* zs, u64* yss, unsigned tag,
                                               const PtkErr& e, const Pf& pf) {
  constexpr int HD = 128;
  if (w >= 4 * P.nvh) {
    pf();
    return true;
  }
  float* qs = lds_ptr<float>(smem, kLdsScratch);
  float* ks = qs + HD;
  float* vs = ks + HD;
  float* red = vs + 32;  // [0..3] q/k norms, [24] inv rms
  float* part = red + 16;  // [8][32]
  float* dsh = part + 8 * 32;
  float* sc = dsh + 32;
  const int vh = w >> 2, quarter = w & 3, kh = vh % P.nkh;
  const int i_loc = tid & 31, js = (tid >> 5) & 7;
  const int i = quarter * 32 + i_loc;
  const int hb = (ring_base + pos) & 3;
  const int64_t kdim = (int64_t)P.nkh * HD, qkvd = P.qkvd;
  const int64_t ldp = (int64_t)Ly.nrb_in * kRowBlock;
  const bool act = tid < 256;
  float s[16];
  float xq = 0.f, x2 = 0.f;
  float r1 = 0.f, r2 = 0.f, r3 = 0.f, w0 = 0.f, w1 = 0.f, w2 = 0.f, w3 = 0.f;
  float v1 = 0.f, v2 = 0.f, v3 = 0.f, u0 = 0.f, u1 = 0.f, u2 = 0.f, u3 = 0.f, ssm_a = 0.f, dtb = 0.f;
  int64_t ch = 0, row2 = -1;
  bool ok = true;
  if (act) {
    float* S = Ly.state + (size_t)vh * HD * HD;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) s[jj] = S[(size_t)(js * 16 + jj) * HD + i];
    ch = tid < HD ? (int64_t)kh * HD + tid : kdim + (int64_t)kh * HD + (tid - HD);
    r1 = co_ld(Ly.conv + (size_t)((hb + 1) & 3) * qkvd + ch);
    r2 = co_ld(Ly.conv + (size_t)((hb + 2) & 3) * qkvd + ch);
    r3 = co_ld(Ly.conv + (size_t)((hb + 3) & 3) * qkvd + ch);
    w0 = Ly.conv_w[ch];
    w1 = Ly.conv_w[qkvd + ch];
    w2 = Ly.conv_w[2 * qkvd + ch];
    w3 = Ly.conv_w[3 * qkvd + ch];
    if (tid < 32) row2 = 2 * kdim + (int64_t)vh * HD + quarter * 32 + tid;
    else if (tid < 64) row2 = P.off_z + (int64_t)vh * HD + quarter * 32 + (tid - 32);
    else if (tid == 64) row2 = P.off_a + vh;
    else if (tid == 65) row2 = P.off_b + vh;
    if (tid < 32) {
      v1 = co_ld(Ly.conv + (size_t)((hb + 1) & 3) * qkvd + row2);
      v2 = co_ld(Ly.conv + (size_t)((hb + 2) & 3) * qkvd + row2);
      v3 = co_ld(Ly.conv + (size_t)((hb + 3) & 3) * qkvd + row2);
      u0 = Ly.conv_w[row2];
      u1 = Ly.conv_w[qkvd + row2];
      u2 = Ly.conv_w[2 * qkvd + row2];
      u3 = Ly.conv_w[3 * qkvd + row2];
    }
    if (tid == 64) {
      ssm_a = Ly.ssm_a[vh];
      dtb = Ly.dt_bias[vh];
    }
  }
  // the layer input's tile sums of squares (inv rms), polled alongside the projections
  u64 sw = (u64)tag_in << 32;
  if ((int)tid < P.nT_h) sw = ll_ld(sst_in + tid);
  if (act) {
    ok = ll_sum<NTH>(pin + ch, ldp, P.nT_h, tag_in, e, xq);
    if (ok && row2 >= 0) ok = ll_sum<NTH>(pin + row2, ldp, P.nT_h, tag_in, e, x2);
  }
  if ((int)tid < P.nT_h && ok) {
    for (int spin = 0; ll_tag(sw) != tag_in; ++spin) {
      if (spin >= e.spin_limit) {
        ptk_fail(e, 4, tag_in);
        ok = false;
        break;
      }
      sw = ll_ld(sst_in + tid);
    }
  }
  if (tid < 64) {
    const float sst = wave_sum((int)tid < P.nT_h ? ll_val(sw) : 0.f);
    if (tid == 0) red[24] = 1.0f / sqrtf(sst / (float)P.H + P.eps);
  }
  if (!wg_ok(smem, ok)) return false;
  const float inv = red[24];
  // conv ring + causal conv + SiLU (ssm.rs:467-518)
  float qk = 0.f;
  if (act) {
    const float xn = xq * inv;
    float o = 0.f;
    o = __builtin_fmaf(r1, w0, o);
    o = __builtin_fmaf(r2, w1, o);
    o = __builtin_fmaf(r3, w2, o);
    o = __builtin_fmaf(xn, w3, o);
    qk = siluf_(o);
    if (vh < P.nkh && quarter == 0) co_st(Ly.conv + (size_t)hb * qkvd + ch, xn);
    const float x2n = x2 * inv;
    if (tid < 32) {
      float ov = 0.f;
      ov = __builtin_fmaf(v1, u0, ov);
      ov = __builtin_fmaf(v2, u1, ov);
      ov = __builtin_fmaf(v3, u2, ov);
      ov = __builtin_fmaf(x2n, u3, ov);
      vs[tid] = siluf_(ov);
      co_st(Ly.conv + (size_t)hb * qkvd + row2, x2n);
    } else if (tid < 64) {
      ll_st(zs + (size_t)vh * HD + quarter * 32 + (tid - 32), siluf_(x2n), tag);
    } else if (tid == 64) {
      const float x = x2n + dtb;
      const float sp = x > 20.0f ? x : logf(1.0f + expf(x));
      sc[0] = expf(ssm_a * sp);
    } else if (tid == 65) {
      sc[1] = sigmoidf_(x2n);
    }
  }
  const float s2 = wave_sum(qk * qk);
  if ((tid & 63u) == 0 && tid < 256) red[tid >> 6] = s2;
  lds_barrier();
  if (tid < HD) {
    const float inq = 1.0f / sqrtf((red[0] + red[1]) + 1e-6f);
    qs[tid] = (qk * inq) * (1.0f / sqrtf((float)HD));
  } else if (tid < 256) {
    const float ink = 1.0f / sqrtf((red[2] + red[3]) + 1e-6f);
    ks[tid - HD] = qk * ink;
  }
  lds_barrier();
  const float decay = sc[0], beta = sc[1];
  if (act) {
    float kvp = 0.f;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      s[jj] *= decay;
      kvp = __builtin_fmaf(s[jj], ks[js * 16 + jj], kvp);
    }
    part[js * 32 + i_loc] = kvp;
  }
  lds_barrier();
  if (tid < 32) {
    float kv = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) kv += part[q * 32 + i_loc];
    dsh[i_loc] = (vs[i_loc] - kv) * beta;
  }
  lds_barrier();
  if (act) {
    const float d = dsh[i_loc];
    float* S = Ly.state + (size_t)vh * HD * HD;
    float yp = 0.f;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int j = js * 16 + jj;
      s[jj] = __builtin_fmaf(d, ks[j], s[jj]);
      S[(size_t)j * HD + i] = s[jj];
      yp = __builtin_fmaf(s[jj], qs[j], yp);
    }
    part[js * 32 + i_loc] = yp;
  }
  lds_barrier();
  // the ring stores above are complete before this step's outputs become visible
  wait_stores();
  if (tid < 64) {
    float yy = 0.f;
    if (tid < 32) {
#pragma unroll
      for (int q = 0; q < 8; ++q) yy += part[q * 32 + i_loc];
      ll_st(y + (size_t)vh * HD + i, yy, tag);
    }
    const float ys = wave_sum(yy * yy);
    if (tid == 0) ll_st(yss + vh * 4 + quarter, ys, tag);
  }
  pf();  // the next matrix phase's weights (issued last: fewer registers live during the math)
  return true;
}

// ------------------------------------------------------------------ attention phases

// R0: q|gate|k|v projections = inv * sum of in-proj partials, for this workgroup's rows (the last
// column sums the layer input's tile sums of squares).
template <int NTH>
__device__ __forceinline__ bool phase_qkv(unsigned char* smem, const PtkPlan& P, const PtkLayer& Ly, int w, unsigned tid,
                                          const u64* sst_in, const u64* pin, unsigned tag_in, u64* qkv, unsigned tag,
                                          const PtkErr& e) {
  int r0, r1;
  even_split(w, P.G, Ly.rows_in, &r0, &r1);
  const int nr = r1 - r0;
  const int64_t ldp = (int64_t)Ly.nrb_in * kRowBlock;
  auto ptr = [&](int j, int k) { return j == nr ? sst_in + k : pin + (size_t)k * ldp + r0 + j; };
  auto tagf = [&](int) { return tag_in; };
  float v = 0.f;
  if (!ll_colsum<kPtkColQ>(smem, nr + 1, P.nT_h, ptr, tagf, tid, e, v)) return false;
  float* red = lds_ptr<float>(smem, kLdsRed);
  if ((int)tid == nr) red[32] = 1.0f / sqrtf(v / (float)P.H + P.eps);
  lds_barrier();
  if ((int)tid < nr) ll_st(qkv + r0 + tid, v * red[32], tag);
  lds_barrier();
  return true;
}

__device__ __forceinline__ void attn_chunks(const PtkPlan& P, int pos, int* chunk, int* gc) {
  const int ctx = pos + 1;
  int ch = (ctx + P.gmax - 1) / P.gmax;
  if (ch < 16) ch = 16;
  *chunk = ch;
  *gc = (ctx + ch - 1) / ch;
}

// B': workgroup (kv-head, chunk g) -- online softmax of attention.rs:124-199 over its positions
// for the kv-head's GRP query heads; q/k RMSNorm, the reference's +/+ partial RoPE, q *= 1/sqrt(hd);
// the chunk holding the new position appends its k/v.  Writes rec = (m, l, o[hd]) per q-head.
template <int GRP>
__device__ __forceinline__ bool phase_attn(unsigned char* smem, const PtkPlan& P, const PtkLayer& Ly, int w,
                                           unsigned tid, int pos, const u64* qkv, unsigned tag_q, u64* rec,
                                           unsigned tag, const PtkErr& e) {
  constexpr int HD = 256;
  const int kvh = w / P.gmax, g = w % P.gmax;
  int chunk, gc;
  attn_chunks(P, pos, &chunk, &gc);
  if (kvh >= P.nkv || g >= gc) return true;
  const unsigned lane = tid & 63u, wave = tid >> 6;
  const int ctx = pos + 1, p0 = g * chunk, p1 = min(ctx, p0 + chunk);
  const bool has_new = p1 == ctx;
  float* qs = lds_ptr<float>(smem, kLdsScratch);        // [GRP][HD]
  float* kn = qs + GRP * HD;                            // [HD]
  float* vn = kn + HD;                                  // [HD]
  float* red = vn + HD;                                 // [GRP+1][4]
  float* wm = red + (GRP + 1) * 4;                      // [8][GRP]
  float* wl = wm + kPtkWaves * GRP;                     // [8][GRP]
  float* wo = lds_ptr<float>(smem, 0);                  // [8][GRP][HD] in the LUT area (unused here)
  const int half = P.rope_dim / 2;
  const float* cs = P.rope + (size_t)pos * P.rope_dim;
  // raw projections, one dim per thread (threads 0..255)
  float qv[GRP];
  float kvv = 0.f, vvv = 0.f;
  bool ok = true;
  if (tid < HD) {
    const u64* a[GRP + 2];
    const int64_t kb = (int64_t)P.nq * 2 * HD;
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) a[gi] = qkv + (int64_t)(kvh * GRP + gi) * 2 * HD + tid;
    a[GRP] = qkv + kb + (int64_t)kvh * HD + tid;
    a[GRP + 1] = qkv + kb + (int64_t)P.nkv * HD + (int64_t)kvh * HD + tid;
    u64 wv[GRP + 2];
    ok = ll_wait<GRP + 2>(a, wv, tag_q, e);
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) qv[gi] = ll_val(wv[gi]);
    kvv = ll_val(wv[GRP]);
    vvv = ll_val(wv[GRP + 1]);
  } else {
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) qv[gi] = 0.f;
  }
  if (!wg_ok(smem, ok)) return false;
  // per-head RMSNorm over 256 dims (waves 0..3 hold the dims)
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    const float sq = wave_sum(qv[gi] * qv[gi]);
    if (lane == 0 && wave < 4) red[gi * 4 + wave] = sq;
  }
  {
    const float sq = wave_sum(kvv * kvv);
    if (lane == 0 && wave < 4) red[GRP * 4 + wave] = sq;
  }
  lds_barrier();
  if (tid < HD) {
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      const float ssum = (red[gi * 4 + 0] + red[gi * 4 + 1]) + (red[gi * 4 + 2] + red[gi * 4 + 3]);
      const float in = 1.0f / sqrtf(ssum / (float)HD + P.eps);
      qs[gi * HD + tid] = (qv[gi] * in) * Ly.q_norm[tid];
    }
    const float ssum = (red[GRP * 4 + 0] + red[GRP * 4 + 1]) + (red[GRP * 4 + 2] + red[GRP * 4 + 3]);
    const float in = 1.0f / sqrtf(ssum / (float)HD + P.eps);
    kn[tid] = (kvv * in) * Ly.k_norm[tid];
    vn[tid] = vvv;
  }
  lds_barrier();
  float r1[GRP], r2[GRP];
  float kr1 = 0.f, kr2 = 0.f;
  if ((int)tid < half) {
    const float c = cs[tid], sn = cs[half + tid];
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      const float x1 = qs[gi * HD + tid], x2 = qs[gi * HD + tid + half];
      r1[gi] = __builtin_fmaf(x1, c, x2 * sn);
      r2[gi] = __builtin_fmaf(x2, c, x1 * sn);
    }
    const float x1 = kn[tid], x2 = kn[tid + half];
    kr1 = __builtin_fmaf(x1, c, x2 * sn);
    kr2 = __builtin_fmaf(x2, c, x1 * sn);
  }
  lds_barrier();
  if ((int)tid < half) {
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      qs[gi * HD + tid] = r1[gi];
      qs[gi * HD + tid + half] = r2[gi];
    }
    kn[tid] = kr1;
    kn[tid + half] = kr2;
  }
  lds_barrier();
  const float qscale = 1.0f / sqrtf((float)HD);
  if (tid < HD) {
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) qs[gi * HD + tid] *= qscale;
    if (has_new) {
      co_st(Ly.kc + ((size_t)kvh * P.max_ctx + pos) * HD + tid, kn[tid]);
      co_st(Ly.vc + ((size_t)kvh * P.max_ctx + pos) * HD + tid, vn[tid]);
    }
  }
  lds_barrier();
  // online softmax over this wave's positions; lane holds dims 4*lane .. 4*lane+3
  float m[GRP], l[GRP];
  float4 o[GRP], q4[GRP];
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    m[gi] = -INFINITY;
    l[gi] = 0.f;
    o[gi] = make_float4(0.f, 0.f, 0.f, 0.f);
    q4[gi] = *reinterpret_cast<const float4*>(&qs[gi * HD + 4 * lane]);
  }
  const float* kb = Ly.kc + (size_t)kvh * P.max_ctx * HD;
  const float* vb = Ly.vc + (size_t)kvh * P.max_ctx * HD;
  auto ld4 = [&](const float* p) {
    return make_float4(co_ld(p), co_ld(p + 1), co_ld(p + 2), co_ld(p + 3));
  };
  auto loadkv = [&](int p, float4& k4, float4& v4) {
    if (p == pos) {
      k4 = *reinterpret_cast<const float4*>(&kn[4 * lane]);
      v4 = *reinterpret_cast<const float4*>(&vn[4 * lane]);
    } else {
      k4 = ld4(kb + (size_t)p * HD + 4 * lane);
      v4 = ld4(vb + (size_t)p * HD + 4 * lane);
    }
  };
  int p = p0 + (int)wave;
  float4 ka = make_float4(0.f, 0.f, 0.f, 0.f), va = ka, kb1 = ka, vb1 = ka;
  if (p < p1) loadkv(p, ka, va);
  if (p + kPtkWaves < p1) loadkv(p + kPtkWaves, kb1, vb1);
  for (; p < p1; p += kPtkWaves) {
    float4 kc = ka, vc = va;
    if (p + 2 * kPtkWaves < p1) loadkv(p + 2 * kPtkWaves, kc, vc);
    const float4 k4 = ka, v4 = va;
    ka = kb1;
    va = vb1;
    kb1 = kc;
    vb1 = vc;
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      float dp = q4[gi].x * k4.x;
      dp = __builtin_fmaf(q4[gi].y, k4.y, dp);
      dp = __builtin_fmaf(q4[gi].z, k4.z, dp);
      dp = __builtin_fmaf(q4[gi].w, k4.w, dp);
      const float score = wave_sum(dp);
      const float mn = fmaxf(m[gi], score);
      const float al = expf(m[gi] - mn), be = expf(score - mn);
      l[gi] = l[gi] * al + be;
      o[gi].x = __builtin_fmaf(be, v4.x, o[gi].x * al);
      o[gi].y = __builtin_fmaf(be, v4.y, o[gi].y * al);
      o[gi].z = __builtin_fmaf(be, v4.z, o[gi].z * al);
      o[gi].w = __builtin_fmaf(be, v4.w, o[gi].w * al);
      m[gi] = mn;
    }
  }
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    if (lane == 0) {
      wm[wave * GRP + gi] = m[gi];
      wl[wave * GRP + gi] = l[gi];
    }
    *reinterpret_cast<float4*>(&wo[(wave * GRP + gi) * HD + 4 * lane]) = o[gi];
  }
  lds_barrier();
  // the KV append is complete before the chunk records become visible
  wait_stores();
  // merge the 8 waves (a wave without positions has l = 0) and publish each q-head's record
  if (tid < HD) {
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      float M = -INFINITY;
      for (int wv = 0; wv < kPtkWaves; ++wv) M = fmaxf(M, wm[wv * GRP + gi]);
      float L = 0.f, O = 0.f;
      for (int wv = 0; wv < kPtkWaves; ++wv) {
        const float ex = wl[wv * GRP + gi] > 0.f ? expf(wm[wv * GRP + gi] - M) : 0.f;
        L = __builtin_fmaf(wl[wv * GRP + gi], ex, L);
        O = __builtin_fmaf(wo[(wv * GRP + gi) * HD + tid], ex, O);
      }
      u64* rc = rec + ((size_t)(kvh * GRP + gi) * P.gmax + g) * (2 + HD);
      if (tid == 0) {
        ll_st(rc, M, tag);
        ll_st(rc + 1, L, tag);
      }
      ll_st(rc + 2 + tid, O, tag);
    }
  }
  lds_barrier();  // wo lives in the LUT area
  return true;
}

// R'': merge the chunk records of each q-head and apply the output gate (attention.rs:189-203):
// ao[h*hd + d] = (O/L) * sigmoid(gate).  Wave v handles outputs j0+v, j0+v+8, ...; lane = chunk.
template <class Pf>
__device__ __forceinline__ bool phase_attn_merge(unsigned char* smem, const PtkPlan& P, int w, unsigned tid, int pos,
                                                 const u64* rec, unsigned tag_r, const u64* qkv, unsigned tag_q,
                                                 u64* ao, unsigned tag, const PtkErr& e, const Pf& pf) {
  constexpr int HD = 256;
  int chunk, gc;
  attn_chunks(P, pos, &chunk, &gc);
  int j0, j1;
  even_split(w, P.G, P.nq * HD, &j0, &j1);
  const unsigned lane = tid & 63u, wave = tid >> 6;
  bool ok = true;
  for (int j = j0 + (int)wave; j < j1 && ok; j += kPtkWaves) {
    const int h = j / HD, d = j % HD;
    float mv = -INFINITY, lv = 0.f, ov = 0.f, gate = 0.f;
    if ((int)lane < gc) {
      const u64* r = rec + ((size_t)h * P.gmax + lane) * (2 + HD);
      const u64* a[3] = {r, r + 1, r + 2 + d};
      u64 wv[3];
      ok = ll_wait<3>(a, wv, tag_r, e);
      mv = ll_val(wv[0]);
      lv = ll_val(wv[1]);
      ov = ll_val(wv[2]);
    }
    if (lane == 0 && ok) ok = ll_wait1(qkv + (int64_t)(h * 2 + 1) * HD + d, gate, tag_q, e);
    ok = __builtin_amdgcn_readfirstlane((int)ok) && __all(ok);
    const float M = wave_max(mv);
    const float ex = (int)lane < gc ? expf(mv - M) : 0.f;
    const float L = wave_sum(lv * ex), O = wave_sum(ov * ex);
    gate = __shfl(gate, 0, 64);
    if (lane == 0 && ok) ll_st(ao + j, (O * (1.0f / L)) * sigmoidf_(gate), tag);
  }
  if (!wg_ok(smem, ok)) return false;
  pf();
  return true;
}

// ------------------------------------------------------------------ phase L: lm_head + argmax

// Full K per workgroup: rows [rb0, rb1) of the vocabulary, tile by tile (LUT per tile), with the
// next tile's weights in flight; logits = inv_rms(h) * W (h * output_norm) (forward.rs:332-341),
// the statistics accumulated while staging.
template <int U>
__device__ __forceinline__ bool phase_lm(unsigned char* smem, const PtkPlan& P, const PtkRun& r, int i, int w,
                                         unsigned tid, const u64* h_fin, unsigned tag_h, u64* cand_v, u64* cand_i,
                                         unsigned tag) {
  const PtkErr& e = r.err;
  const unsigned lane = tid & 63u, wave = tid >> 6;
  int rb0, rb1;
  even_split(w, P.G, P.nrb_v, &rb0, &rb1);
  float acc[U];
#pragma unroll
  for (int m = 0; m < U; ++m) acc[m] = 0.f;
  float* lut = lds_ptr<float>(smem, 0);
  float* xs = lds_ptr<float>(smem, kLdsXs);
  WRegs<U> cur;
  {
    Assign a0;
    a0.t = 0;
    a0.rb0 = rb0;
    a0.rb1 = rb1;
    gemv_prefetch(P.w_lm, P.nT_h, a0, wave, lane, cur);
  }
  float ssq = 0.f;  // this thread's share of sum(h^2): the output norm's statistics
  for (int t = 0; t < P.nT_h; ++t) {
    SrcNormedLL src{h_fin, tag_h, P.output_norm, P.H, nullptr};
    float sq;
    const bool ok = src.stage(xs, t, tid, e, sq);
    ssq += sq;
    if (!wg_ok(smem, ok)) return false;
    build_lut<kPtkThreads>(lut, xs, tid);
    lds_barrier();
    WRegs<U> nxt;
    const bool more = t + 1 < P.nT_h;
    {
      Assign an;
      an.t = more ? t + 1 : t;
      an.rb0 = rb0;
      an.rb1 = more ? rb1 : rb0;
      gemv_prefetch(P.w_lm, P.nT_h, an, wave, lane, nxt);
    }
    unsigned c[16];
    make_pos_consts(lane, c);
#pragma unroll
    for (int m = 0; m < U; ++m) {
      const int rb = rb0 + (int)wave + kPtkWaves * m;
      if (rb < rb1) acc[m] += unit_dot(cur.u[m], c);
    }
#pragma unroll
    for (int m = 0; m < U; ++m) cur.u[m] = nxt.u[m];
    lds_barrier();
  }
  // logits = inv_rms(h) * W (h * output_norm), and this workgroup's (max, first index)
  const float inv = 1.0f / sqrtf(block_sum512(ssq, lds_ptr<float>(smem, kLdsRed), tid) / (float)P.H + P.eps);
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  const bool last = i == r.n_tok - 1;
#pragma unroll
  for (int m = 0; m < U; ++m) {
    const int rb = rb0 + (int)wave + kPtkWaves * m;
    const int row = rb * kRowBlock + (int)lane;
    if (rb < rb1 && row < P.vocab) {
      const float lg = acc[m] * inv;
      if (r.want_logits) {
        if (P.logits_all) P.logits_all[(size_t)i * P.vocab + row] = lg;
        if (last) P.logits[row] = lg;
      }
      if (am_better(lg, row, bv, bi)) {
        bv = lg;
        bi = row;
      }
    }
  }
  wave_argmax(bv, bi);
  float* sv = lds_ptr<float>(smem, kLdsScratch + 64);
  int* si = lds_ptr<int>(smem, kLdsScratch + 128);
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  lds_barrier();
  if (tid == 0) {
    for (int wv = 1; wv < kPtkWaves; ++wv)
      if (am_better(sv[wv], si[wv], bv, bi)) {
        bv = sv[wv];
        bi = si[wv];
      }
    ll_st(cand_v + w, bv, tag);
    ll_st(cand_i + w, __int_as_float(bi), tag);
  }
  lds_barrier();
  return true;
}

// ------------------------------------------------------------------ the kernel

// This workgroup's assignment for matrix kind k (written to LDS at kernel start).
__device__ __forceinline__ Assign asg_at(unsigned char* smem, int k) {
  const int* q = lds_ptr<int>(smem, kLdsAsg) + 4 * k;
  Assign a;
  a.t = q[0];
  a.rb0 = q[1];
  a.rb1 = q[2];
  return a;
}
__device__ __forceinline__ bool asg_lead(unsigned char* smem, int k) { return lds_ptr<int>(smem, kLdsAsg)[4 * k + 3] != 0; }

// Completion time of phase `ph` of token i on this workgroup (tracing runs only).
__device__ __forceinline__ void ptk_mark(const PtkRun& r, const PtkPlan& P, int i, int ph, int w, unsigned tid) {
  if (r.trace && tid == 0) glb(r.trace)[((size_t)i * P.ppt + ph) * P.G + w] = __builtin_amdgcn_s_memrealtime();
}

// NTH / NTO / NTF bound the K-tile counts of hidden, mixer output and ffn; U_* are the row-block
// slots per wave of the in-proj, out-proj, gate/up, down and lm_head phases.
template <int NTH, int NTO, int NTF, int GRP, int U_IN, int U_OUT, int U_GU, int U_DN, int U_LM>
__global__ __launch_bounds__(kPtkThreads) void ptk_kernel(const PtkRun r) {
  extern __shared__ __align__(16) unsigned char smem[];
  const PtkPlan P = plan_view(r.plan);
  const PtkErr& e = r.err;
  const unsigned tid = threadIdx.x, lane = tid & 63u;
  const int w = (int)blockIdx.x, G = P.G;
  if (tid == 0) *lds_ptr<int>(smem, kLdsFlag) = 0;
  // this workgroup's GEMV assignments per matrix kind (0/1: in-proj of a DeltaNet/attention layer,
  // 2/3: out-proj, 4: gate/up, 5: down) and the conv ring bases, fixed for the launch
  if (tid < 6) {
    const int k = (int)tid;
    const int T = k < 2 ? P.nT_h : k < 4 ? P.nt_out_k[k - 2] : k == 4 ? P.nT_h : P.nT_f;
    const int nrb = k < 2 ? P.nrb_in_k[k] : k < 4 ? P.nrb_h : k == 4 ? P.nrb_gu : P.nrb_h;
    const Assign a = gemv_assign(w, G, T, nrb);
    int* q = lds_ptr<int>(smem, kLdsAsg) + 4 * k;
    q[0] = a.t;
    q[1] = a.rb0;
    q[2] = a.rb1;
    q[3] = w == tile_first_wg(a.t, T, G);
  }
  for (int l = (int)tid; l < P.n_layers; l += kPtkThreads) {
    const DZ_AS_CONST PtkLayer* t = (const DZ_AS_CONST PtkLayer*)P.L + l;
    lds_ptr<int>(smem, kLdsRing)[l] = t->attn ? 0 : *glb(t->ring_base);
  }
  lds_barrier();
  const PtkOffsets& O = P.off;
  const int64_t ld_in_h = (int64_t)P.nrb_h * kRowBlock;
  const int64_t cand_off = ld_in_h;  // token region: h_emb [ld_in_h], cand_v [G], cand_i [G]
  // one register set carries the next matrix phase's weights from the phase that requested them
  // to the phase that uses them (their live ranges never overlap)
  constexpr int UW = U_IN > U_OUT ? (U_IN > U_GU ? (U_IN > U_DN ? U_IN : U_DN) : (U_GU > U_DN ? U_GU : U_DN))
                                  : (U_OUT > U_GU ? (U_OUT > U_DN ? U_OUT : U_DN) : (U_GU > U_DN ? U_GU : U_DN));
  WRegs<UW> wn;
  const unsigned wave = tid >> 6;
  for (int i = 0; i < r.n_tok; ++i) {
    const unsigned tb = r.tag0 + (unsigned)i * (unsigned)P.ppt;
    const int par = (int)((r.tag0 / (unsigned)P.ppt + (unsigned)i) & 1u);
    const int pos = r.pos0 + i;
    u64* tokreg = ll_region(P, par, P.n_layers);
    const u64* prev_tok = ll_region(P, par ^ 1, P.n_layers);
    int tok;
    // weights of the next matrix phase are requested right after a phase's own polls
    auto pf_in = [&](int l) {
      return [&, l]() {
        const PtkLayer Ln = layer_at(P, l);
        gemv_prefetch(Ln.w_in, P.nT_h, asg_at(smem, Ln.attn), wave, lane, wn);
      };
    };
    if (!phase_select(smem, P, r, i, w, tid, tokreg, prev_tok + cand_off, prev_tok + cand_off + G,
                      tb - (unsigned)P.ppt + (unsigned)P.ph_l, tb, pos, tok, pf_in(0)))
      return;
    ptk_mark(r, P, i, 0, w, tid);
    const u64* h_in = tokreg;
    unsigned tag_h = tb;
    for (int l = 0; l < P.n_layers; ++l) {
      // an opaque copy of the thread index: values derived from it are recomputed in each layer
      // instead of being hoisted out of the loops (and kept live, or spilled, for the whole kernel)
      unsigned tid = threadIdx.x;
      asm volatile("" : "+v"(tid));
      const unsigned lane = tid & 63u, wave = tid >> 6;
      const PtkLayer Ly = layer_at(P, l);
      u64* R = ll_region(P, par, l);
      const unsigned t0 = tb + (unsigned)Ly.ph0;
      const int64_t ld_in = (int64_t)Ly.nrb_in * kRowBlock;
      const Assign a_out = asg_at(smem, 2 + Ly.attn);
      auto pf_out = [&]() { gemv_prefetch(Ly.w_out, Ly.nt_out, a_out, wave, lane, wn); };
      // A: in-proj of h * attn_norm; tile leaders publish sum(h^2) per tile (1/rms applied downstream)
      {
        const Assign a = asg_at(smem, Ly.attn);
        SrcNormedLL src{h_in, tag_h, Ly.attn_norm, P.H, R + O.sst_in};
        if (!gemv_phase(smem, src, wn, a, asg_lead(smem, Ly.attn), R + O.pin, ld_in, t0, tid, e)) return;
        ptk_mark(r, P, i, Ly.ph0, w, tid);
      }
      unsigned tag_o;
      int k;
      if (!Ly.attn) {
        // B: DeltaNet (then C's weights)
        if (!phase_deltanet<NTH>(smem, P, Ly, lds_ptr<int>(smem, kLdsRing)[l], w, tid, pos, R + O.sst_in, R + O.pin,
                                 t0, R + O.y, R + O.zs, R + O.yss, t0 + 1, e, pf_out))
          return;
        ptk_mark(r, P, i, Ly.ph0 + 1, w, tid);
        // C: out-proj
        SrcGatedYLL src{R + O.y, R + O.zs, R + O.yss, t0 + 1, Ly.ssm_norm, P.inner};
        if (!gemv_phase(smem, src, wn, a_out, false, R + O.po, ld_in_h, t0 + 2, tid, e)) return;
        ptk_mark(r, P, i, Ly.ph0 + 2, w, tid);
        tag_o = t0 + 2;
        k = 3;
      } else {
        if (!phase_qkv<NTH>(smem, P, Ly, w, tid, R + O.sst_in, R + O.pin, t0, R + O.qkv, t0 + 1, e)) return;
        ptk_mark(r, P, i, Ly.ph0 + 1, w, tid);
        if (!phase_attn<GRP>(smem, P, Ly, w, tid, pos, R + O.qkv, t0 + 1, R + O.rec, t0 + 2, e)) return;
        ptk_mark(r, P, i, Ly.ph0 + 2, w, tid);
        if (!phase_attn_merge(smem, P, w, tid, pos, R + O.rec, t0 + 2, R + O.qkv, t0 + 1, R + O.ao, t0 + 3, e, pf_out))
          return;
        ptk_mark(r, P, i, Ly.ph0 + 3, w, tid);
        SrcPlainLL src{R + O.ao, t0 + 3, P.nq * 256};
        if (!gemv_phase(smem, src, wn, a_out, false, R + O.po, ld_in_h, t0 + 4, tid, e)) return;
        ptk_mark(r, P, i, Ly.ph0 + 4, w, tid);
        tag_o = t0 + 4;
        k = 5;
      }
      // R1: h_mid = h + out-proj (then D's weights)
      const Assign a_gu = asg_at(smem, 4);
      auto pf_gu = [&]() { gemv_prefetch(Ly.w_gu, P.nT_h, a_gu, wave, lane, wn); };
      if (!phase_resid<NTO>(smem, P, w, tid, h_in, tag_h, R + O.po, Ly.nt_out, ld_in_h, tag_o, R + O.hmid, t0 + k, e,
                            pf_gu))
        return;
      ptk_mark(r, P, i, Ly.ph0 + k, w, tid);
      // D: gate/up of h_mid * post_norm; tile leaders publish sum(h_mid^2) per tile
      {
        SrcNormedLL src{R + O.hmid, t0 + k, Ly.post_norm, P.H, R + O.sst_mid};
        if (!gemv_phase(smem, src, wn, a_gu, asg_lead(smem, 4), R + O.pgu, (int64_t)P.nrb_gu * kRowBlock, t0 + k + 1,
                        tid, e))
          return;
        ptk_mark(r, P, i, Ly.ph0 + k + 1, w, tid);
      }
      // R2: SwiGLU (then E's weights)
      const Assign a_dn = asg_at(smem, 5);
      auto pf_dn = [&]() { gemv_prefetch(Ly.w_dn, P.nT_f, a_dn, wave, lane, wn); };
      if (!phase_swiglu<NTH>(smem, P, w, tid, R + O.sst_mid, R + O.pgu, t0 + k + 1, R + O.sw, t0 + k + 2, e, pf_dn))
        return;
      ptk_mark(r, P, i, Ly.ph0 + k + 2, w, tid);
      // E: down
      {
        SrcPlainLL src{R + O.sw, t0 + k + 2, P.F};
        if (!gemv_phase(smem, src, wn, a_dn, false, R + O.pd, ld_in_h, t0 + k + 3, tid, e)) return;
        ptk_mark(r, P, i, Ly.ph0 + k + 3, w, tid);
      }
      // R3: h = h_mid + down (then the next layer's in-proj weights; none after the last layer)
      auto pf_next = [&]() {
        const bool more = l + 1 < P.n_layers;
        const PtkLayer Ln = layer_at(P, more ? l + 1 : l);
        Assign an = asg_at(smem, Ln.attn);
        if (!more) an.rb1 = an.rb0;
        gemv_prefetch(Ln.w_in, P.nT_h, an, wave, lane, wn);
      };
      if (!phase_resid<NTF>(smem, P, w, tid, R + O.hmid, t0 + k, R + O.pd, P.nT_f, ld_in_h, t0 + k + 3, R + O.h,
                            t0 + k + 4, e, pf_next))
        return;
      ptk_mark(r, P, i, Ly.ph0 + k + 4, w, tid);
      h_in = R + O.h;
      tag_h = t0 + k + 4;
    }
    // L: lm_head + argmax candidates
    if (!phase_lm<U_LM>(smem, P, r, i, w, tid, h_in, tag_h, tokreg + cand_off, tokreg + cand_off + G,
                        tb + (unsigned)P.ph_l))
      return;
    ptk_mark(r, P, i, P.ph_l, w, tid);
    (void)tok;
  }
  // greedy pick after the last token, published as toklog[pos0 + n_tok] (workgroup 0 only)
  if (w == 0) {
    const int i = r.n_tok;
    const unsigned tb = r.tag0 + (unsigned)i * (unsigned)P.ppt;
    const int par = (int)((r.tag0 / (unsigned)P.ppt + (unsigned)i) & 1u);
    const u64* prev_tok = ll_region(P, par ^ 1, P.n_layers);
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    bool ok = true;
    if ((int)tid < G) {
      const u64* a[2] = {prev_tok + cand_off + tid, prev_tok + cand_off + G + tid};
      u64 wv[2];
      ok = ll_wait<2>(a, wv, tb - (unsigned)P.ppt + (unsigned)P.ph_l, e);
      bv = ll_val(wv[0]);
      bi = __float_as_int(ll_val(wv[1]));
    }
    if (!wg_ok(smem, ok)) return;
    wave_argmax(bv, bi);
    float* sv = lds_ptr<float>(smem, kLdsScratch + 64);
    int* si = lds_ptr<int>(smem, kLdsScratch + 128);
    if (lane == 0) {
      sv[tid >> 6] = bv;
      si[tid >> 6] = bi;
    }
    lds_barrier();
    if (tid == 0) {
      for (int wv = 1; wv < kPtkWaves; ++wv)
        if (am_better(sv[wv], si[wv], bv, bi)) {
          bv = sv[wv];
          bi = si[wv];
        }
      P.toklog[r.pos0 + r.n_tok] = bi == 0x7FFFFFFF ? 0 : bi;
    }
  }
}

}  // namespace dz
