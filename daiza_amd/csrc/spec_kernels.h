// spec_kernels.h — the vocabulary-wide parts of speculative sampling on the device, so that a verify
// step returns a few words instead of k+1 logits rows: per-row softmax statistics with the draft
// token's probabilities (softmax_pair_single_avx2, Daiza-engine/src/math/simd_exp.rs:656-767) and the
// target's argmax (argmax_avx2, simd_exp.rs:551-598), and the top-k candidates of a row or of the
// residual distribution max(0, p - q) with its mass (sample_bonus, Daiza-runtime/src/engine.rs:
// 1833-1866; residual_max_zero_sum_avx2, simd_exp.rs:605-642).  For a verify step the host finishes
// the reference's temperature / top-k / top-p draw (sampling.rs:144-247) on those candidates; the
// device decode loop (dz_decode_sample) draws on the device, in the merge kernel.
#pragma once
#include "topk.h"

namespace dz {

struct SpecRowStats {
  float tmax, tsum, dmax, dsum;  // target / draft maximum and sum of exp(x - max)
  float p, q;                    // softmax(target)[token], softmax(draft)[token]
  int argmax;                    // first maximum of the target
  int pad;
};

// (v, i) is ahead of (w, j) in the order "larger value first, then lower index".
__device__ __forceinline__ bool cand_ahead(float v, int i, float w, int j) { return v > w || (v == w && i < j); }

template <int NT>
__device__ __forceinline__ void block_best(float& v, int& i, float* sv, int* si) {
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o);
    const int j = __shfl_xor(i, o);
    if (cand_ahead(w, j, v, i)) {
      v = w;
      i = j;
    }
  }
  const unsigned tid = threadIdx.x;
  __syncthreads();
  if ((tid & 63u) == 0) {
    sv[tid >> 6] = v;
    si[tid >> 6] = i;
  }
  __syncthreads();
  v = sv[0];
  i = si[0];
  for (int w = 1; w < NT / 64; ++w)
    if (cand_ahead(sv[w], si[w], v, i)) {
      v = sv[w];
      i = si[w];
    }
}

template <int NT>
__device__ __forceinline__ float block_total(float s, float* sv) {
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const unsigned tid = threadIdx.x;
  __syncthreads();
  if ((tid & 63u) == 0) sv[tid >> 6] = s;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < NT / 64; ++w) t += sv[w];
  return t;
}

constexpr int kSpecSlice = 4096;  // elements per slice of a row (a workgroup's share)
constexpr int kSpecMaxK = 64;
__host__ __device__ inline int spec_slices(int V) { return (V + kSpecSlice - 1) / kSpecSlice; }

// Per-slice softmax statistics of one row: maxima (the target's first maximum) and sums of
// exp(x - slice max), merged per row by spec_stats_merge_kernel.
struct SpecPart {
  float tmax, tsum, dmax, dsum;
  int targ;
  int pad[3];
};

// Grid (n rows, spec_slices(V) slices), 256 threads.  Row r's target logits: row0 for r = 0,
// rows + (r-1)·V after; its draft logits drafts + r·V for r < nd (none for greedy or past the
// drafts: statistics of the target only).
__global__ __launch_bounds__(256) void spec_stats_part_kernel(const float* __restrict__ row0,
                                                              const float* __restrict__ rows,
                                                              const float* __restrict__ drafts, int nd, int V,
                                                              SpecPart* __restrict__ part) {
  constexpr int NT = 256;
  __shared__ float sv[NT / 64];
  __shared__ int si[NT / 64];
  const int r = blockIdx.x, sl = blockIdx.y;
  const float* t = r == 0 ? row0 : rows + (size_t)(r - 1) * V;
  const float* d = drafts && r < nd ? drafts + (size_t)r * V : nullptr;
  const int i0 = sl * kSpecSlice, i1 = min(V, i0 + kSpecSlice);
  float tm = -INFINITY, dm = -INFINITY;
  int ti = 0x7FFFFFFF;
  for (int i = i0 + (int)threadIdx.x; i < i1; i += NT) {
    const float x = t[i];
    if (cand_ahead(x, i, tm, ti)) {
      tm = x;
      ti = i;
    }
    if (d) dm = fmaxf(dm, d[i]);
  }
  block_best<NT>(tm, ti, sv, si);
  int dummy = 0;
  block_best<NT>(dm, dummy, sv, si);
  float ts = 0.f, ds = 0.f;
  for (int i = i0 + (int)threadIdx.x; i < i1; i += NT) {
    ts += expf(t[i] - tm);
    if (d) ds += expf(d[i] - dm);
  }
  ts = block_total<NT>(ts, sv);
  ds = block_total<NT>(ds, sv);
  if (threadIdx.x == 0) {
    SpecPart q;
    q.tmax = tm;
    q.tsum = ts;
    q.dmax = dm;
    q.dsum = ds;
    q.targ = ti;
    q.pad[0] = q.pad[1] = q.pad[2] = 0;
    part[(size_t)r * gridDim.y + sl] = q;
  }
}

// Grid n rows, 64 threads: the row's statistics from its slices (sums rescaled to the row maximum),
// then p = softmax(target)[tok[r]] and q = softmax(draft)[tok[r]] for r < nd (draft token r).
__global__ __launch_bounds__(64) void spec_stats_merge_kernel(const float* __restrict__ row0,
                                                              const float* __restrict__ rows,
                                                              const float* __restrict__ drafts, int nd, int V,
                                                              int nsl, const SpecPart* __restrict__ part,
                                                              const uint32_t* __restrict__ tok,
                                                              SpecRowStats* __restrict__ out) {
  const int r = blockIdx.x;
  const unsigned lane = threadIdx.x;
  const SpecPart* pr = part + (size_t)r * nsl;
  const bool has_d = drafts && r < nd;
  float tm = -INFINITY, dm = -INFINITY;
  int ti = 0x7FFFFFFF;
  for (int s = (int)lane; s < nsl; s += 64) {
    if (cand_ahead(pr[s].tmax, pr[s].targ, tm, ti)) {
      tm = pr[s].tmax;
      ti = pr[s].targ;
    }
    dm = fmaxf(dm, pr[s].dmax);
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(tm, o);
    const int j = __shfl_xor(ti, o);
    if (cand_ahead(w, j, tm, ti)) {
      tm = w;
      ti = j;
    }
    dm = fmaxf(dm, __shfl_xor(dm, o));
  }
  float ts = 0.f, ds = 0.f;
  for (int s = (int)lane; s < nsl; s += 64) {
    ts += pr[s].tsum * expf(pr[s].tmax - tm);
    if (has_d) ds += pr[s].dsum * expf(pr[s].dmax - dm);
  }
  for (int o = 32; o > 0; o >>= 1) {
    ts += __shfl_xor(ts, o);
    ds += __shfl_xor(ds, o);
  }
  if (lane == 0) {
    const float* t = r == 0 ? row0 : rows + (size_t)(r - 1) * V;
    const float* d = has_d ? drafts + (size_t)r * V : nullptr;
    const int k = r < nd ? (int)tok[r] : 0;
    SpecRowStats s;
    s.tmax = tm;
    s.tsum = ts;
    s.dmax = d ? dm : -INFINITY;
    s.dsum = d ? ds : 0.f;
    const float tsn = ts > 0.f ? ts : 1.f, dsn = ds > 0.f ? ds : 1.f;
    s.p = expf(t[k] - tm) / tsn;
    s.q = d ? expf(d[k] - dm) / dsn : 0.f;
    s.argmax = ti;
    s.pad = 0;
    out[r] = s;
  }
}

// The value a top-k pass ranks: the logit itself (mode 0) or the residual mass
// max(0, softmax(t)_i - softmax(d)_i) of sample_bonus (mode 1, softmax as softmax_inplace: times 1/sum).
__device__ __forceinline__ float spec_value(const float* t, const float* d, int i, int mode, const SpecRowStats& s) {
  if (mode == 0) return t[i];
  const float p = expf(t[i] - s.tmax) * (1.0f / s.tsum), q = expf(d[i] - s.dmax) * (1.0f / s.dsum);
  return fmaxf(p - q, 0.0f);
}

// Stage 1: grid spec_slices(V), 256 threads.  Slice s of the row (kSpecSlice elements, in LDS) keeps
// its K best candidates in order (as keys, cand_key) and, in mode 1, its residual mass.  Each wave
// ranks its quarter of the slice in registers (16 keys per lane): K rounds of a lane's largest key
// below the previous pick and a wave maximum, with no workgroup barrier; the first wave then merges
// the four ordered lists by their heads.  Past the row's end the keys are kCandNone, and a list runs
// out with kCandNone entries.
__global__ __launch_bounds__(256) void spec_topk_slice_kernel(const float* __restrict__ t, const float* __restrict__ d,
                                                              int V, int mode, const SpecRowStats* __restrict__ st,
                                                              int K, uint64_t* __restrict__ cand,
                                                              float* __restrict__ mass) {
  constexpr int NT = 256, NW = NT / 64, PER = kSpecSlice / NT;
  __shared__ float sv[NW];
  __shared__ float vals[kSpecSlice];
  __shared__ uint64_t lst[NW][kSpecMaxK];
  const SpecRowStats s = *st;
  const int i0 = blockIdx.x * kSpecSlice, n = min(V - i0, kSpecSlice);
  // the thread's PER values requested together (a loop with a run-time bound waits one memory round
  // trip per value), then added in index order
  float x[PER];
  if (mode == 0) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int j = (int)threadIdx.x + NT * q;
      x[q] = j < n ? t[i0 + j] : 0.f;
    }
  } else {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int j = (int)threadIdx.x + NT * q;
      x[q] = j < n ? spec_value(t, d, i0 + j, 1, s) : 0.f;
    }
  }
  float m = 0.f;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int j = (int)threadIdx.x + NT * q;
    if (j < n) {
      vals[j] = x[q];
      m += x[q];
    }
  }
  m = block_total<NT>(m, sv);  // (its barriers also publish vals)
  if (threadIdx.x == 0) mass[blockIdx.x] = mode == 1 ? m : 0.f;
  const int lane = (int)(threadIdx.x & 63u), w = (int)(threadIdx.x >> 6);
  uint64_t key[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int j = w * (kSpecSlice / NW) + 64 * q + lane;
    key[q] = j < n ? cand_key(vals[j], i0 + j) : kCandNone;
  }
  uint64_t prev = ~0ull;  // the previous pick: candidates must come after it
  for (int k = 0; k < K; ++k) {
    uint64_t best = kCandNone;
#pragma unroll
    for (int q = 0; q < PER; ++q) best = key[q] < prev && key[q] > best ? key[q] : best;
    best = wave_max_key(best);
    if (lane == 0) lst[w][k] = best;
    prev = best;
  }
  __syncthreads();
  if (w != 0) return;
  int h = 0;  // lane l < NW: the head of wave l's list
  for (int k = 0; k < K; ++k) {
    const uint64_t c = lane < NW && h < K ? lst[lane][h] : kCandNone;
    const uint64_t best = wave_max_key(c);
    if (best != kCandNone && c == best) ++h;  // keys are unique within a row (the index is part of it)
    if (lane == 0) cand[(size_t)blockIdx.x * K + k] = best;
  }
}

// The draw of sample_top_k_top_p_into (sampling.rs:144-247) after a merge, for the device decode
// loop: rng null = no draw.
struct SpecDraw {
  float inv_t, top_p;
  uint64_t* rng;  // LcgRng state (sampling.rs:14-18)
  uint32_t* next; // the chosen id
};

// Stage 2: one workgroup of 256 threads merges the slices' candidates into the row's K best, in
// order (as (value, index) pairs), and adds the slices' masses in slice order.  The keys are staged
// in LDS (dynamic: slices * K entries); the first wave follows every slice's ordered list by its
// head (lane l: slices l, l + 64, ...; up to 4 per lane) and takes K rounds of the largest head.
// With dr.rng set it then draws the next id from the K best logits (spec_draw: temperature, softmax
// over the K, top-p cut, one LcgRng draw).
__global__ __launch_bounds__(256) void spec_topk_merge_kernel(const uint64_t* __restrict__ cand, int slices, int K,
                                                              const float* __restrict__ mass, SpecCand* __restrict__ out,
                                                              float* __restrict__ total, const SpecDraw dr) {
  constexpr int NT = 256, MAXL = 4, U = 8;
  extern __shared__ uint64_t lc[];
  const int nc = slices * K;
  for (int c0 = 0; c0 < nc; c0 += NT * U) {  // U keys per thread in flight at once
    uint64_t r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + (int)threadIdx.x + NT * u;
      r[u] = c < nc ? cand[c] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + (int)threadIdx.x + NT * u;
      if (c < nc) lc[c] = r[u];
    }
  }
  __syncthreads();
  const int lane = (int)(threadIdx.x & 63u), w = (int)(threadIdx.x >> 6);
  auto at = [](float x, int j) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j)); };
  if (w == 1) {  // the masses in slice order, 64 loaded at a time
    float m = 0.f;
    for (int s0 = 0; s0 < slices; s0 += 64) {
      const float x = s0 + lane < slices ? mass[s0 + lane] : 0.f;
      const int cnt = min(64, slices - s0);
      for (int j = 0; j < cnt; ++j) m += at(x, j);
    }
    if (lane == 0) *total = m;
  }
  if (w != 0) return;
  int h[MAXL] = {0, 0, 0, 0};
  uint64_t mine = kCandNone;  // lane j < K: candidate j of the result
  for (int k = 0; k < K; ++k) {
    uint64_t best = kCandNone;
    int bm = -1;
#pragma unroll
    for (int m = 0; m < MAXL; ++m) {
      const int sl = lane + 64 * m;
      if (sl < slices && h[m] < K) {
        const uint64_t c = lc[sl * K + h[m]];
        if (c > best) {
          best = c;
          bm = m;
        }
      }
    }
    const uint64_t top = wave_max_key(best);
#pragma unroll
    for (int m = 0; m < MAXL; ++m)
      if (m == bm && top != kCandNone && best == top) ++h[m];
    if (lane == 0) out[k] = cand_of(top);
    if (lane == k) mine = top;
  }
  if (dr.rng == nullptr) return;
  uint64_t rs = *dr.rng;
  const int chosen = spec_draw(mine, K, dr.inv_t, dr.top_p, rs);
  if (lane == 0) {
    *dr.rng = rs;
    *dr.next = (uint32_t)chosen;
  }
}

// LDS bytes of spec_topk_merge_kernel for `slices` slices of K candidates (0 when they do not fit:
// more than 256 slices, or above 64 KiB).
__host__ __device__ inline size_t spec_merge_shmem(int slices, int K) {
  const size_t b = (size_t)slices * (size_t)K * sizeof(uint64_t);
  return slices > 256 || b > 65536 ? 0 : b;
}

}  // namespace dz
