// topk.h — candidate keys, the wave maximum over them and the top-k / top-p draw, shared by the
// vocabulary top-k kernels (spec_kernels.h) and the persistent token kernel's sampled selection
// (ptk_kernel.h), so that both rank and draw with the same instructions.
#pragma once
#include "common.h"

namespace dz {

struct SpecCand {
  float v;
  int i;
};

// Candidates as 64-bit keys whose unsigned order is "larger value first, then lower index": the
// value's bits mapped to an order-preserving unsigned word (a zero of either sign as +0, which
// compares equal to -0) in the high half, the complement of the index in the low half.  A NaN value
// gets key 0, below every other key, so it is never taken; "none" (-inf, 0x7FFFFFFF) is the key
// below every real candidate.
__device__ __forceinline__ uint64_t cand_key(float v, int i) {
  if (v != v) return 0ull;
  const unsigned u = __float_as_uint(v == 0.f ? 0.f : v);
  const unsigned o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)o << 32) | (uint64_t)(~(unsigned)i);
}
constexpr uint64_t kCandNone = ((uint64_t)0x007FFFFFu << 32) | 0x80000000u;  // cand_key(-inf, 0x7FFFFFFF)
__device__ __forceinline__ SpecCand cand_of(uint64_t k) {
  const unsigned o = (unsigned)(k >> 32);
  const unsigned u = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
  return SpecCand{__uint_as_float(u), (int)~(unsigned)k};
}

// The largest key of the wave, in every lane: the 16 lanes of each DPP row (xor 1, xor 2, half-row
// mirror, row mirror), then the four rows' lanes 0, 16, 32, 48.
template <int CTRL>
__device__ __forceinline__ uint64_t key_max_dpp(uint64_t k) {
  const unsigned lo = (unsigned)__builtin_amdgcn_mov_dpp((int)(unsigned)k, CTRL, 0xF, 0xF, false);
  const unsigned hi = (unsigned)__builtin_amdgcn_mov_dpp((int)(unsigned)(k >> 32), CTRL, 0xF, 0xF, false);
  const uint64_t o = ((uint64_t)hi << 32) | lo;
  return o > k ? o : k;
}
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
  k = key_max_dpp<0xB1>(k);
  k = key_max_dpp<0x4E>(k);
  k = key_max_dpp<0x141>(k);
  k = key_max_dpp<0x140>(k);
  uint64_t m = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t o = ((uint64_t)(unsigned)__builtin_amdgcn_readlane((int)(unsigned)(k >> 32), 16 * r) << 32) |
                       (unsigned)__builtin_amdgcn_readlane((int)(unsigned)k, 16 * r);
    m = o > m ? o : m;
  }
  return m;
}

// The largest word of the wave (every lane's result is the same): the 16 lanes of each DPP row, then
// the four rows' lanes 0, 16, 32, 48.
// (Each DPP move reads a lane of its own row, never out of range; written with 0, the identity of
// the maximum, as the value of an invalid lane, it folds into the maximum instruction.)
template <int CTRL>
__device__ __forceinline__ unsigned max_dpp_u32(unsigned v) {
  return max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
  v = max_dpp_u32<0xB1>(v);
  v = max_dpp_u32<0x4E>(v);
  v = max_dpp_u32<0x141>(v);
  v = max_dpp_u32<0x140>(v);
  const unsigned a = (unsigned)__builtin_amdgcn_readlane((int)v, 0), b = (unsigned)__builtin_amdgcn_readlane((int)v, 16);
  const unsigned c = (unsigned)__builtin_amdgcn_readlane((int)v, 32), d = (unsigned)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// The K largest keys over per-lane queues, for a whole wave (all 64 lanes active): lane l's queue
// q[0..Q) holds keys in descending order, padded with kCandNone.  Each round takes the largest high
// half of the queue heads (wave_max_u32), and, when more than one lane holds it (equal values), the
// largest low half among those lanes; the lane holding the winner advances its queue.  Lane k < K
// returns the k-th largest key, in cand_key's order; past the last real candidate, kCandNone.
template <int Q>
__device__ __forceinline__ uint64_t queue_select(uint64_t (&q)[Q], int K) {
  const int lane = (int)(threadIdx.x & 63u);
  uint64_t mine = kCandNone;
  for (int k = 0; k < K; ++k) {
    const unsigned hi = (unsigned)(q[0] >> 32), lo = (unsigned)q[0];
    const unsigned M = wave_max_u32(hi);
    const unsigned long long tie = __ballot(hi == M);
    unsigned L;
    int wl;
    if (__popcll(tie) == 1) {
      wl = __ffsll((long long)tie) - 1;
      L = (unsigned)__builtin_amdgcn_readlane((int)lo, wl);
    } else {
      L = wave_max_u32(hi == M ? lo : 0u);
      wl = __ffsll((long long)__ballot(hi == M && lo == L)) - 1;
    }
    const uint64_t key = ((uint64_t)M << 32) | L;
    if (key <= kCandNone) break;  // keys of real candidates are unique and above kCandNone
    if (lane == k) mine = key;
    if (lane == wl) {
#pragma unroll
      for (int i = 0; i + 1 < Q; ++i) q[i] = q[i + 1];
      q[Q - 1] = kCandNone;
    }
  }
  return mine;
}

// The draw of sample_top_k_top_p_into (Daiza-engine/src/math/sampling.rs:144-247) over the k best
// logits, run by one wave whose lane j < K holds candidate j's key (in rank order; temperature > 0):
// softmax over the K, the top-p cut at the first cumulative probability >= top_p, renormalisation,
// one LcgRng draw r (sampling.rs:14-18, state advanced in *rs) and the first candidate whose
// cumulative probability reaches r.  The operations and their order are the host sampler's
// (Sampler::top_k_top_p), each sum taken in candidate order.  Returns the chosen id in every lane.
__device__ __forceinline__ int spec_draw(uint64_t mine, int K, float inv_t, float top_p, uint64_t& rs) {
  const int lane = (int)(threadIdx.x & 63u);
  auto at = [](float x, int j) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j)); };
  const SpecCand c = cand_of(mine);
  const float sc = lane < K ? c.v * inv_t : -INFINITY;
  // the candidates are in descending order and inv_t > 0: the largest scaled value is candidate 0's
  const float mx = at(sc, 0);
  float pr = lane < K ? expf(sc - mx) : 0.f;
  float sum = 0.f;
  for (int j = 0; j < K; ++j) sum += at(pr, j);
  const float inv_sum = 1.0f / sum;
  pr *= inv_sum;
  float cum = 0.f;
  int cutoff = K;
  for (int j = 0; j < K; ++j) {
    cum += at(pr, j);
    if (cum >= top_p) {
      cutoff = j + 1;
      break;
    }
  }
  float ns = 0.f;
  for (int j = 0; j < cutoff; ++j) ns += at(pr, j);
  const float ninv = 1.0f / ns;
  pr *= ninv;
  rs = rs * 6364136223846793005ull + 1442695040888963407ull;
  const float r = (float)(uint32_t)((rs >> 40) & 0xFFFFFFu) / (float)0x1000000;
  float acc = 0.f;
  int chosen = __builtin_amdgcn_readlane(c.i, 0);
  for (int j = 0; j < cutoff; ++j) {
    acc += at(pr, j);
    if (r <= acc) {
      chosen = __builtin_amdgcn_readlane(c.i, j);
      break;
    }
  }
  return chosen;
}

}  // namespace dz
