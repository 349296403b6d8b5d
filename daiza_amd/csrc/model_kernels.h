// model_kernels.h — device side of the per-token forward (forward_single_token, forward.rs:204-375).
//
// One token is a fixed sequence of kernels (captured once in a hipGraph):
//   select_token -> per layer { GEMV(norm+in-proj) -> DeltaNet | attention -> GEMV(out-proj)
//                              -> GEMV(norm+gate/up) -> GEMV(swiglu+down) } -> final_reduce -> lm_head.
// GEMV kernels write split-K partials part[tile][row]; the consumer of a GEMV sums its tiles in
// order 0..T-1 while staging its own inputs, so no reduction kernel sits between phases.  The
// residual stream h is materialised tile by tile by the chunk-0 workgroup of each consuming GEMV
// (double buffered), together with that tile's sum of squares; RMSNorm's 1/rms is applied to
// the GEMV result (y = inv * W(h*w), equal to W((h*inv)*w) up to rounding).
#pragma once
#include "q1_gemv.h"

#include <type_traits>

namespace dz {

// Position/token bookkeeping of the token being processed (device resident).
struct TokState {
  int pos;        // position of this token
  int token;      // its id
  int feed_len;   // host-fed ids remaining in `feed` are consumed first
  int feed_idx;
  int pos_next;   // position the next token will take
  int pad[3];
};

// Sum over a full wave (all 64 lanes active).  DPP inside each row of 16 lanes (xor 1, xor 2,
// half-row mirror, row mirror: every lane then holds its row's sum), then the four row sums
// read with v_readlane; the result is wave-uniform and independent of lane order.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Deterministic block sum (wave sums, then wave order).  All threads get the result.
__device__ __forceinline__ float block_sum(float v, float* red, unsigned tid, int nt) {
  v = wave_sum(v);
  __syncthreads();
  if ((tid & 63u) == 0) red[tid >> 6] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < nt / 64; ++w) s += red[w];
  __syncthreads();
  return s;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }

// Upper bounds on split-K tile counts summed by consumers (checked at model creation):
// K = hidden (<= 16 tiles of 512) and K = ffn or the out-projection width (<= 48 tiles).
constexpr int kMaxTilesH = 16;
constexpr int kMaxTilesF = 48;

// Calls f(std::integral_constant<int, B>{}) with the smallest partial-count bucket B >= np, so
// that a consumer's unconditional loads (sum_strided) waste at most a few slots.
template <class F>
__host__ inline auto with_np_bucket(int np, F&& f) {
  if (np <= 2) return f(std::integral_constant<int, 2>{});
  if (np <= 4) return f(std::integral_constant<int, 4>{});
  if (np <= 8) return f(std::integral_constant<int, 8>{});
  if (np <= 12) return f(std::integral_constant<int, 12>{});
  if (np <= 16) return f(std::integral_constant<int, 16>{});
  if (np <= 24) return f(std::integral_constant<int, 24>{});
  if (np <= 36) return f(std::integral_constant<int, 36>{});
  return f(std::integral_constant<int, 48>{});
}

// sum_{k<n} p[k*ld + idx] in order k = 0..n-1 (0 when n == 0), n <= MAXN, with every load
// issued before the first add: one memory round trip instead of n.  The loads are unconditional
// -- slots k >= n re-read slot n-1 (same cache line, no extra memory traffic) and are masked out
// of the sum -- and walk one pointer, so no branch, wait or per-slot scalar address sits between
// them.
template <int MAXN>
__device__ __forceinline__ float sum_strided(const float* __restrict__ p, int64_t ld, int n, int64_t idx) {
  if (n <= 0) return 0.f;
  float v[MAXN];
  const float* q = p + idx;
  // keep the stride in vector registers: a wave-uniform stride would be scalarised into MAXN live
  // 64-bit scalar addresses (spilled to VGPR lanes) before the first load could issue
  int64_t step = ld;
  asm volatile("" : "+v"(step));
#pragma unroll
  for (int k = 0; k < MAXN; ++k) {
    v[k] = *q;
    q += (k + 1 < n) ? step : 0;
  }
  float d = 0.f;
#pragma unroll
  for (int k = 0; k < MAXN; ++k) d += (k < n) ? v[k] : 0.f;
  return d;
}

// inverse RMS from per-tile sums of squares ss[0..nss), nss <= 64 (rmsnorm.rs:53-55):
// lane i loads ss[i], a butterfly sums them; every lane of every calling wave gets the value.
__device__ __forceinline__ float inv_rms_from(const float* ss, int nss, int64_t n, float eps) {
  const unsigned lane = threadIdx.x & 63u;
  const float s = wave_sum((int)lane < nss ? ss[lane] : 0.f);
  return 1.0f / sqrtf(s / (float)n + eps);
}

// ---------------------------------------------------------------- GEMV sources

// LUT input (h + sum_k part_k) * w; chunk 0 also writes h_out and the tile's sum of squares.
// NP bounds the partial count np (a launch picks the smallest instantiation that holds np).
template <int NP>
struct ResidSrc {
  const float* h_in;
  const float* part;
  int np;
  int64_t ldp;
  const float* w;
  float* h_out;
  float* ss_out;
  int64_t H;
  __device__ __forceinline__ void stage(float* xs, float* red, int t, unsigned tid, int nt, int64_t chunk) const {
    float ssl = 0.f;
    {  // one thread per tile column (nt == kTileCols)
      const int i = (int)tid;
      const int64_t col = (int64_t)t * kTileCols + i;
      float u = 0.f;
      if (col < H) {
        const float d = sum_strided<NP>(part, ldp, np, col);
        const float v = np ? h_in[col] + d : h_in[col];
        u = v * w[col];
        if (chunk == 0) h_out[col] = v;
        ssl = __builtin_fmaf(v, v, ssl);
      }
      xs[i] = u;
    }
    if (chunk == 0) {
      const float s = block_sum(ssl, red, tid, nt);
      if (tid == 0) ss_out[t] = s;
    }
  }
};

// LUT input silu(g) * u with g, u = inv_rms * sum of gate/up partials (swiglu_inplace_simd, simd_exp.rs:273-296).
template <int NP>
struct SwigluSrc {
  const float* part;  // [np][ldp]: gate rows [0, F), up rows [F, 2F)
  int np;
  int64_t ldp;
  int64_t F;
  const float* ss;
  int nss;
  int64_t H;
  float eps;
  __device__ __forceinline__ void stage(float* xs, float*, int t, unsigned tid, int nt, int64_t) const {
    const float inv = inv_rms_from(ss, nss, H, eps);
    {  // one thread per tile column (nt == kTileCols)
      const int i = (int)tid;
      const int64_t col = (int64_t)t * kTileCols + i;
      float u = 0.f;
      if (col < F) {
        float g = sum_strided<NP>(part, ldp, np, col);
        float up = sum_strided<NP>(part, ldp, np, F + col);
        g *= inv;
        up *= inv;
        u = siluf_(g) * up;
      }
      xs[i] = u;
    }
  }
};

// LUT input of the DeltaNet out-projection: per v-head RMSNorm * weight * silu(z)
// (Qwen3NextRMSNormGated, ssm_output_gate_avx2 in model/ssm.rs:246-286).
struct GatedYSrc {
  const float* y;
  const float* zs;
  const float* nw;  // [128]
  int64_t K;        // v_heads * 128
  float eps;
  __device__ __forceinline__ void stage(float* xs, float* red, int t, unsigned tid, int nt, int64_t) const {
    // 512 columns = 4 heads of 128; wave h (< 4) reduces head h
    {  // one thread per tile column (nt == kTileCols)
      const int i = (int)tid;
      const int64_t col = (int64_t)t * kTileCols + i;
      xs[i] = col < K ? y[col] : 0.f;
    }
    __syncthreads();
    const unsigned w = tid >> 6, l = tid & 63u;
    if (w < 4) {
      const float a = xs[w * 128 + l], b = xs[w * 128 + 64 + l];
      const float s = wave_sum(__builtin_fmaf(a, a, b * b));
      if (l == 0) red[w] = 1.0f / sqrtf(s * (1.0f / 128.0f) + eps);
    }
    __syncthreads();
    {  // one thread per tile column (nt == kTileCols)
      const int i = (int)tid;
      const int64_t col = (int64_t)t * kTileCols + i;
      xs[i] = col < K ? ((xs[i] * red[i >> 7]) * nw[i & 127]) * zs[col] : 0.f;
    }
  }
};

// Positions per chunk of the graph path's attention at context ctx with at most gmax chunks per kv
// head: whole 16-position tiles (so that no chunk ends in a tile of one position), at least 64 (four
// waves of one tile each).
__device__ __forceinline__ int attn_chunk(int ctx, int gmax) {
  int c = (ctx + gmax - 1) / gmax;
  c = (c + 15) / 16 * 16;
  return c < 64 ? 64 : c;
}

// The attention output of one token: combine the split-K softmax partials of each q-head and gate
// with sigmoid (attention.rs:189-203), once, into u[n_head * hd] for the out-projection.  Partial
// record: [m, l, o[hd]] per (head, chunk).  Workgroup (head, 64 dims), four waves: wave w sums
// chunks [32w, 32w + 32) in chunk order with weights exp(m_g - M), M the maximum over all chunks
// (every wave forms it from the (m, l) of all chunks); the four partial sums are then added in wave
// order.  Every load is issued at the start: the o values do not depend on M.
struct AttnMergeArgs {
  const float* apart;  // [n_head][gmax][2 + hd]
  int gmax;            // <= 128
  int hd;
  const TokState* st;
  int pos;            // this token's position, or -1: TokState.pos
  const float* p_in;  // in-projection partials (gate half of each q-head)
  int np;
  int64_t ldp;
  const float* ss;
  int nss;
  int64_t H;
  float eps;
  float* u;  // [n_head * hd]
};

template <int NP>
__global__ __launch_bounds__(256) void attn_merge_kernel(const AttnMergeArgs a) {
  __shared__ float wl[4][128][2];
  __shared__ float part[4][2][64];
  const unsigned tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  const int dq = a.hd / 64;
  const int h = blockIdx.x / dq, d = (blockIdx.x % dq) * 64 + (int)lane;
  const int ctx = (a.pos >= 0 ? a.pos : a.st->pos) + 1;
  const int chunk = attn_chunk(ctx, a.gmax);
  const int geff = (ctx + chunk - 1) / chunk;
  const size_t rs = (size_t)(2 + a.hd);
  const float* rec = a.apart + (size_t)h * a.gmax * rs;
  const int g0 = 32 * (int)w;
  float o[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) o[k] = g0 + k < geff ? rec[(g0 + k) * rs + 2 + d] : 0.f;
  float gate = 0.f;
  if (w == 0) gate = sum_strided<NP>(a.p_in, a.ldp, a.np, (int64_t)h * 2 * a.hd + a.hd + d);
  float mg[2], lg[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int g = (int)lane + 64 * k;
    mg[k] = g < geff ? rec[g * rs] : -INFINITY;
    lg[k] = g < geff ? rec[g * rs + 1] : 0.f;
  }
  const float M = wave_max(fmaxf(mg[0], mg[1]));
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int g = (int)lane + 64 * k;
    wl[w][g][0] = g < geff ? expf(mg[k] - M) : 0.f;
    wl[w][g][1] = lg[k];
  }
  __builtin_amdgcn_wave_barrier();
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    if (g0 + k < geff) {
      const float e = wl[w][g0 + k][0];
      L = __builtin_fmaf(wl[w][g0 + k][1], e, L);
      O = __builtin_fmaf(o[k], e, O);
    }
  }
  part[w][0][lane] = L;
  part[w][1][lane] = O;
  __syncthreads();
  if (w == 0) {
    const float Lt = ((part[0][0][lane] + part[1][0][lane]) + part[2][0][lane]) + part[3][0][lane];
    const float Ot = ((part[0][1][lane] + part[1][1][lane]) + part[2][1][lane]) + part[3][1][lane];
    const float inv = inv_rms_from(a.ss, a.nss, a.H, a.eps);
    a.u[(size_t)h * a.hd + d] = (Ot * (1.0f / Lt)) * sigmoidf_(gate * inv);
  }
}

// LUT input (h * inv_rms) * w with h already final (output norm before lm_head, forward.rs:332).
struct NormedSrc {
  const float* h;
  const float* w;
  const float* ss;
  int nss;
  int64_t H;
  float eps;
  __device__ __forceinline__ void stage(float* xs, float*, int t, unsigned tid, int nt, int64_t) const {
    const float inv = inv_rms_from(ss, nss, H, eps);
    {  // one thread per tile column (nt == kTileCols)
      const int i = (int)tid;
      const int64_t col = (int64_t)t * kTileCols + i;
      xs[i] = col < H ? (h[col] * inv) * w[col] : 0.f;
    }
  }
};

// ---------------------------------------------------------------- GEMV destinations

// (value, index) order of greedy argmax: larger value wins, equal values keep the lower index,
// NaN never wins (argmax_avx2 compares with `>`, simd_exp.rs:551-598).
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    if (am_better(ov, oi, v, i)) { v = ov; i = oi; }
  }
}

// Final logits plus one (max, first index) per row-block for greedy argmax.
struct LogitsDst {
  float* logits;
  int64_t V;
  float* am_val;  // [nrb]
  int* am_idx;
  __device__ __forceinline__ void store(int, int64_t rb, unsigned lane, float v) const {
    const int64_t row = rb * kRowBlock + lane;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    if (row < V) {
      logits[row] = v;
      bv = v;
      bi = (int)row;
    }
    wave_argmax(bv, bi);
    if (lane == 0) {
      am_val[rb] = bv;
      am_idx[rb] = bi;
    }
  }
};

// ---------------------------------------------------------------- token selection

struct SelectArgs {
  TokState* st;
  const int* feed;      // host-fed token ids (prompt / forced tokens)
  const float* am_val;  // argmax partials of the previous lm_head
  const int* am_idx;
  int n_am;
  int* toklog;          // toklog[pos] = token consumed at pos
  // embedding row -> emb_out (f32): f16 table, or Q1_0 GEMV layout with the reference's dequant
  const uint16_t* emb_f16;
  const uint8_t* emb_q1;
  int64_t emb_ntiles;
  int64_t H;
  float* emb_out;
  int commit;           // 1: consume the token (advance pos); 0: only publish the argmax to toklog[pos_next]
};

__device__ __forceinline__ float ref_f16_to_f32_dev(unsigned bits) {
  const unsigned sign = (bits >> 15) & 1u, exp = (bits >> 10) & 0x1Fu, mant = bits & 0x3FFu;
  const unsigned s32 = sign << 31;
  unsigned out;
  if (exp == 0) {
    if (mant == 0) {
      out = s32;
    } else {
      unsigned m = mant, e = 1;
      while ((m & 0x400u) == 0) { m <<= 1; ++e; }
      out = s32 | ((112u + e) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (exp == 0x1F) {
    out = s32 | 0x7F800000u | (mant << 13);
  } else {
    out = s32 | ((exp + 112u) << 23) | (mant << 13);
  }
  return __builtin_bit_cast(float, out);
}

// (Not in the translation units that hold only token-kernel instances and include this header for
// its device helpers: the kernel is defined once, with the graph path that launches it.)
#ifndef DZ_PTK_ONLY_TU
// One workgroup: pick the next token (host feed first, else argmax of the last logits),
// bump the position and write its embedding row (forward.rs:212-213).
__global__ __launch_bounds__(1024) void select_token_kernel(const SelectArgs a) {
  __shared__ float sv[16];
  __shared__ int si[16];
  __shared__ int tok_s;
  const unsigned tid = threadIdx.x;
  TokState* st = a.st;
  const bool fed = a.commit && st->feed_idx < st->feed_len;
  if (!fed) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = tid; i < a.n_am; i += blockDim.x)
      if (am_better(a.am_val[i], a.am_idx[i], bv, bi)) { bv = a.am_val[i]; bi = a.am_idx[i]; }
    wave_argmax(bv, bi);
    if ((tid & 63u) == 0) { sv[tid >> 6] = bv; si[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
      for (unsigned w = 1; w < blockDim.x / 64; ++w)
        if (am_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
      tok_s = bi == 0x7FFFFFFF ? 0 : bi;
    }
  } else if (tid == 0) {
    tok_s = a.feed[st->feed_idx];
  }
  __syncthreads();
  const int tok = tok_s;
  if (!a.commit) {
    if (tid == 0) a.toklog[st->pos_next] = tok;
    return;
  }
  __syncthreads();
  if (tid == 0) {
    if (fed) st->feed_idx += 1;
    st->pos = st->pos_next;
    st->pos_next += 1;
    st->token = tok;
    a.toklog[st->pos] = tok;
  }
  if (a.emb_f16) {
    // an F16 tensor converts element-wise with the reference's f16_to_f32 (Tensor::load_as_f32,
    // tensor/tensor.rs:62-76), subnormal handling included
    const uint16_t* row = a.emb_f16 + (size_t)tok * a.H;
    for (int64_t c = tid; c < a.H; c += blockDim.x) a.emb_out[c] = ref_f16_to_f32_dev(row[c]);
  } else {
    // dequantize_q1_0_row_into (quant.rs:161-194) from the GEMV layout
    const int64_t rb = tok / kRowBlock;
    const unsigned L = (unsigned)(tok % kRowBlock);
    for (int64_t k = tid; k < a.H; k += blockDim.x) {
      const int t = (int)(k / kTileCols);
      const unsigned p = (unsigned)((k % kTileCols) / 8), j = (unsigned)(k % 8), s = L ^ p;
      const uint8_t* u = a.emb_q1 + ((size_t)rb * a.emb_ntiles + t) * kUnitBytes;
      const unsigned byte = u[((s >> 4) * 64 + L) * 16 + (s & 15)];
      const uint16_t* scp = reinterpret_cast<const uint16_t*>(u + kUnitSignBytes);
      const float scale = ref_f16_to_f32_dev(scp[L * 4 + ((p >> 4) ^ (L >> 4))]);
      a.emb_out[k] = ((float)((byte >> j) & 1u) * 2.0f - 1.0f) * scale;
    }
  }
}
#endif

// ---------------------------------------------------------------- Gated DeltaNet step

struct DeltaArgs {
  const TokState* st;
  int pos;            // this token's position, or -1: TokState.pos (replays of the captured token graph)
  const float* p_in;  // in-proj partials [np][ldp]: rows [qkv | z | alpha | beta]
  int np;
  int64_t ldp;
  const float* ss;    // sums of squares of the layer input, per tile
  int nss;
  int64_t H;
  float rms_eps;
  float* conv;        // ring [4][qkvd]
  const int* ring_base_ptr;  // ring head at pos 0 (mod 4) of this layer
  const float* conv_w;  // [4][qkvd] (tap-major, tap 3 = newest)
  const float* ssm_a;   // [nvh]
  const float* dt_bias; // [nvh]
  float* state;         // [nvh][128 i][128 j] (row-major S[i][j])
  float* y;             // [nvh*128] raw readout
  float* zs;            // [nvh*128] silu(z)
  int nkh, nvh;
  int64_t qkvd, off_z, off_a, off_b;
};

// One workgroup per (v-head, quarter of its 128 rows); 256 threads = 32 rows x 8 slices of k.
// Follows ssm_forward_into (model/ssm.rs:465-574): conv ring + causal conv (kernel 4) + SiLU,
// per-head L2 norm of q/k, q *= 1/sqrt(128), g = A*softplus(alpha + dt_bias), decay = exp(g),
// beta = sigmoid(b), then for each state row i: s *= decay; kv = s.k; d = (v_i - kv)*beta;
// s += d*k; y_i = s.q.  k-head of v-head vh is vh % nkh (ssm.rs:558-561).
template <int NP>
__global__ __launch_bounds__(256) void deltanet_kernel(const DeltaArgs a) {
  constexpr int HD = 128;
  __shared__ float qs[HD], ks[HD], vs[32], red[16], part[8][32], dsh[32], sc[4];
  const unsigned tid = threadIdx.x;
  const int vh = blockIdx.x >> 2, quarter = blockIdx.x & 3, kh = vh % a.nkh;
  const int i_loc = tid & 31, js = tid >> 5;
  const int i = quarter * 32 + i_loc;
  const int pos = a.pos >= 0 ? a.pos : a.st->pos;
  const int hb = (*a.ring_base_ptr + pos) & 3;  // ring head before this token = slot of the new value
  const int64_t kdim = (int64_t)a.nkh * HD;
  const int64_t qkvd = a.qkvd;

  // ---- every global load first (one memory round trip) ----
  // state rows i, k-slice [16*js, 16*js+16)
  float* S = a.state + (size_t)vh * HD * HD + (size_t)i * HD + 16 * js;
  float s[16];
  state_row_load(S, s);
  const float inv = inv_rms_from(a.ss, a.nss, a.H, a.rms_eps);
  // conv channel of this thread: q (tid < 128) or k (tid >= 128) of k-head kh
  const int64_t ch = tid < HD ? (int64_t)kh * HD + tid : kdim + (int64_t)kh * HD + (tid - HD);
  const float xq = sum_strided<NP>(a.p_in, a.ldp, a.np, ch);
  const float r1 = a.conv[(size_t)((hb + 1) & 3) * qkvd + ch], r2 = a.conv[(size_t)((hb + 2) & 3) * qkvd + ch],
              r3 = a.conv[(size_t)((hb + 3) & 3) * qkvd + ch];
  const float w0 = a.conv_w[ch], w1 = a.conv_w[qkvd + ch], w2 = a.conv_w[2 * qkvd + ch], w3 = a.conv_w[3 * qkvd + ch];
  // second role: v channel (tid < 32), z (32..63), alpha (64), beta (65)
  int64_t row2 = -1;
  if (tid < 32) row2 = 2 * kdim + (int64_t)vh * HD + quarter * 32 + tid;
  else if (tid < 64) row2 = a.off_z + (int64_t)vh * HD + quarter * 32 + (tid - 32);
  else if (tid == 64) row2 = a.off_a + vh;
  else if (tid == 65) row2 = a.off_b + vh;
  float x2 = 0.f, v1 = 0.f, v2 = 0.f, v3 = 0.f, u0 = 0.f, u1 = 0.f, u2 = 0.f, u3 = 0.f;
  if (row2 >= 0) x2 = sum_strided<NP>(a.p_in, a.ldp, a.np, row2);
  if (tid < 32) {
    v1 = a.conv[(size_t)((hb + 1) & 3) * qkvd + row2];
    v2 = a.conv[(size_t)((hb + 2) & 3) * qkvd + row2];
    v3 = a.conv[(size_t)((hb + 3) & 3) * qkvd + row2];
    u0 = a.conv_w[row2]; u1 = a.conv_w[qkvd + row2]; u2 = a.conv_w[2 * qkvd + row2]; u3 = a.conv_w[3 * qkvd + row2];
  }
  float ssm_a = 0.f, dtb = 0.f;
  if (tid == 64) { ssm_a = a.ssm_a[vh]; dtb = a.dt_bias[vh]; }

  // ---- conv ring + causal conv (fma in tap order, oldest first) + SiLU (ssm.rs:467-518) ----
  const float xn = xq * inv;
  float o = 0.f;
  o = __builtin_fmaf(r1, w0, o);
  o = __builtin_fmaf(r2, w1, o);
  o = __builtin_fmaf(r3, w2, o);
  o = __builtin_fmaf(xn, w3, o);
  const float qk = siluf_(o);
  const bool owner = (vh < a.nkh) && quarter == 0;  // one writer per shared q/k ring channel
  if (owner) a.conv[(size_t)hb * qkvd + ch] = xn;
  const float x2n = x2 * inv;
  if (tid < 32) {
    float ov = 0.f;
    ov = __builtin_fmaf(v1, u0, ov);
    ov = __builtin_fmaf(v2, u1, ov);
    ov = __builtin_fmaf(v3, u2, ov);
    ov = __builtin_fmaf(x2n, u3, ov);
    vs[tid] = siluf_(ov);
    a.conv[(size_t)hb * qkvd + row2] = x2n;
  } else if (tid < 64) {
    a.zs[(size_t)vh * HD + quarter * 32 + (tid - 32)] = siluf_(x2n);
  } else if (tid == 64) {
    // g = A * softplus(alpha + dt_bias), decay = exp(g)  (ssm.rs:61-67, 163-166)
    const float x = x2n + dtb;
    const float sp = x > 20.0f ? x : logf(1.0f + expf(x));
    sc[0] = expf(ssm_a * sp);
  } else if (tid == 65) {
    sc[1] = sigmoidf_(x2n);  // beta = sigmoid(b)
  }
  // per-head L2 norms of q and k (ssm.rs:523-530): waves 0-1 hold q, waves 2-3 hold k
  const float s2 = wave_sum(qk * qk);
  if ((tid & 63u) == 0) red[tid >> 6] = s2;
  __syncthreads();
  if (tid < HD) {
    const float inq = 1.0f / sqrtf((red[0] + red[1]) + 1e-6f);
    qs[tid] = (qk * inq) * (1.0f / sqrtf((float)HD));
  } else {
    const float ink = 1.0f / sqrtf((red[2] + red[3]) + 1e-6f);
    ks[tid - HD] = qk * ink;
  }
  __syncthreads();

  // ---- gated delta rule on rows i (ssm.rs:378-418) ----
  const float decay = sc[0], beta = sc[1];
  float kvp = 0.f;
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    s[jj] *= decay;
    kvp = __builtin_fmaf(s[jj], ks[js * 16 + jj], kvp);
  }
  part[js][i_loc] = kvp;
  __syncthreads();
  if (js == 0) {
    float kv = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) kv += part[q][i_loc];
    dsh[i_loc] = (vs[i_loc] - kv) * beta;
  }
  __syncthreads();
  const float d = dsh[i_loc];
  float yp = 0.f;
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    const int j = js * 16 + jj;
    s[jj] = __builtin_fmaf(d, ks[j], s[jj]);
    yp = __builtin_fmaf(s[jj], qs[j], yp);
  }
  state_row_store(S, s);
  part[js][i_loc] = yp;  // the kv reads of part finished before the previous barrier
  __syncthreads();
  if (js == 0) {
    float yy = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) yy += part[q][i_loc];
    a.y[(size_t)vh * HD + i] = yy;
  }
}

// ---------------------------------------------------------------- gated GQA attention (split-K)

struct AttnArgs {
  const TokState* st;
  int pos;            // this token's position, or -1: TokState.pos (replays of the captured token graph)
  const float* p_in;  // qkv partials: rows [q+gate interleaved per head (n_head*2*hd) | k | v]
  int np;
  int64_t ldp;
  const float* ss;
  int nss;
  int64_t H;
  float eps;
  const float* q_norm;
  const float* k_norm;
  const float* rope;  // [max_ctx][rope_dim]: cos[0..half) sin[half..rope_dim)
  int rope_dim;
  float* kcache;      // [nkv][max_ctx][hd]
  float* vcache;
  int max_ctx;
  float* apart;       // [n_head][gmax][2+hd]
  int gmax;
  int nq, nkv;
};

// Workgroup (kv-head, chunk g) runs the online softmax of attention.rs:124-199 over positions
// [g*chunk, (g+1)*chunk) for the kv-head's n_head/n_kv query heads (grouped GQA: q-head
// kvh*grp + gi, attention.rs:163-165) and writes (m, l, o) per q-head.  q/k get RMSNorm with
// q_norm/k_norm, then the reference's partial RoPE on the first rope_dim dims with both terms
// added (rope.rs:205-208), and q *= 1/sqrt(hd).  The chunk holding the new position also appends
// its k/v to the cache.  hd = 256, 256 threads (4 waves).
template <int GRP, int NP>
__global__ __launch_bounds__(256) void attention_kernel(const AttnArgs a) {
  constexpr int HD = 256;
  __shared__ float qs[GRP][HD];
  __shared__ float kn[HD], vn[HD];
  __shared__ float red[GRP + 1][4];
  __shared__ float wm[4][GRP], wl[4][GRP];
  __shared__ float wo[4][GRP][HD];
  __shared__ float ew[4][GRP][16];
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const int kvh = blockIdx.x / a.gmax, g = blockIdx.x % a.gmax;
  const int P = a.pos >= 0 ? a.pos : a.st->pos, ctx = P + 1;
  const int chunk = attn_chunk(ctx, a.gmax);
  const int geff = (ctx + chunk - 1) / chunk;
  if (g >= geff) return;
  const int p0 = g * chunk, p1 = min(ctx, p0 + chunk);
  const bool has_new = p1 == ctx;
  // K rows and V rows of the cache, global loads only (so that waiting on LDS reads never waits on
  // them).  Tiles of 16 positions, wave w takes tiles w, w + 4, ...; the first tile's rows load
  // before the prologue unless the tile holds the new position, whose rows this workgroup stores
  // below (and reads after the barrier that follows).
  const float* kb = a.kcache + (size_t)kvh * a.max_ctx * HD;
  const float* vb = a.vcache + (size_t)kvh * a.max_ctx * HD;
  const int pj = (int)(lane >> 2), qtr = (int)(lane & 3u);
  constexpr int kT = 16;
  const int ntile = (p1 - p0 + kT - 1) / kT;
  float4 kk[16], vv[kT];
  auto load_k = [&](int t) {
    const int tp0 = p0 + kT * t;
    const int row = tp0 + pj < p1 ? tp0 + pj : tp0;
    const float4* kr = reinterpret_cast<const float4*>(kb + (size_t)row * HD) + qtr;
#pragma unroll
    for (int u = 0; u < 16; ++u) kk[u] = kr[4 * u];  // the quad reads 64 contiguous bytes per step
  };
  auto load_v = [&](int t) {
    const int tp0 = p0 + kT * t;
    const int npos = min(kT, p1 - tp0);
#pragma unroll
    for (int j = 0; j < kT; ++j)
      vv[j] = j < npos ? *reinterpret_cast<const float4*>(vb + (size_t)(tp0 + j) * HD + 4 * lane)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  const bool pre = (int)wave < ntile && p0 + kT * ((int)wave + 1) <= P;
  if (pre) {
    load_k((int)wave);
    load_v((int)wave);
  }
  const float inv = inv_rms_from(a.ss, a.nss, a.H, a.eps);
  const int half = a.rope_dim / 2;
  const float* cs = a.rope + (size_t)P * a.rope_dim;

  auto proj = [&](int64_t row) { return sum_strided<NP>(a.p_in, a.ldp, a.np, row) * inv; };
  // raw q of the group's heads, one dim per thread
  float qv[GRP];
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) qv[gi] = proj((int64_t)(kvh * GRP + gi) * 2 * HD + tid);
  float kvv = 0.f, vvv = 0.f;
  if (has_new) {
    kvv = proj((int64_t)a.nq * 2 * HD + (int64_t)kvh * HD + tid);
    vvv = proj((int64_t)a.nq * 2 * HD + (int64_t)a.nkv * HD + (int64_t)kvh * HD + tid);
  }
  // per-head RMSNorm over 256 dims (rmsnorm_inplace, rmsnorm.rs:158-176)
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    const float sq = wave_sum(qv[gi] * qv[gi]);
    if (lane == 0) red[gi][wave] = sq;
  }
  {
    const float sq = wave_sum(kvv * kvv);
    if (lane == 0) red[GRP][wave] = sq;
  }
  __syncthreads();
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    const float ssum = (red[gi][0] + red[gi][1]) + (red[gi][2] + red[gi][3]);
    const float in = 1.0f / sqrtf(ssum / (float)HD + a.eps);
    qs[gi][tid] = (qv[gi] * in) * a.q_norm[tid];
  }
  if (has_new) {
    const float ssum = (red[GRP][0] + red[GRP][1]) + (red[GRP][2] + red[GRP][3]);
    const float in = 1.0f / sqrtf(ssum / (float)HD + a.eps);
    kn[tid] = (kvv * in) * a.k_norm[tid];
    vn[tid] = vvv;
  }
  __syncthreads();
  // RoPE on dims [0, rope_dim): pairs (d, d+half); thread d < half rotates the pair
  float r1[GRP], r2[GRP];
  float kr1 = 0.f, kr2 = 0.f;
  if ((int)tid < half) {
    const float c = cs[tid], sn = cs[half + tid];
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      const float x1 = qs[gi][tid], x2 = qs[gi][tid + half];
      r1[gi] = __builtin_fmaf(x1, c, x2 * sn);
      r2[gi] = __builtin_fmaf(x2, c, x1 * sn);
    }
    if (has_new) {
      const float x1 = kn[tid], x2 = kn[tid + half];
      kr1 = __builtin_fmaf(x1, c, x2 * sn);
      kr2 = __builtin_fmaf(x2, c, x1 * sn);
    }
  }
  __syncthreads();
  if ((int)tid < half) {
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      qs[gi][tid] = r1[gi];
      qs[gi][tid + half] = r2[gi];
    }
    if (has_new) {
      kn[tid] = kr1;
      kn[tid + half] = kr2;
    }
  }
  __syncthreads();
  const float qscale = 1.0f / sqrtf((float)HD);
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) qs[gi][tid] *= qscale;
  if (has_new) {
    a.kcache[((size_t)kvh * a.max_ctx + P) * HD + tid] = kn[tid];
    a.vcache[((size_t)kvh * a.max_ctx + P) * HD + tid] = vn[tid];
  }
  __syncthreads();

  // Online softmax over this wave's tiles.  Scores: the four lanes 4j .. 4j+3 hold position tp0 + j,
  // lane 4j+r the float4 columns r, r+4, ..., r+60 of its K row; they dot them with the same
  // columns of q (from LDS) and add the four within the quad; one softmax update per tile.
  // Values: lane j holds dims 4j .. 4j+3 and sums the tile's V rows weighted by the exp-scores,
  // read back from LDS.  The next tile's K rows load during this tile's softmax and values, its V
  // rows during the next tile's scores.  l is kept per position lane (quarter 0) until the end.
  float m[GRP], l[GRP];
  float4 o[GRP];
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    m[gi] = -INFINITY;
    l[gi] = 0.f;
    o[gi] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float(*es)[16] = ew[wave];
  if ((int)wave < ntile && !pre) {
    load_k((int)wave);
    load_v((int)wave);
  }
  for (int t = (int)wave; t < ntile; t += 4) {
    const int tp0 = p0 + kT * t;
    const int npos = min(kT, p1 - tp0);
    const bool valid = pj < npos;
    float sc[GRP];
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      float d = 0.f;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float4 q = *reinterpret_cast<const float4*>(&qs[gi][16 * u + 4 * qtr]);
        d = __builtin_fmaf(q.x, kk[u].x, d);
        d = __builtin_fmaf(q.y, kk[u].y, d);
        d = __builtin_fmaf(q.z, kk[u].z, d);
        d = __builtin_fmaf(q.w, kk[u].w, d);
      }
      d = dpp_add<0xB1>(d);  // quad_perm [1,0,3,2]
      sc[gi] = dpp_add<0x4E>(d);  // quad_perm [2,3,0,1]: every lane of the quad has the sum
    }
    if (t + 4 < ntile) load_k(t + 4);
#pragma unroll
    for (int gi = 0; gi < GRP; ++gi) {
      const float sv = valid ? sc[gi] : -INFINITY;
      const float mn = fmaxf(m[gi], wave_max(sv));
      const float al = expf(m[gi] - mn);
      const float e = valid ? expf(sv - mn) : 0.f;
      l[gi] = __builtin_fmaf(l[gi], al, qtr == 0 ? e : 0.f);
      o[gi].x *= al;
      o[gi].y *= al;
      o[gi].z *= al;
      o[gi].w *= al;
      m[gi] = mn;
      if (qtr == 0) es[gi][pj] = e;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j4 = 0; j4 < kT; j4 += 4) {
      if (j4 < npos) {
#pragma unroll
        for (int gi = 0; gi < GRP; ++gi) {
          const float4 e4 = *reinterpret_cast<const float4*>(&es[gi][j4]);
          const float ee[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float4 v = vv[j4 + r];
            o[gi].x = __builtin_fmaf(ee[r], v.x, o[gi].x);
            o[gi].y = __builtin_fmaf(ee[r], v.y, o[gi].y);
            o[gi].z = __builtin_fmaf(ee[r], v.z, o[gi].z);
            o[gi].w = __builtin_fmaf(ee[r], v.w, o[gi].w);
          }
        }
      }
    }
    if (t + 4 < ntile) load_v(t + 4);
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) l[gi] = wave_sum(l[gi]);
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    if (lane == 0) {
      wm[wave][gi] = m[gi];
      wl[wave][gi] = l[gi];
    }
    *reinterpret_cast<float4*>(&wo[wave][gi][4 * lane]) = o[gi];
  }
  __syncthreads();
  // merge the 4 waves (a wave without positions has l = 0) and write each q-head's chunk record
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    float M = -INFINITY;
    for (int w = 0; w < 4; ++w) M = fmaxf(M, wm[w][gi]);
    float L = 0.f, O = 0.f;
    for (int w = 0; w < 4; ++w) {
      const float e = wl[w][gi] > 0.f ? expf(wm[w][gi] - M) : 0.f;
      L = __builtin_fmaf(wl[w][gi], e, L);
      O = __builtin_fmaf(wo[w][gi][tid], e, O);
    }
    float* rec = a.apart + ((size_t)(kvh * GRP + gi) * a.gmax + g) * (2 + HD);
    if (tid == 0) {
      rec[0] = M;
      rec[1] = L;
    }
    rec[2 + tid] = O;
  }
}

// h = h_in + sum_k part_k tile by tile with the tile's sum of squares (the output norm's input).
struct FinalArgs {
  const float* h_in;
  const float* part;
  int np;
  int64_t ldp;
  float* h_out;
  float* ss_out;
  int64_t H;
  TokState* st = nullptr;  // when set, TokState.pos / pos_next become pos / pos + 1 (a direct mixer step)
  int pos = 0;
};

template <int NP>
__global__ __launch_bounds__(512) void final_reduce_kernel(const FinalArgs a) {
  __shared__ float red[16];
  const int t = blockIdx.x;
  const unsigned tid = threadIdx.x;
  const int64_t col = (int64_t)t * kTileCols + tid;
  float v = 0.f;
  if (col < a.H) {
    const float d = sum_strided<NP>(a.part, a.ldp, a.np, col);
    v = a.h_in[col] + d;
    a.h_out[col] = v;
  }
  const float s = block_sum(v * v, red, tid, 512);
  if (tid == 0) a.ss_out[t] = s;
  if (a.st && t == 0 && tid == 0) {
    a.st->pos = a.pos;
    a.st->pos_next = a.pos + 1;
  }
}

}  // namespace dz
