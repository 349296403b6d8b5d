// batch_kernels.h — the n-token forward (forward_batch, Daiza-engine/src/model/forward.rs:394-1407)
// outside the projections, which run on the matrix cores (q1_gemm.h).  Activations are token-major
// [n][width] f32.  Used for prefill (dz_forward_batch) and for speculative verify, where the
// DeltaNet scan records what a rollback needs instead of writing the state back.
#pragma once
#include "model_kernels.h"

namespace dz {

// The 8-lane sum of v within each aligned group of 8 lanes (quad xor 1, quad xor 2, half-row
// mirror); every lane of the group gets it.
__device__ __forceinline__ float lane8_sum(float v) {
  v = dpp_add<0xB1>(v);
  v = dpp_add<0x4E>(v);
  v = dpp_add<0x141>(v);
  return v;
}

// h[t] = embedding row of ids[t] (forward.rs:212): the f16 table through the reference's
// f16_to_f32 (tensor/tensor.rs:62-76), or a Q1_0 table through dequantize_q1_0_row_into
// (quant.rs:161-194).  Grid n, 256 threads.
__global__ __launch_bounds__(256) void bt_embed_kernel(const int* __restrict__ ids, int64_t H,
                                                       const uint16_t* __restrict__ emb_f16,
                                                       const uint8_t* __restrict__ emb_q1, int emb_ntiles,
                                                       float* __restrict__ h) {
  const int t = blockIdx.x;
  const int tok = ids[t];
  float* out = h + (size_t)t * H;
  if (emb_f16) {
    const uint16_t* row = emb_f16 + (size_t)tok * H;
    for (int64_t c = threadIdx.x; c < H; c += 256) out[c] = ref_f16_to_f32_dev(row[c]);
    return;
  }
  const int64_t rb = tok / kRowBlock;
  const unsigned L = (unsigned)(tok % kRowBlock);
  for (int64_t k = threadIdx.x; k < H; k += 256) {
    const int tt = (int)(k / kTileCols);
    const unsigned p = (unsigned)((k % kTileCols) / 8), j = (unsigned)(k % 8), s = L ^ p;
    const uint8_t* u = emb_q1 + ((size_t)rb * emb_ntiles + tt) * kUnitBytes;
    const unsigned byte = u[((s >> 4) * 64 + L) * 16 + (s & 15)];
    const uint16_t* scp = reinterpret_cast<const uint16_t*>(u + kUnitSignBytes);
    const float scale = ref_f16_to_f32_dev(scp[L * 4 + ((p >> 4) ^ (L >> 4))]);
    out[k] = ((float)((byte >> j) & 1u) * 2.0f - 1.0f) * scale;
  }
}

// Causal conv over the chunk + SiLU (ssm.rs:467-518): out[t][ch] = silu(Σ_tap x[t-3+tap][ch]·w[tap][ch]),
// fma in tap order (oldest first), x[t'] = in-proj output of token t' for t' >= 0 and the conv
// ring's entry for the earlier tokens (the token at chunk offset t' < 0 sits in slot
// (head0 + t') & 3, head0 = slot of token 0).  Thread per (token, channel).  keep (verify, else null)
// receives the conv inputs themselves, keep[t][ch] = x[t][ch], from which the commit rebuilds the ring.
// The q and k channels (the first 2 nkh·128, whole heads per workgroup: 2 nkh·128 is a multiple of
// 256) also get their per-head L2 norm (l2norm_inplace, ssm.rs:76-135; q additionally times
// 1/sqrt(128), ssm.rs:532-533) into qk[t][0 .. 2 nkh·128): a head is two whole waves of the workgroup.
__global__ __launch_bounds__(256) void bt_conv_kernel(const float* __restrict__ yin, int64_t ldin, int n,
                                                      const float* __restrict__ ring, int head0,
                                                      const float* __restrict__ conv_w, int64_t qkvd,
                                                      float* __restrict__ cout, float* __restrict__ keep, int nkh,
                                                      float* __restrict__ qk) {
  __shared__ float red[4];
  const unsigned tid = threadIdx.x;
  const int64_t ch = (int64_t)blockIdx.x * 256 + tid;
  const int t = blockIdx.y;
  const bool live = ch < qkvd && t < n;
  float o = 0.f, xt = 0.f;
  if (live) {
    // every tap's input and weight requested before the sums (the address is selected, not the
    // load: a load under a branch waits for the loads before it)
    float xs[4], ws[4];
#pragma unroll
    for (int tap = 0; tap < 4; ++tap) {
      const int tt = t - 3 + tap;
      const float* src = tt >= 0 ? yin + (size_t)tt * ldin + ch : ring + (size_t)((head0 + tt) & 3) * qkvd + ch;
      xs[tap] = *src;
      ws[tap] = conv_w[(size_t)tap * qkvd + ch];
    }
    __builtin_amdgcn_sched_barrier(0);  // all eight loads issued before the first sum waits for one
#pragma unroll
    for (int tap = 0; tap < 4; ++tap) o = __builtin_fmaf(xs[tap], ws[tap], o);
    xt = xs[3];
  }
  const float v = siluf_(o);
  if (live) {
    cout[(size_t)t * qkvd + ch] = v;
    if (keep) keep[(size_t)t * qkvd + ch] = xt;
  }
  const int64_t kdim = (int64_t)nkh * 128;
  if ((int64_t)blockIdx.x * 256 >= 2 * kdim) return;  // a v-channel workgroup (uniform)
  const float sq = wave_sum(v * v);
  if ((tid & 63u) == 0) red[tid >> 6] = sq;
  __syncthreads();
  const int hw = (int)(tid >> 7) * 2;  // this head's first wave
  const float inv = 1.0f / sqrtf((red[hw] + red[hw + 1]) + 1e-6f);
  if (live) qk[(size_t)t * 2 * kdim + ch] = ch < kdim ? (v * inv) * (1.0f / sqrtf(128.0f)) : v * inv;
}

// Conv ring after tokens [0, t1) of a chunk: the inputs of tokens [t0, t1) (t0 = max(0, t1 - 4))
// go to their slots (head0 + t) & 3 (ssm.rs:467-470).
__global__ __launch_bounds__(256) void bt_ring_kernel(const float* __restrict__ yin, int64_t ldin, int t0, int t1,
                                                      float* __restrict__ ring, int head0, int64_t qkvd) {
  const int64_t ch = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (ch >= qkvd) return;
  for (int t = t0; t < t1; ++t) ring[(size_t)((head0 + t) & 3) * qkvd + ch] = yin[(size_t)t * ldin + ch];
}

// Rollback record of a verify chunk for one DeltaNet layer: the decay and the delta of every token
// (the rank-1 update S <- decay·S + d ⊗ k) and the token's key; replaying the first a of them
// reproduces the state after a tokens bit for bit.
struct DnRecord {
  float* decay;  // [n][nvh]
  float* d;      // [n][nvh * 128]
  float* k;      // [n][nkh * 128]
};

// Gated delta rule over the chunk's tokens in order (ssm_scan_vhead, ssm.rs:153-180; fused form
// 378-418).  Workgroup (v-head vh, quarter) holds state rows i = quarter·32 + (tid >> 3),
// columns j = 16·(tid & 7) .. +16 of S[vh][i][j] in registers (64 contiguous bytes per thread); the 8
// threads of a row sum with DPP.
// Per token: g = ssm_a·softplus(alpha + dt_bias), decay = exp(g), beta = sigmoid(b); s *= decay;
// kv = s·k; d = (v_i - kv)·beta; s += d·k; y_i = s·q.  The inputs of 16 tokens at a time (q and k
// of the k-head, v of the workgroup's rows, alpha, beta) are staged in LDS by the whole workgroup,
// the next 16 requested while these compute: one load latency per 16 tokens instead of one per
// token.  With rec == null the state is written back at the end; otherwise it is left as it was
// and every token's (decay, d, k) is recorded.
__global__ __launch_bounds__(256) void bt_scan_kernel(const float* __restrict__ yin, int64_t ldin,
                                                      const float* __restrict__ cout, int64_t qkvd,
                                                      const float* __restrict__ qk, int n, int nkh, int nvh,
                                                      int64_t off_a, int64_t off_b, const float* __restrict__ ssm_a,
                                                      const float* __restrict__ dt_bias, float* __restrict__ state,
                                                      float* __restrict__ y, DnRecord rec) {
  constexpr int HD = 128, G = 16;
  __shared__ __align__(16) float sqk[G][2 * HD];  // token's q then k of this k-head
  __shared__ float sv[G][32], sab[G][2];
  const unsigned tid = threadIdx.x;
  const int vh = blockIdx.x >> 2, quarter = blockIdx.x & 3, kh = vh % nkh;
  const int i = quarter * 32 + (int)(tid >> 3), js = (int)(tid & 7u);
  const int64_t kdim = (int64_t)nkh * HD;
  float* S = state + (size_t)vh * HD * HD + (size_t)i * HD + 16 * js;
  float s[16];
  state_row_load(S, s);
  const float A = ssm_a[vh], dtb = dt_bias[vh];
  // staging of tokens [g0, g0 + G): thread (tt = tid >> 4, part = tid & 15) takes 16 of token tt's
  // 256 q|k values, 2 of its v rows, and (tid < 32) one alpha or beta
  // (the staged values are returned by value and kept in named registers: held in an array
  // captured by a lambda, they went to scratch memory, one wait per load)
  const int st = (int)(tid >> 4), sp = (int)(tid & 15u);
  struct Stage {
    float4 q0, q1, q2, q3;
    float v0, v1, ab;
  };
  auto gload = [&](int g0) -> Stage {
    const int t = min(g0 + st, n - 1);
    const float* src = qk + (size_t)t * 2 * kdim + (sp < 8 ? (size_t)kh * HD + 16 * sp : kdim + (size_t)kh * HD + 16 * (sp - 8));
    const float* vr = cout + (size_t)t * qkvd + 2 * kdim + (int64_t)vh * HD + quarter * 32 + 2 * sp;
    // every thread loads alpha or beta (a valid address) and tid < 32 keep it: a load under a
    // branch waits for the loads before it
    const int ta = min(g0 + (int)(tid & 15u), n - 1);
    Stage r;
    r.q0 = *reinterpret_cast<const float4*>(src);
    r.q1 = *reinterpret_cast<const float4*>(src + 4);
    r.q2 = *reinterpret_cast<const float4*>(src + 8);
    r.q3 = *reinterpret_cast<const float4*>(src + 12);
    r.v0 = vr[0];
    r.v1 = vr[1];
    r.ab = yin[(size_t)ta * ldin + ((tid & 16u) ? off_b : off_a) + vh];
    return r;
  };
  auto gstore = [&](const Stage& r) {
    float4* dq = reinterpret_cast<float4*>(&sqk[st][16 * sp]);
    dq[0] = r.q0;
    dq[1] = r.q1;
    dq[2] = r.q2;
    dq[3] = r.q3;
    sv[st][2 * sp] = r.v0;
    sv[st][2 * sp + 1] = r.v1;
    if (tid < 32) sab[tid & 15u][tid >> 4] = r.ab;
  };
  Stage nx = gload(0);
  gstore(nx);
  __syncthreads();
  for (int g0 = 0; g0 < n; g0 += G) {
    const bool more = g0 + G < n;
    if (more) nx = gload(g0 + G);
    const int gn = min(G, n - g0);
    for (int tt = 0; tt < gn; ++tt) {
      const int t = g0 + tt;
      const float x = sab[tt][0] + dtb;
      const float spl = x > 20.0f ? x : logf(1.0f + expf(x));
      const float decay = expf(A * spl);
      const float beta = sigmoidf_(sab[tt][1]);
      float kf[16], qf[16];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 q4 = *reinterpret_cast<const float4*>(&sqk[tt][16 * js + 4 * c]);
        const float4 k4 = *reinterpret_cast<const float4*>(&sqk[tt][HD + 16 * js + 4 * c]);
        qf[4 * c] = q4.x; qf[4 * c + 1] = q4.y; qf[4 * c + 2] = q4.z; qf[4 * c + 3] = q4.w;
        kf[4 * c] = k4.x; kf[4 * c + 1] = k4.y; kf[4 * c + 2] = k4.z; kf[4 * c + 3] = k4.w;
      }
      float kvp = 0.f;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        s[jj] *= decay;
        kvp = __builtin_fmaf(s[jj], kf[jj], kvp);
      }
      const float kv = lane8_sum(kvp);
      const float d = (sv[tt][i & 31] - kv) * beta;
      float yp = 0.f;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        s[jj] = __builtin_fmaf(d, kf[jj], s[jj]);
        yp = __builtin_fmaf(s[jj], qf[jj], yp);
      }
      const float yy = lane8_sum(yp);
      if (js == 0) {
        y[(size_t)t * nvh * HD + (int64_t)vh * HD + i] = yy;
        if (rec.d) rec.d[(size_t)t * nvh * HD + (int64_t)vh * HD + i] = d;
      }
      if (rec.d && tid == 0) rec.decay[(size_t)t * nvh + vh] = decay;
      if (rec.d && vh < nkh && quarter == 0 && js == 0) {
        // the key of k-head vh, written once: rows i < 32 of quarter 0 cover 32 of its 128 columns x 4
#pragma unroll
        for (int c = 0; c < 4; ++c) rec.k[(size_t)t * kdim + (int64_t)vh * HD + 4 * (i & 31) + c] = sqk[tt][HD + 4 * (i & 31) + c];
      }
    }
    if (more) {
      __syncthreads();  // every thread is done with this group's inputs
      gstore(nx);
      __syncthreads();
    }
  }
  if (!rec.d) state_row_store(S, s);
}

// Applies the first a recorded tokens of a verify chunk to the state: s = decay·s, s = fma(d, k, s)
// per token, the same operations in the same order as the scan, so the result equals a scan over
// those a tokens.  Grid 4·nvh, 256 threads (the scan's row mapping).
__global__ __launch_bounds__(256) void bt_commit_state_kernel(float* __restrict__ state, DnRecord rec, int a, int nkh,
                                                              int nvh) {
  constexpr int HD = 128;
  const unsigned tid = threadIdx.x;
  const int vh = blockIdx.x >> 2, quarter = blockIdx.x & 3, kh = vh % nkh;
  const int i = quarter * 32 + (int)(tid >> 3), js = (int)(tid & 7u);
  float* S = state + (size_t)vh * HD * HD + (size_t)i * HD + 16 * js;
  float s[16];
  state_row_load(S, s);
  for (int t = 0; t < a; ++t) {
    const float decay = rec.decay[(size_t)t * nvh + vh];
    const float d = rec.d[(size_t)t * nvh * HD + (int64_t)vh * HD + i];
    const float* kr = rec.k + (size_t)t * nkh * HD + (size_t)kh * HD + 16 * js;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) s[jj] *= decay;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) s[jj] = __builtin_fmaf(d, kr[jj], s[jj]);
  }
  state_row_store(S, s);
}

// Output gate per v-head (ssm_output_gate_avx2, ssm.rs:246-286):
// g[t][vh·128 + i] = ((y·(1/sqrt(Σy²/128 + eps)))·w_norm[i])·silu(z).  Grid (n, nvh), 128 threads.
__global__ __launch_bounds__(128) void bt_gate_y_kernel(const float* __restrict__ y, const float* __restrict__ yin,
                                                        int64_t ldin, int64_t off_z, const float* __restrict__ nw,
                                                        float eps, int nvh, float* __restrict__ g) {
  __shared__ float red[2];
  const int t = blockIdx.x, vh = blockIdx.y;
  const unsigned tid = threadIdx.x;
  const int64_t col = (int64_t)vh * 128 + tid;
  const float v = y[(size_t)t * nvh * 128 + col];
  const float z = yin[(size_t)t * ldin + off_z + col];  // requested with y: one memory round trip
  const float w = nw[tid];
  const float s = wave_sum(v * v);
  if ((tid & 63u) == 0) red[tid >> 6] = s;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[0] + red[1]) * (1.0f / 128.0f) + eps);
  g[(size_t)t * nvh * 128 + col] = ((v * inv) * w) * siluf_(z);
}

// Attention inputs of token t at position pos0 + t (attention.rs:87-123): per q-head RMSNorm
// (q_norm), the reference's partial RoPE (pairs (d, d + rope_dim/2) on d < rope_dim/2, both terms
// added: rope.rs:205-208), q·1/sqrt(256) -> qb[t][h]; the gate half -> gate[t][h]; per kv-head the
// same for k (k_norm, no scale) appended to the cache with v.  Grid (n, nq + nkv), 256 threads.
__global__ __launch_bounds__(256) void bt_attn_prep_kernel(const float* __restrict__ yin, int64_t ldin, int nq,
                                                           int nkv, const float* __restrict__ q_norm,
                                                           const float* __restrict__ k_norm, float eps,
                                                           const float* __restrict__ rope, int rope_dim, int pos0,
                                                           float* __restrict__ qb, float* __restrict__ gate,
                                                           float* __restrict__ kcache, float* __restrict__ vcache,
                                                           int max_ctx) {
  constexpr int HD = 256;
  __shared__ float xs[HD];
  __shared__ float red[4];
  const int t = blockIdx.x, hh = blockIdx.y;
  const unsigned tid = threadIdx.x;
  const float* row = yin + (size_t)t * ldin;
  const bool isq = hh < nq;
  const int kvh = hh - nq;
  const float raw = isq ? row[(size_t)hh * 2 * HD + tid] : row[(size_t)nq * 2 * HD + (size_t)kvh * HD + tid];
  // the gate (q-head) or v (kv-head) value of this dim, the norm weight and the RoPE factors,
  // requested with raw: one memory round trip
  const float other = isq ? row[(size_t)hh * 2 * HD + HD + tid] : row[(size_t)nq * 2 * HD + (size_t)nkv * HD + (size_t)kvh * HD + tid];
  const float nwt = isq ? q_norm[tid] : k_norm[tid];
  const int half = rope_dim / 2;
  const int pos = pos0 + t;
  const int dd = (int)tid < half ? (int)tid : (int)tid - half;
  const bool rot = (int)tid < rope_dim;
  const float* cs = rope + (size_t)pos * rope_dim;
  const float c = rot ? cs[dd] : 0.f, sn = rot ? cs[half + dd] : 0.f;
  const float s = wave_sum(raw * raw);
  if ((tid & 63u) == 0) red[tid >> 6] = s;
  __syncthreads();
  const float ssum = (red[0] + red[1]) + (red[2] + red[3]);
  const float in = 1.0f / sqrtf(ssum / (float)HD + eps);
  xs[tid] = (raw * in) * nwt;
  __syncthreads();
  float v = xs[tid];
  if (rot) {
    const float x1 = xs[dd], x2 = xs[dd + half];
    v = (int)tid < half ? __builtin_fmaf(x1, c, x2 * sn) : __builtin_fmaf(x2, c, x1 * sn);
  }
  if (isq) {
    qb[((size_t)t * nq + hh) * HD + tid] = v * (1.0f / sqrtf((float)HD));
    gate[((size_t)t * nq + hh) * HD + tid] = other;
  } else {
    kcache[((size_t)kvh * max_ctx + pos) * HD + tid] = v;
    vcache[((size_t)kvh * max_ctx + pos) * HD + tid] = other;
  }
}

// Causal GQA attention of tokens t0 .. t0+TPW-1 (positions pos0 + t) over cache positions
// [0, pos0 + t] for the GRP q-heads of kv-head kvh (online softmax, attention.rs:149-199), then
// o·sigmoid(gate) (attention.rs:202-203) -> ao[t][h·256 ..].  The TPW tokens of a workgroup share
// every cache row it reads (R = TPW·GRP query rows).  The 4 waves take blocks of 64 positions in turn
// with their own running (m, l, o) per row and are merged at the end.  Grid (ceil(n/TPW), nkv, nch),
// 256 threads: with nch > 1 workgroup z takes positions [z·csz, (z+1)·csz) and writes its record
// (m, l, o[256]) per (token, q-head) to rec[t][h][z] for bt_attn_merge_kernel instead.
template <int GRP, int TPW>
__global__ __launch_bounds__(256) void bt_attn_kernel(const float* __restrict__ qb, const float* __restrict__ gate,
                                                      const float* __restrict__ kcache,
                                                      const float* __restrict__ vcache, int max_ctx, int nq,
                                                      int pos0, int n, float* __restrict__ ao, int csz,
                                                      float* __restrict__ rec, int n_xcd, int nkv_x, int nch_x) {
  constexpr int HD = 256, BP = 64, R = TPW * GRP;
  // the query rows and block probabilities during the walk; the waves' (o) for the final merge after
  // it, in the same memory
  constexpr int kWalk = (R * HD + 4 * R * BP) * 4, kMerge = 4 * R * HD * 4;
  __shared__ __align__(16) unsigned char buf[kWalk > kMerge ? kWalk : kMerge];
  __shared__ float wm[4][R], wl[4][R];
  float(*qs)[HD] = reinterpret_cast<float(*)[HD]>(buf);
  float(*ps)[R][BP] = reinterpret_cast<float(*)[R][BP]>(buf + R * HD * 4);
  float(*wo)[R][HD] = reinterpret_cast<float(*)[R][HD]>(buf);
  int tg, kvh, z, nch;
  if (n_xcd > 0) {
    // 1-D grid: workgroup L runs on XCD L % 8 (round-robin dispatch); the token groups of one
    // (kv-head, chunk) pair get indices with the same residue, so the chunk's cache rows are fetched
    // into one XCD's L2 and read there once per group, instead of once per XCD
    const int L = (int)blockIdx.x, u = L >> 3, pair = (u / n_xcd) * 8 + (L & 7);
    if (pair >= nkv_x * nch_x) return;
    tg = u % n_xcd;
    kvh = pair % nkv_x;
    z = pair / nkv_x;
    nch = nch_x;
  } else {
    tg = (int)blockIdx.x;
    kvh = (int)blockIdx.y;
    z = (int)blockIdx.z;
    nch = (int)gridDim.z;
  }
  const int t0 = tg * TPW, nt = min(TPW, n - t0);
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const int pbeg = nch > 1 ? z * csz : 0;
  const int pend = nch > 1 ? (z + 1) * csz : 0x7FFFFFFF;
  int ctxt[TPW];  // positions visible to each token within this chunk: [pbeg, ctxt)
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) ctxt[tt] = tt < nt ? min(pos0 + t0 + tt + 1, pend) : pbeg;
  const int ctx = ctxt[nt - 1];  // the group's last token sees the most
  for (int i = (int)tid; i < R * HD; i += 256) {
    const int r = i / HD, tt = r / GRP, gi = r % GRP;
    qs[r][i % HD] = tt < nt ? qb[((size_t)(t0 + tt) * nq + kvh * GRP + gi) * HD + i % HD] : 0.f;
  }
  __syncthreads();
  const float* kb = kcache + (size_t)kvh * max_ctx * HD;
  const float* vb = vcache + (size_t)kvh * max_ctx * HD;
  float m[R], l[R];
  float4 o[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
    o[r] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // Blocks of 64 positions, wave w taking blocks w, w+4, ...  Scores: lane = position, each lane
  // walks its key row against the query rows in LDS (a broadcast read), so a score costs 256 FMAs in
  // one lane instead of a 64-lane reduction per (position, row).  (Four lanes per position, each
  // reading a quarter of the row so that a load touches 16 rows instead of 64, measured slower here:
  // 119 against 83 us per layer at context 8192.)  Values: lane = 4 dims, walking the block's
  // positions with their probabilities from LDS.
  for (int b0 = pbeg + (int)wave * BP; b0 < ctx; b0 += 4 * BP) {
    const int pp = b0 + (int)lane;
    const float* kr = kb + (size_t)(pp < ctx ? pp : b0) * HD;
    float sc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) sc[r] = 0.f;
#pragma unroll 4
    for (int j = 0; j < HD / 4; ++j) {
      const float4 k4 = *reinterpret_cast<const float4*>(kr + 4 * j);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float4 q4 = *reinterpret_cast<const float4*>(&qs[r][4 * j]);
        float d = sc[r];
        d = __builtin_fmaf(q4.x, k4.x, d);
        d = __builtin_fmaf(q4.y, k4.y, d);
        d = __builtin_fmaf(q4.z, k4.z, d);
        sc[r] = __builtin_fmaf(q4.w, k4.w, d);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool valid = pp < ctxt[r / GRP];
      const float x = valid ? sc[r] : -INFINITY;
      const float mn = fmaxf(m[r], wave_max(x));
      // a row with no visible position yet keeps m = -inf: its factors are 0 and 1 by definition
      const float al = mn == -INFINITY ? 1.0f : expf(m[r] - mn);
      const float pr = valid ? expf(x - mn) : 0.f;
      l[r] = l[r] * al + wave_sum(pr);
      o[r].x *= al;
      o[r].y *= al;
      o[r].z *= al;
      o[r].w *= al;
      m[r] = mn;
      ps[wave][r][lane] = pr;
    }
    // the other lanes' probabilities of this wave (LDS accesses of one wave complete in order)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    const int np = min(BP, ctx - b0);
#pragma unroll 4
    for (int pi = 0; pi < np; ++pi) {
      const float4 v4 = *reinterpret_cast<const float4*>(vb + (size_t)(b0 + pi) * HD + 4 * lane);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float pr = ps[wave][r][pi];
        o[r].x = __builtin_fmaf(pr, v4.x, o[r].x);
        o[r].y = __builtin_fmaf(pr, v4.y, o[r].y);
        o[r].z = __builtin_fmaf(pr, v4.z, o[r].z);
        o[r].w = __builtin_fmaf(pr, v4.w, o[r].w);
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();  // this block's reads of ps before the next block's writes
  }
  __syncthreads();  // every wave is done with qs and ps: the merge buffer reuses them
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (lane == 0) {
      wm[wave][r] = m[r];
      wl[wave][r] = l[r];
    }
    *reinterpret_cast<float4*>(&wo[wave][r][4 * lane]) = o[r];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int tt = r / GRP, gi = r % GRP;
    if (tt >= nt) continue;
    const int t = t0 + tt;
    float M = -INFINITY;
    for (int w = 0; w < 4; ++w)
      if (wl[w][r] > 0.f) M = fmaxf(M, wm[w][r]);
    float L = 0.f, O = 0.f;
    for (int w = 0; w < 4; ++w) {
      const float e = wl[w][r] > 0.f ? expf(wm[w][r] - M) : 0.f;
      L = __builtin_fmaf(wl[w][r], e, L);
      O = __builtin_fmaf(wo[w][r][tid], e, O);
    }
    const int h = kvh * GRP + gi;
    if (nch > 1) {
      float* rr = rec + (((size_t)t * nq + h) * nch + z) * (2 + HD);
      if (tid == 0) {
        rr[0] = M;
        rr[1] = L;
      }
      rr[2 + tid] = O;
    } else {
      const float gt = gate[((size_t)t * nq + h) * HD + tid];
      ao[((size_t)t * nq + h) * HD + tid] = (O * (1.0f / L)) * sigmoidf_(gt);
    }
  }
}

// Causal GQA attention of few tokens on the matrix cores, f32 operands (v_mfma_f32_16x16x4_f32: the
// products and sums are f32, in another order than the reference's loop, attention.rs:149-203).
// The n·GRP (token, q-head) rows of kv-head kvh, row ρ = t·GRP + g, are one matrix: wave w holds
// rows 16w .. 16w+15 (n·GRP <= 64), so each cache row is read by one workgroup for every token.
// Workgroup (z, kvh) takes positions [z·csz, (z+1)·csz) in blocks of 16 and writes the record
// (m, l, o[256]) of each row to rec[t][h][z] for bt_attn_merge_kernel.  Per block:
//   S^T = K_blk · Q^T: A = K rows (lane = position p0 + (lane & 15), dims 16j + 4(lane >> 4) + c
//   in step 4j + c), B = the same dims of the wave's Q rows (registers); the result leaves lane
//   (r, k) the scores of row 16w + r at positions p0 + 4k + i, so the online softmax of a row runs
//   in the 4 lanes r, r+16, r+32, r+48, and those probabilities are already the A operand of
//   O += P · V_blk in position order 4k + s (step s): no transpose through LDS.
//   B of step s, tile (th, c): V[p0 + 4k + s][64th + 4r + c]; O tile (th, c) leaves lane (r, k)
//   rows 16w + 4k + i at dim 64th + 4r + c.
// Grid (nch, nkv), 256 threads, no LDS.
template <int GRP>
__global__ __launch_bounds__(256) void bt_attn_mfma_kernel(const float* __restrict__ qb, const float* __restrict__ kcache,
                                                           const float* __restrict__ vcache, int max_ctx, int nq,
                                                           int pos0, int n, int csz, int nch, float* __restrict__ rec) {
  constexpr int HD = 256;
  const int z = (int)blockIdx.x, kvh = (int)blockIdx.y;
  const unsigned tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  const int ln = (int)(lane & 15u), lk = (int)(lane >> 4);
  const int rows = n * GRP;
  const int pbeg = z * csz, pend = min((z + 1) * csz, pos0 + n);  // the chunk's positions seen by anyone
  // the softmax row of this lane: ρ = 16w + ln, visible positions [pbeg, ctx_r)
  const int rho = 16 * (int)w + ln;
  const bool rv = rho < rows;
  const int ctx_r = rv ? min(pos0 + rho / GRP + 1, pend) : pbeg;
  float4 q[16];  // Q[ρ][16j + 4lk .. +3]
  {
    const float* qr = qb + ((size_t)(rv ? rho / GRP : 0) * nq + kvh * GRP + (rv ? rho % GRP : 0)) * HD + 4 * lk;
#pragma unroll
    for (int j = 0; j < 16; ++j) q[j] = rv ? *reinterpret_cast<const float4*>(qr + 16 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  f32x4 o[16];  // tile 4th + c
#pragma unroll
  for (int t = 0; t < 16; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float* kb = kcache + (size_t)kvh * max_ctx * HD;
  const float* vb = vcache + (size_t)kvh * max_ctx * HD;
  // A block's key and value rows are requested one block ahead (keys while the previous block's
  // values are multiplied, values while its scores are formed), so that no matrix instruction waits
  // for a load issued just before it.  Positions past the chunk are clamped to its last one
  // (written, finite) and masked.
  float4 kk[16], vv[16];  // kk[j]: K[p][16j + 4lk ..]; vv[4s + th]: V[p0 + 4lk + s][64th + 4ln ..]
  auto load_k = [&](int pb) {
    const float* kr = kb + (size_t)min(pb + ln, pend - 1) * HD + 4 * lk;
#pragma unroll
    for (int j = 0; j < 16; ++j) kk[j] = *reinterpret_cast<const float4*>(kr + 16 * j);
  };
  auto load_v = [&](int pb) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float* vr = vb + (size_t)min(pb + 4 * lk + s, pend - 1) * HD + 4 * ln;
#pragma unroll
      for (int th = 0; th < 4; ++th) vv[4 * s + th] = *reinterpret_cast<const float4*>(vr + 64 * th);
    }
  };
  if (pbeg < pend) {
    load_k(pbeg);
    load_v(pbeg);
  }
  for (int p0 = pbeg; p0 < pend; p0 += 16) {
    const int pn = p0 + 16 < pend ? p0 + 16 : p0;  // the next block (the last one reloads itself)
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j].x, q[j].x, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j + 1].x, q[j + 1].x, s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j].y, q[j].y, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j + 1].y, q[j + 1].y, s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j].z, q[j].z, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j + 1].z, q[j + 1].z, s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j].w, q[j].w, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[j + 1].w, q[j + 1].w, s1, 0, 0, 0);
    }
    load_k(pn);
    float sc[4], bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = p0 + 4 * lk + i < ctx_r ? s0[i] + s1[i] : -INFINITY;
      bm = fmaxf(bm, sc[i]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float mn = fmaxf(m, bm);
    // a row with no visible position yet keeps m = -inf: its factors are 0 and 1 by definition
    const float al = mn == -INFINITY ? 1.0f : expf(m - mn);
    float p[4], ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = sc[i] == -INFINITY ? 0.f : expf(sc[i] - mn);
      ps += p[i];
    }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l = l * al + ps;
    m = mn;
    // the O rows of this lane are 16w + 4lk + i: their factors live in lanes 4lk + i (skipped when
    // no row of the wave has a new maximum: every factor is then exactly 1)
    if (__builtin_amdgcn_ballot_w64(al != 1.0f)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = __shfl(al, 4 * lk + i);
#pragma unroll
        for (int t = 0; t < 16; ++t) o[t][i] *= a;
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int th = 0; th < 4; ++th) {
        const float4 v4 = vv[4 * s + th];
        o[4 * th + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[s], v4.x, o[4 * th + 0], 0, 0, 0);
        o[4 * th + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[s], v4.y, o[4 * th + 1], 0, 0, 0);
        o[4 * th + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[s], v4.z, o[4 * th + 2], 0, 0, 0);
        o[4 * th + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[s], v4.w, o[4 * th + 3], 0, 0, 0);
      }
    load_v(pn);
  }
  // records: (m, l) of row ρ from lanes lk = 0; o rows 16w + 4lk + i, dims 64th + 4ln .. +3
  if (lk == 0 && rv) {
    float* rr = rec + (((size_t)(rho / GRP) * nq + kvh * GRP + rho % GRP) * nch + z) * (2 + HD);
    rr[0] = m;
    rr[1] = l;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ro = 16 * (int)w + 4 * lk + i;
    if (ro >= rows) continue;
    float* rr = rec + (((size_t)(ro / GRP) * nq + kvh * GRP + ro % GRP) * nch + z) * (2 + HD) + 2 + 4 * ln;
#pragma unroll
    for (int th = 0; th < 4; ++th)
      *reinterpret_cast<float4*>(rr + 64 * th) = make_float4(o[4 * th][i], o[4 * th + 1][i], o[4 * th + 2][i], o[4 * th + 3][i]);
  }
}

// Merge of the position chunks of bt_attn_kernel (records with l = 0 held no position), then
// o·sigmoid(gate).  Grid (n, nq), 256 threads (one output dim each); nch <= 256.  Thread z < nch
// brings chunk z's (m, l) to LDS, so that every chunk's weight exp(m_z - M) is formed once, and the
// dims are summed over the chunks in order, the first 64 requested with the statistics and the
// rest 16 at a time.
__global__ __launch_bounds__(256) void bt_attn_merge_kernel(const float* __restrict__ rec, int nch,
                                                            const float* __restrict__ gate, int nq,
                                                            float* __restrict__ ao) {
  constexpr int HD = 256;
  __shared__ float ml[2][256];  // m, then the chunk weight; l
  __shared__ float red[8];
  const int t = blockIdx.x, h = blockIdx.y;
  const unsigned tid = threadIdx.x;
  const float* rr = rec + ((size_t)t * nq + h) * nch * (2 + HD);
  const bool has = (int)tid < nch;
  // this dim of the first NO chunks, requested together with the chunk statistics (they do not
  // depend on the maximum): one memory round trip for up to NO chunks
  constexpr int NO = 64;
  const float gt = gate[((size_t)t * nq + h) * HD + tid];  // the output gate, with the rest
  float o0[NO];
#pragma unroll
  for (int k = 0; k < NO; ++k) o0[k] = k < nch ? rr[(size_t)k * (2 + HD) + 2 + tid] : 0.f;
  const float mz = has ? rr[(size_t)tid * (2 + HD)] : -INFINITY;
  const float lz = has ? rr[(size_t)tid * (2 + HD) + 1] : 0.f;
  // M = max of m over the chunks that held a position (in any order: max is exact)
  float m = lz > 0.f ? mz : -INFINITY;
  m = wave_max(m);
  if ((tid & 63u) == 0) red[tid >> 6] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  ml[0][tid] = lz > 0.f ? expf(mz - M) : 0.f;
  ml[1][tid] = lz;
  __syncthreads();
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int k = 0; k < NO; ++k) {
    if (k < nch) {
      const float e = ml[0][k];
      L = __builtin_fmaf(ml[1][k], e, L);
      O = __builtin_fmaf(o0[k], e, O);
    }
  }
  for (int z0 = NO; z0 < nch; z0 += 16) {
    float o[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) o[k] = z0 + k < nch ? rr[(size_t)(z0 + k) * (2 + HD) + 2 + tid] : 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (z0 + k < nch) {
        const float e = ml[0][z0 + k];
        L = __builtin_fmaf(ml[1][z0 + k], e, L);
        O = __builtin_fmaf(o[k], e, O);
      }
    }
  }
  ao[((size_t)t * nq + h) * HD + tid] = (O * (1.0f / L)) * sigmoidf_(gt);
}

// SwiGLU (mlp.rs:28-47, swiglu_inplace_simd): s[t][i] = silu(gate[t][i]) · up[t][i], gate rows
// [0, F) and up rows [F, 2F) of the gate/up product.
__global__ __launch_bounds__(256) void bt_swiglu_kernel(const float* __restrict__ gu, int64_t F, int n,
                                                        float* __restrict__ s) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int t = blockIdx.y;
  if (i >= F || t >= n) return;
  const float* row = gu + (size_t)t * 2 * F;
  s[(size_t)t * F + i] = siluf_(row[i]) * row[F + i];
}

// The same from the partials of a split gate/up product (part[z][t][2F], zstride apart): each sum in
// split order, as gemm_split_reduce_kernel forms it (times the token's 1/rms for a normed raw
// product), then silu(gate) · up.
__global__ __launch_bounds__(256) void bt_split_swiglu_kernel(const float* __restrict__ part, int splits,
                                                              int64_t zstride, int64_t F, int n,
                                                              float* __restrict__ s, const float* __restrict__ ssq,
                                                              int ssq_ld, int64_t K, float eps) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int t = blockIdx.y;
  if (i >= F || t >= n) return;
  const size_t off = (size_t)t * 2 * F + i;
  float g = ordered_sum(part + off, zstride, splits), u = ordered_sum(part + off + F, zstride, splits);
  if (ssq) {  // a normed raw product: 1/rms applied to the sums
    const float inv = split_inv_rms(ssq, ssq_ld, splits, t, K, eps);
    g *= inv;
    u *= inv;
  }
  s[(size_t)t * F + i] = siluf_(g) * u;
}

}  // namespace dz
