// ptk.h — the persistent token kernel: one launch runs whole tokens of the decode loop
// (forward_single_token, Daiza-engine/src/model/forward.rs:204-375, and the greedy selection of
// engine.rs:850-871) with every phase of every layer inside it.
//
// One workgroup per CU (512 threads, >80 KiB of LDS so that no CU takes two).  A token is a fixed
// sequence of phases; every workgroup walks the same sequence and knows statically which work of
// each phase is its own.  Phases hand their results over in "LL words": 64-bit {f32 value, 32-bit
// tag} stored and loaded with agent-scope relaxed atomics (write-through to the device coherence
// point, no fences).  A consumer polls the words it needs until each carries the producing phase's
// tag, so readiness and data travel together and no counter or barrier is involved.  Wave 0 of a
// workgroup does all polling; waves 1..7 hold the GEMV weights, requested as soon as the previous
// GEMV's weights are consumed, so the weight stream overlaps the hand-overs (ptk_kernel.h).
//
// Data outside LL words.  The conv ring rows and the KV appends of a token are written by sync waves
// with agent-scope write-through stores (co_st) and read by other workgroups one token or more later
// (co_ld).  Each sync wave waits for its stores to complete (s_waitcnt vmcnt(0)) at the start of the
// next token, before its first publish of that token, and every workgroup's layer-0 input depends on
// every workgroup's embedding columns: any read of those rows in a later token happens after the
// stores are visible at the device's coherence point.  The DeltaNet state rows are read and written
// by the same threads of the same workgroup every token (program order on one CU).
//
// Per DeltaNet layer: A in-proj GEMV -> R0 (in-proj partial sums) -> B DeltaNet -> C out-proj GEMV
// -> R1 (h_mid = h + sum of out-proj partials) -> D gate/up GEMV -> R2 (SwiGLU of the gate/up
// partials) -> E down GEMV -> R3 (h = h_mid + sum of down partials).  An attention layer replaces
// B, C by B' (split-K attention chunks) -> R'' (chunk merge and output gate) -> C'.  A token starts
// with S (greedy pick or fed id, embedding) and ends with L (lm_head, full K per workgroup,
// per-workgroup argmax).
#pragma once
#include "model_kernels.h"

namespace dz {

typedef unsigned long long u64;

// ------------------------------------------------------------------ address spaces

// The plan and the layer table are read through the constant address space (scalar loads through
// the scalar cache), and every data pointer taken from them is re-marked global.  A pointer loaded
// from memory is otherwise generic, and generic (flat) accesses count on both the vector-memory and
// the LDS counters: every LDS wait would also wait for outstanding HBM loads and LL stores, and
// every field read would wait for the weight prefetch in flight.
#define DZ_AS_GLOBAL __attribute__((address_space(1)))
#define DZ_AS_CONST __attribute__((address_space(4)))

template <class T>
__device__ __forceinline__ T* glb(T* p) {
  return (T*)(DZ_AS_GLOBAL T*)p;
}

// ------------------------------------------------------------------ LL words

__device__ __forceinline__ u64 ll_ld(const u64* p) {
  return __hip_atomic_load((const DZ_AS_GLOBAL u64*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_st(u64* p, float v, unsigned tag) {
  __hip_atomic_store((DZ_AS_GLOBAL u64*)p, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ll_val(u64 w) { return __uint_as_float((unsigned)w); }
__device__ __forceinline__ unsigned ll_tag(u64 w) { return (unsigned)(w >> 32); }

// Plain f32 in memory that other workgroups read in a later token (conv ring, KV cache):
// written through and read past the non-coherent caches.
__device__ __forceinline__ float co_ld(const float* p) {
  return __hip_atomic_load((const DZ_AS_GLOBAL float*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void co_st(float* p, float v) {
  __hip_atomic_store((DZ_AS_GLOBAL float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int flag_ld(const int* p) {
  return __hip_atomic_load((const DZ_AS_GLOBAL int*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct PtkErr {
  int* flag;  // first failure: code, phase tag, workgroup (0 = none); [3]: tokens forwarded
  int spin_limit;
};

__device__ __forceinline__ void ptk_fail(const PtkErr& e, int code, unsigned tag) {
  DZ_AS_GLOBAL int* f = (DZ_AS_GLOBAL int*)e.flag;
  int expected = 0;
  if (__hip_atomic_compare_exchange_strong(f, &expected, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT)) {
    __hip_atomic_store(f + 1, (int)tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(f + 2, (int)blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------------ work assignment

// Split-K GEMV over G workgroups: tile t owns workgroups [t*G/T, (t+1)*G/T); the n_t workgroups of a
// tile split its nrb row-blocks evenly.  Requires T <= G.
struct Assign {
  int t, rb0, rb1;
};
__host__ __device__ inline int tile_first_wg(int t, int T, int G) { return (int)(((int64_t)t * G) / T); }
__host__ __device__ inline Assign gemv_assign(int w, int G, int T, int nrb) {
  Assign a;
  a.t = (int)((((int64_t)w + 1) * T - 1) / G);
  const int w0 = tile_first_wg(a.t, T, G), w1 = tile_first_wg(a.t + 1, T, G);
  const int nw = w1 - w0, j = w - w0;
  a.rb0 = (int)(((int64_t)j * nrb) / nw);
  a.rb1 = (int)(((int64_t)(j + 1) * nrb) / nw);
  return a;
}
// Even split of n items over G workgroups: [w*n/G, (w+1)*n/G).
__host__ __device__ inline void even_split(int w, int G, int n, int* a, int* b) {
  *a = (int)(((int64_t)w * n) / G);
  *b = (int)(((int64_t)(w + 1) * n) / G);
}

constexpr int kPtkThreads = 512;
constexpr int kPtkWaves = kPtkThreads / 64;

// ------------------------------------------------------------------ plan (device memory)

struct PtkLayer {
  int attn;
  int rows_in;                 // in-proj rows; its partials have leading dimension nrb_in*64
  int nrb_in;
  int nt_out;                  // out-proj K tiles
  const uint8_t* w_in;
  const uint8_t* w_out;
  const uint8_t* w_gu;
  const uint8_t* w_dn;
  const float* attn_norm;
  const float* post_norm;
  const float* conv_w;         // [4][qkvd]
  const float* ssm_a;
  const float* dt_bias;
  const float* ssm_norm;
  float* conv;                 // ring [4][qkvd]
  float* state;                // [nvh][128 i][128 j] (row-major S[i][j])
  const int* ring_base;
  const float* q_norm;
  const float* k_norm;
  float* kc;                   // [nkv][max_ctx][hd]
  float* vc;
  int ph0;                     // index of this layer's first phase within a token
};

// Word offsets of the per-layer LL buffers inside one layer region.
struct PtkOffsets {
  int64_t pin, sst_in, po, hmid, sst_mid, pgu, sw, pd, h, y, zs, yss, qkv, rec, ao, words;
};

struct PtkPlan {
  // dimensions
  int G;                       // workgroups (one per CU)
  int Gp, NR;                  // GEMV workgroups [0, Gp) and reducer workgroups [Gp, G)
  int n_layers;
  int H, F, vocab;
  int nT_h, nrb_h, nT_f, nrb_gu, nrb_v;
  int nkh, nvh, qkvd, inner, off_z, off_a, off_b;
  int nq, nkv, hd, rope_dim, grp;
  int nrb_in_k[2];             // in-proj row-blocks of a DeltaNet [0] / attention [1] layer
  int nt_out_k[2];             // out-proj K tiles of a DeltaNet [0] / attention [1] layer
  int gmax;                    // attention chunks per kv-head at most (Gp / nkv)
  int max_ctx;
  float eps;
  int embd_f16;
  int ppt;                     // phases per token
  int ph_l;                    // index of the lm_head phase
  PtkOffsets off;
  // weights
  const uint8_t* w_lm;
  const float* output_norm;
  const uint16_t* emb_f16;
  const uint8_t* emb_q1;
  int emb_ntiles;
  const float* rope;           // [max_ctx][rope_dim]
  const PtkLayer* L;
  // LL memory: [2 parities][n_layers + 1 regions][off.words]; region n_layers holds the token-level
  // words: hemb (nrb_h*64), candv (G), candi (G), then (from ptk_samp_off) the sampled selection's
  // lists: G lists of 2K words, kPtkFan merged lists of 2K words, the drawn id (one word)
  u64* ll;
  // state / outputs
  TokState* st;
  int* toklog;
  float* logits;               // logits of the last token (vocab)
  float* logits_all;           // per-token logits [n][vocab] when requested, else null
};

constexpr int kPtkMaxLayers = 128;
// Sampled selection inside the token kernel: top_k up to kPtkSampMax, merged kPtkFan lists at a time
// in two levels (so G <= kPtkFan^2 workgroups).
constexpr int kPtkSampMax = 32;
constexpr int kPtkFan = 16;
// Word offsets of the sampled selection's lists within the token region (G workgroups; sizes fixed
// at kPtkSampMax so that the layout does not depend on the run's top_k).
__host__ __device__ inline int64_t ptk_samp_off(int64_t ld_h, int G) { return (ld_h + 2 * (int64_t)G + 63) / 64 * 64; }
__host__ __device__ inline int64_t ptk_samp_words(int G) {
  return 2 * (int64_t)kPtkSampMax * (G + kPtkFan) + 64;
}
// Trace stamps per (token, phase, workgroup): 0 = phase done; in a GEMV phase 1 = first compute
// wave at the staging barrier, 2 = table built (lookups start), 3 = sync wave done staging; in a
// DeltaNet phase 2 = inputs polled, 4 = conv inputs in LDS, 5 = conv and SiLU done, 3 = prologue
// done, 1 = delta-rule waves at the barrier, 6 = delta rule computed, 7 = its stores issued.
constexpr int kPtkTraceSlots = 8;

// Kernel instantiation for a model shape (the template bounds of ptk_kernel): K tiles of hidden
// (exact), GQA group, row-block slots per compute wave of each GEMV kind, terms per thread of the
// reducers' residual sums, gate/up items per thread of their SwiGLU sums, rows per thread of their
// in-projection sums and outputs per workgroup of the attention merge.  Other shapes run on the
// graph path.
struct PtkShape {
  int th, grp, u_in, u_out, u_gu, u_dn, u_lm, qr, mf, mr, mo;
};
constexpr PtkShape kPtkShape27b{10, 6, 2, 1, 4, 2, 3, 12, 3, 2, 32};
constexpr PtkShape kPtkShapeSmall{1, 2, 1, 1, 1, 1, 3, 4, 1, 1, 8};
inline bool ptk_fits(const PtkShape& s, const PtkShape& b) {
  return s.th == b.th && s.grp == b.grp && s.u_in <= b.u_in && s.u_out <= b.u_out && s.u_gu <= b.u_gu &&
         s.u_dn <= b.u_dn && s.u_lm <= b.u_lm && s.qr <= b.qr && s.mf <= b.mf && s.mr <= b.mr && s.mo <= b.mo;
}
// The sampled instance for a shape (ptk_samp.hip), or null.
const void* ptk_pick_samp(const PtkShape& s);
// The traced instance, greedy or sampled, for a shape (ptk_trace.hip), or null.
const void* ptk_pick_trace(const PtkShape& s, bool samp);

// Sampled selection: tokens past the fed ones are drawn from the previous logits' k best
// (temperature 1/inv_t, top_p) with the LcgRng state *rng (device memory); k = 0: the greedy pick.
struct PtkSamp {
  int k = 0;
  float inv_t = 1.f, top_p = 1.f;
  uint64_t* rng = nullptr;
};

struct PtkRun {
  PtkPlan plan;                // by value: kernel arguments are read with scalar loads
  const int* feed;             // fed ids for tokens [0, n_feed)
  int n_feed;
  int n_tok;
  int pos0;                    // position of the first token
  unsigned tag0;               // tag base of the first token (token i: tag0 + i*ppt)
  int want_logits;             // 1: write logits (last token; all tokens when logits_all is set)
  int eos;                     // >= 0: a greedy pick equal to eos ends the launch unforwarded
  PtkErr err;                  // err.flag[3] receives the number of tokens forwarded
  u64* trace;                  // optional [n_tok][ppt][G][kPtkTraceSlots] times (s_memrealtime), else null
  PtkSamp samp;                // tokens past the fed ones: drawn (samp.k > 0) or the greedy pick
};

static_assert(sizeof(PtkRun) <= 4096, "kernel arguments are limited to 4 KiB");

__device__ __forceinline__ u64* ll_region(const PtkPlan& P, int parity, int layer) {
  return P.ll + ((size_t)parity * (P.n_layers + 1) + (size_t)layer) * (size_t)P.off.words;
}

// The kernel's view of the plan: its data pointers marked global.
__device__ __forceinline__ PtkPlan plan_globals(PtkPlan v) {
  v.w_lm = glb(v.w_lm);
  v.output_norm = glb(v.output_norm);
  v.emb_f16 = glb(v.emb_f16);
  v.emb_q1 = glb(v.emb_q1);
  v.rope = glb(v.rope);
  v.ll = glb(v.ll);
  v.st = glb(v.st);
  v.toklog = glb(v.toklog);
  v.logits = glb(v.logits);
  v.logits_all = v.logits_all ? glb(v.logits_all) : nullptr;
  return v;
}

__device__ __forceinline__ PtkPlan plan_view(const PtkPlan& p) { return plan_globals(p); }


// Layer l of the table, read through the constant address space (l is uniform), data pointers
// marked global.
__device__ __forceinline__ PtkLayer layer_at(const PtkPlan& P, int l) {
  const DZ_AS_CONST PtkLayer* t = (const DZ_AS_CONST PtkLayer*)P.L + l;
  PtkLayer y;
  y.attn = t->attn;
  y.rows_in = t->rows_in;
  y.nrb_in = t->nrb_in;
  y.nt_out = t->nt_out;
  y.w_in = glb(t->w_in);
  y.w_out = glb(t->w_out);
  y.w_gu = glb(t->w_gu);
  y.w_dn = glb(t->w_dn);
  y.attn_norm = glb(t->attn_norm);
  y.post_norm = glb(t->post_norm);
  y.conv_w = glb(t->conv_w);
  y.ssm_a = glb(t->ssm_a);
  y.dt_bias = glb(t->dt_bias);
  y.ssm_norm = glb(t->ssm_norm);
  y.conv = glb(t->conv);
  y.state = glb(t->state);
  y.ring_base = glb(t->ring_base);
  y.q_norm = glb(t->q_norm);
  y.k_norm = glb(t->k_norm);
  y.kc = glb(t->kc);
  y.vc = glb(t->vc);
  y.ph0 = t->ph0;
  return y;
}

}  // namespace dz
