// ptk_kernel.h — device code of the persistent token kernel (declarations in ptk.h).
//
// Wave roles.  Wave 0 of every workgroup is the sync wave: it does every LL poll of the kernel, the
// small per-column phases (residual sums, SwiGLU, q/k/v sums, attention chunk merge, token
// selection), the per-head prologues of the DeltaNet and attention phases, and it stages every GEMV
// input into LDS.  Waves 1..7 are compute waves: they hold GEMV weights in registers, build the
// lookup table together with the sync wave and publish the split-K partials; they never poll.  In
// the layer GEMV phases the sync wave also runs a share of the table lookups once its input is
// staged (eight lookup waves, two per SIMD); in the lm_head it stages the next tile instead.  A
// wave's vector memory operations complete in issue order (gfx9 counts loads and stores on one
// vmcnt), so a poll issued behind a weight load waits for that load, and the CU returns results in
// issue order across its waves.  With the roles split, a compute wave requests the next GEMV's
// weights as soon as the current ones are consumed, and the weight stream overlaps every hand-over;
// the sync wave issues its next polls only after its workgroup's partial stores (an LDS count it
// waits on), so that those stores do not queue behind a poll round.
#pragma once
#include "ptk.h"
#include "topk.h"

namespace dz {

// The trace stamps (DAIZA_PTK_TRACE) exist only in the kernels of a translation unit that defines
// DZ_PTK_TRACE before it includes this header (ptk_trace.hip: ptk_kernel_trace, ptk_kernel_samp_trace).
// The production kernels carry none of their code.  The kernel's code is several times the size of
// the instruction cache, and the stamps' branches, skipped but interleaved with the hot code, cost 1%
// of a token.
#ifdef DZ_PTK_TRACE
constexpr bool kPtkTraced = true;
#else
constexpr bool kPtkTraced = false;
#endif

constexpr int kCW = kPtkWaves - 1;  // compute waves per workgroup
constexpr int kLW = kPtkWaves;      // lookup waves of a layer GEMV phase (the sync wave included)

// Index of this thread's wave among the NW lookup waves of a phase: all waves (NW == kLW), or the
// compute waves 1..7 (NW == kCW, the lm_head, where the sync wave stages the next tile meanwhile).
template <int NW>
__device__ __forceinline__ unsigned lookup_wave(unsigned tid) {
  static_assert(NW == kLW || NW == kCW, "lookup waves: all waves or the compute waves");
  return NW == kLW ? (tid >> 6) : (tid >> 6) - 1;
}

// Hardware reciprocal, reciprocal square root, exp and log (v_rcp_f32, v_rsq_f32 about 1 ulp;
// v_exp_f32 / v_log_f32 on the scaled argument) for the code that one wave runs on the token's
// critical path, where every instruction of a serial chain adds to the token's time.  The
// reference's own AVX2 path approximates the same functions (exp_ps, a degree-5 polynomial;
// sigmoid_ps / silu_ps, rcp_ps with one Newton step: simd_exp.rs:44-123).
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_rsq(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ float fast_sigmoid(float x) { return fast_rcp(1.0f + __expf(-x)); }
__device__ __forceinline__ float fast_silu(float x) { return x * fast_rcp(1.0f + __expf(-x)); }

// LDS map (dynamic LDS only, so that the lookup table sits at LDS address 0 as unit_dot needs).
constexpr int kLdsXs = kLutBytes;                                // staged LUT inputs: up to 16 tiles (lm_head)
constexpr int kLdsRed = kLdsXs + kMaxTilesH * kTileCols * 4;     // 64 floats: reductions
constexpr int kLdsFlag = kLdsRed + 64 * 4;                       // abort flag, trace, hand-off, arrival counts
constexpr int kLdsAsg = kLdsFlag + 16;                           // 8 x {t, rb0, rb1, lead}: GEMV assignments
constexpr int kLdsRng = kLdsAsg + 6 * 16;                        // u64: the sampled selection's generator state
constexpr int kLdsRing = kLdsAsg + 8 * 16;                       // kPtkMaxLayers ints: conv ring bases
constexpr int kLdsScratch = kLdsRing + kPtkMaxLayers * 4;        // phase scratch
constexpr int kLdsScratchBytes = 16 * 1024;
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

// Sum over each row of 16 lanes (DPP); every lane gets its row's sum.
__device__ __forceinline__ float row16_sum(float v) {
  v = dpp_add<0xB1>(v);
  v = dpp_add<0x4E>(v);
  v = dpp_add<0x141>(v);
  v = dpp_add<0x140>(v);
  return v;
}

// Coherent 16-byte row read of memory written earlier in the launch by another workgroup.
__device__ __forceinline__ float4 co_ld4(const float* p) {
  const u64* q = reinterpret_cast<const u64*>(p);
  const u64 a = __hip_atomic_load((const DZ_AS_GLOBAL u64*)q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const u64 b = __hip_atomic_load((const DZ_AS_GLOBAL u64*)(q + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((unsigned)a), __uint_as_float((unsigned)(a >> 32)), __uint_as_float((unsigned)b),
                     __uint_as_float((unsigned)(b >> 32)));
}

// A uniform value the compiler cannot see through: anything derived from it is recomputed where it
// is used instead of being hoisted out of the enclosing loop.
__device__ __forceinline__ int opaque_s(int v) {
  v = __builtin_amdgcn_readfirstlane(v);
  asm volatile("" : "+s"(v));
  return v;
}

// ------------------------------------------------------------------ polling (sync wave)

// Waits until every valid slot i < N of this lane (word addr(i, lane), expected tag tagf(i)) carries
// its tag, re-polling only the stale slots; invalid slots count as ready and are never loaded.
// Bounded: past spin_limit rounds, or once another workgroup has failed, it records a failure and
// returns false.  Each round passes addr an opaque copy of the lane index, so that slot addresses
// are recomputed per round instead of being kept live (two registers per slot) across the loop.
template <int N, class A, class V, class T>
__device__ __forceinline__ bool poll(const A& addr, const V& valid, const T& tagf, u64 (&w)[N], const PtkErr& e) {
  const unsigned lane0 = threadIdx.x & 63u;
#pragma unroll
  for (int i = 0; i < N; ++i) w[i] = valid(i) ? ll_ld(addr(i, lane0)) : ((u64)tagf(i) << 32);
  for (int spin = 0;; ++spin) {
    bool all = true;
#pragma unroll
    for (int i = 0; i < N; ++i) all &= ll_tag(w[i]) == tagf(i);
    if (all) return true;
    if (spin >= e.spin_limit) {
      ptk_fail(e, 1, tagf(0));
      return false;
    }
    if ((spin & 31) == 31 && flag_ld(e.flag)) return false;
    unsigned ln = threadIdx.x & 63u;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (ll_tag(w[i]) != tagf(i)) w[i] = ll_ld(addr(i, ln));
  }
}

struct TagC {
  unsigned t;
  __device__ __forceinline__ unsigned operator()(int) const { return t; }
};

// ------------------------------------------------------------------ GEMV phase pieces

// Weights of one GEMV phase held by a compute wave: up to U row-blocks of the phase's tile.
template <int U>
struct WRegs {
  UnitRegs u[U];
};

// Lookup wave cw (0..NW-1) loads its row-blocks rb0 + cw + NW*m of tile t into slots m < UN
// (slots >= UN are left alone: the phase that uses these registers reads only its UN slots).  Every
// slot m < UN is loaded: one without a row-block reads 16 bytes of the matrix's first cache line, at
// an offset of its own, in every lane, and its registers are never used.  A slot that were either
// loaded or left as it was would become a phi, and the register allocator resolves phis (as it does
// identical, merged loads) with copies next to the loads -- each copy waits for its load and turns
// the prefetch into a stall.
template <int UN, int U, int NW = kLW>
__device__ __forceinline__ void gemv_prefetch(const uint8_t* W, int ntiles, int t, int rb0, int rb1, unsigned tid,
                                              WRegs<U>& r) {
  static_assert(UN <= U, "prefetch slots exceed the register set");
  const unsigned lane = tid & 63u, cw = lookup_wave<NW>(tid);
#pragma unroll
  for (int m = 0; m < UN; ++m) {
    const int rb = rb0 + (int)cw + NW * m;
    const bool v = rb < rb1;
    const uint8_t* unit = W + ((size_t)(v ? rb : 0) * ntiles + t) * kUnitBytes;
    const u32x4* sp = reinterpret_cast<const u32x4*>(v ? unit + (size_t)lane * 16 : W + (size_t)m * 80);
    const int cs = v ? 64 : 1;  // chunk stride in 16-byte words
#pragma unroll
    for (int c = 0; c < 4; ++c) r.u[m].s[c] = __builtin_nontemporal_load(sp + c * cs);
    const u32x2* scp = reinterpret_cast<const u32x2*>(v ? unit + kUnitSignBytes + (size_t)lane * 8 : W + (size_t)m * 80 + 64);
    r.u[m].sc = __builtin_nontemporal_load(scp);
  }
}

// One slot of gemv_prefetch.
template <int U>
__device__ __forceinline__ void gemv_prefetch_slot(const uint8_t* W, int ntiles, int t, int rb0, int rb1, unsigned tid,
                                                   WRegs<U>& r, int m) {
  const unsigned lane = tid & 63u, cw = lookup_wave<kLW>(tid);
  const int rb = rb0 + (int)cw + kLW * m;
  const bool v = rb < rb1;
  const uint8_t* unit = W + ((size_t)(v ? rb : 0) * ntiles + t) * kUnitBytes;
  const u32x4* sp = reinterpret_cast<const u32x4*>(v ? unit + (size_t)lane * 16 : W + (size_t)m * 80);
  const int cs = v ? 64 : 1;
#pragma unroll
  for (int c = 0; c < 4; ++c) r.u[m].s[c] = __builtin_nontemporal_load(sp + c * cs);
  const u32x2* scp = reinterpret_cast<const u32x2*>(v ? unit + kUnitSignBytes + (size_t)lane * 8 : W + (size_t)m * 80 + 64);
  r.u[m].sc = __builtin_nontemporal_load(scp);
}

// The next GEMV phase's weights (UNX slots, 0 for none), requested by a GEMV phase when it is done
// with its own.
struct NextW {
  const uint8_t* W;
  int ntiles, t, rb0, rb1;
};

// LUT input sources: the sync wave (lane = 0..63) writes xs[lane + 64*m] (m < 8) for tile t after
// waiting for their words.  sq receives this lane's share of the tile's sum of v^2 when the source
// is normed (the GEMV publishes the tile sum from one workgroup per tile when sst is set: the
// RMSNorm statistics of v, applied to the GEMV result by its consumers).
struct SrcNormedLL {  // v[col] * w[col]
  const u64* v;
  unsigned tag;
  const float* w;
  int K;
  u64* sst;
  __device__ __forceinline__ bool stage(float* xs, int t, unsigned lane, const PtkErr& e, float& sq) const {
    // an opaque lane index: the loads below stay in this stage (when the stages of several tiles are
    // unrolled one after another they would otherwise all be hoisted to the first)
    asm volatile("" : "+v"(lane));
    const int base = t * kTileCols + (int)lane;
    float wv[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) wv[m] = base + 64 * m < K ? w[base + 64 * m] : 0.f;
    u64 x[8];
    const bool ok = poll<8>([&](int m, unsigned ln) { return v + t * kTileCols + ln + 64 * m; },
                            [&](int m) { return base + 64 * m < K; }, TagC{tag}, x, e);
    float s = 0.f;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      float o = 0.f;
      if (base + 64 * m < K) {
        const float hv = ll_val(x[m]);
        o = hv * wv[m];
        s += hv * hv;
      }
      xs[lane + 64 * m] = o;
    }
    sq = s;
    return ok;
  }
};

struct SrcPlainLL {
  const u64* v;
  unsigned tag;
  int K;
  static constexpr u64* sst = nullptr;
  __device__ __forceinline__ bool stage(float* xs, int t, unsigned lane, const PtkErr& e, float& sq) const {
    const int base = t * kTileCols + (int)lane;
    u64 x[8];
    const bool ok = poll<8>([&](int m, unsigned ln) { return v + t * kTileCols + ln + 64 * m; },
                            [&](int m) { return base + 64 * m < K; }, TagC{tag}, x, e);
#pragma unroll
    for (int m = 0; m < 8; ++m) xs[lane + 64 * m] = base + 64 * m < K ? ll_val(x[m]) : 0.f;
    sq = 0.f;
    return ok;
  }
};

// DeltaNet out-projection input: per v-head RMSNorm of y (from 16 per-wave sums of squares per head)
// times ssm_norm times silu(z) (ssm_output_gate_avx2, model/ssm.rs:246-286).  A tile holds 4 heads.
struct SrcGatedYLL {
  const u64* y;
  const u64* zs;
  const u64* yss;  // [nvh][16]
  unsigned tag;
  const float* nw;
  int K;
  static constexpr u64* sst = nullptr;
  __device__ __forceinline__ bool stage(float* xs, int t, unsigned lane, const PtkErr& e, float& sq) const {
    const int base = t * kTileCols + (int)lane;
    const int nh = K / 128, h0 = t * (kTileCols / 128);
    float nwv[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) nwv[m] = base + 64 * m < K ? nw[(base + 64 * m) & 127] : 0.f;
    u64 x[17];
    auto addr = [&](int s, unsigned ln) -> const u64* {
      const int b = t * kTileCols + (int)ln;
      if (s < 8) return y + b + 64 * s;
      if (s < 16) return zs + b + 64 * (s - 8);
      return yss + (size_t)(h0 + (int)(ln >> 4)) * 16 + (ln & 15u);
    };
    auto valid = [&](int s) { return s < 16 ? base + 64 * (s & 7) < K : h0 + (int)(lane >> 4) < nh; };
    const bool ok = poll<17>(addr, valid, TagC{tag}, x, e);
    // lanes 16h..16h+15 hold the 16 partial sums of head h0 + h
    const float hs = row16_sum(valid(16) ? ll_val(x[16]) : 0.f);
    {
      // every lane forms the inverse norm of its row's head once; columns lane + 64m of the tile
      // belong to head m / 2, whose value lane 16 * (m / 2) holds
      const float hinv = fast_rsq(hs * (1.0f / 128.0f) + 1e-6f);
      const int hb = __builtin_bit_cast(int, hinv);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const float inv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(hb, 16 * (m >> 1)));
        xs[lane + 64 * m] = base + 64 * m < K ? ((ll_val(x[m]) * inv) * nwv[m]) * ll_val(x[8 + m]) : 0.f;
      }
    }
    sq = 0.f;
    return ok;
  }
};

// Trace stamp `slot` of phase `ph` of token i, written by thread `by` (tracing runs only).
__device__ __forceinline__ void ptk_mark(const PtkRun& r, const PtkPlan& P, int i, int ph, int w, unsigned tid,
                                         unsigned by, int slot = 0) {
  if constexpr (kPtkTraced) {
    if (r.trace && tid == by)
      glb(r.trace)[(((size_t)i * P.ppt + ph) * P.G + w) * kPtkTraceSlots + slot] = __builtin_amdgcn_s_memrealtime();
  }
}
struct TraceAt;
__device__ __forceinline__ bool r_trace_wait(const TraceAt& tr);
struct TraceAt {  // where a GEMV phase stamps its sub-points
  const PtkRun* r;
  const PtkPlan* P;
  int i, ph, w;
  __device__ __forceinline__ void operator()(unsigned tid, unsigned by, int slot) const {
    ptk_mark(*r, *P, i, ph, w, tid, by, slot);
  }
  // slot 0 from the last compute wave to finish its stores (an LDS arrival count, tracing runs only)
  __device__ __forceinline__ void last_wave(unsigned char* smem, unsigned tid) const {
    if (!kPtkTraced || !r->trace) return;
    if ((tid & 63u) == 0) {
      int* cnt = reinterpret_cast<int*>(smem + kLdsFlag + 4);
      const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if ((old + 1) % kCW == 0) ptk_mark(*r, *P, i, ph, w, tid, tid, 0);
    }
  }
};
__device__ __forceinline__ bool r_trace_wait(const TraceAt& tr) { return kPtkTraced && tr.r->trace != nullptr; }

// One split-K GEMV phase, run by both roles (SYNC: the sync wave, else a compute wave) with the same
// barriers (prior: this thread's previous phases succeeded).  The sync wave stages the tile's inputs and the
// first workgroup of each tile publishes the tile's sum of squares when the source provides one;
// all waves build the table; the compute waves run their row-blocks on weights already in
// registers (requested by an earlier phase), publish LL partials [t][row] and request the next
// GEMV's weights (nx, UNX slots) into the same registers.  The sync wave leaves once the table is
// built and goes on to its next phase while the compute waves finish.
struct NoPost {
  __device__ __forceinline__ void operator()() const {}
};
// The sync wave's gate.  A CU returns its vector-memory operations in issue order, stores included,
// so a compute wave's partial stores issued while the sync wave has a poll round in flight leave
// the CU only after that round returns (a memory round trip).  The next phase's inputs cannot be
// ready before this workgroup's own outputs are out, so the sync wave holds its next polls until
// every compute wave has issued its stores: compute waves count themselves in at LDS int [60] (GEMV
// phases) or [61] (the DeltaNet outputs), and the sync wave waits for the count of the phases passed.
// Bounded LDS spin of the sync wave until the count at LDS int index `idx` reaches `target`.
__device__ __forceinline__ void lds_gate_wait(unsigned char* smem, int idx, int target) {
  int* c = lds_ptr<int>(smem, kLdsRed) + idx;
  for (int spin = 0; spin < (1 << 22); ++spin) {
    if (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
    __builtin_amdgcn_s_sleep(1);
  }
}
__device__ __forceinline__ void lds_gate_arrive(unsigned char* smem, int idx, unsigned tid) {
  if ((tid & 63u) == 0)
    __hip_atomic_fetch_add(lds_ptr<int>(smem, kLdsRed) + idx, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <bool SYNC, int UN, int UNX, int U, class Src, class Post = NoPost>
__device__ __forceinline__ bool gemv_phase(unsigned char* smem, bool prior, const Src& src, WRegs<U>& r, const Assign& a,
                                           bool lead, u64* out, int64_t ld, unsigned tag, unsigned tid,
                                           const PtkErr& e, const NextW& nx, const TraceAt& tr, int& gs,
                                           const Post& post = Post{}) {
  float* lut = lds_ptr<float>(smem, 0);
  float* xs = lds_ptr<float>(smem, kLdsXs);
  bool ok = prior;
  if constexpr (SYNC) {
    if (ok) {
      float sq = 0.f;
      ok = src.stage(xs, a.t, tid, e, sq);
      if (src.sst != nullptr && lead) {
        const float s = wave_sum(sq);
        if (tid == 0 && ok) ll_st(src.sst + a.t, s, tag);
      }
    }
    tr(tid, 0, 3);
  } else {
    tr(tid, 64, 1);
  }
  if (!wg_ok(smem, ok)) return false;  // inputs staged; every compute wave is done with the previous table
  build_lut<kPtkThreads>(lut, xs, tid);
  lds_barrier();
  ++gs;
  if constexpr (!SYNC) tr(tid, 64, 2);
  {
    // all waves, the sync wave included, run their row-blocks
    const unsigned cw = lookup_wave<kLW>(tid), lane = tid & 63u;
    unsigned c[16];
    make_pos_consts(lane, c);
    // Every lookup before the first store: gfx9 counts loads and stores on one vmcnt, and with a
    // store pending the wait for a row-block's weights becomes a wait for everything.  The next
    // GEMV's weights after the stores: the CU's memory pipeline is in order, and stores queued
    // behind a prefetch reach the consumers only after it.
    float y[UN];
#pragma unroll
    for (int m = 0; m < UN; ++m) y[m] = a.rb0 + (int)cw + kLW * m < a.rb1 ? unit_dot(r.u[m], c) : 0.f;
#pragma unroll
    for (int m = 0; m < UN; ++m) {
      const int rb = a.rb0 + (int)cw + kLW * m;
      if (rb < a.rb1) ll_st(out + (size_t)a.t * ld + (size_t)rb * kRowBlock + lane, y[m], tag);
    }
  }
  if constexpr (SYNC) {
    lds_gate_wait(smem, 60, kCW * gs);
  } else {
    lds_gate_arrive(smem, 60, tid);
    tr.last_wave(smem, tid);
    post();
  }
#pragma unroll
  for (int m = 0; m < UNX; ++m) gemv_prefetch_slot<U>(nx.W, nx.ntiles, nx.t, nx.rb0, nx.rb1, tid, r, m);
  return true;
}

// ------------------------------------------------------------------ sync-wave phases

// S: token of step i -- a fed id, or the greedy pick over the previous lm_head's per-workgroup
// candidates (first maximum, simd_exp.rs:551-598) -- and this workgroup's embedding columns
// (forward.rs:212-213), published as LL words.
__device__ __forceinline__ int s_pick(const PtkPlan& P, unsigned lane, const u64* cand_v, const u64* cand_i,
                                      unsigned tag_prev, const PtkErr& e, bool& ok) {
  u64 x[16];
  auto addr = [&](int s, unsigned ln) {
    const int c = (int)ln + 64 * (s >> 1);
    return (s & 1) ? cand_i + c : cand_v + c;
  };
  auto valid = [&](int s) { return (int)lane + 64 * (s >> 1) < P.G; };
  ok = poll<16>(addr, valid, TagC{tag_prev}, x, e);
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
#pragma unroll
  for (int s = 0; s < 8; ++s)
    if (valid(2 * s)) {
      const float v = ll_val(x[2 * s]);
      const int id = __float_as_int(ll_val(x[2 * s + 1]));
      if (am_better(v, id, bv, bi)) {
        bv = v;
        bi = id;
      }
    }
  wave_argmax(bv, bi);
  int tok = __builtin_amdgcn_readfirstlane(bi);
  if (tok < 0 || tok >= P.vocab) tok = 0;  // no candidate (or a failed wait): token 0
  return tok;
}

// Sampled selection (sample_top_k_top_p_into, sampling.rs:144-247, over the previous lm_head's
// logits): each workgroup's lm_head phase published its samp.k best as an ordered list of keys
// (cand_key, two LL words each: high half, low half) at `sl`; workgroups [0, nm) merge kPtkFan lists
// each into the lists behind them, and every workgroup merges those and draws (spec_draw) with its
// own copy of the generator state (in LDS, kLdsRng), so that all of them draw the same id with no
// further hand-over.  With `fin` (the pick after a launch's last token) only workgroup 0 draws.

// Polls nl <= kPtkFan ordered lists of K <= kPtkSampMax keys (2K LL words each, contiguous from src)
// and selects their K best: lane 4j + r holds list j's keys r, r + 4, ... (descending) as its queue.
__device__ __forceinline__ uint64_t s_lists(const u64* src, int nl, int K, unsigned tag, unsigned lane,
                                            const PtkErr& e, bool& ok) {
  constexpr int Q = kPtkSampMax / 4;
  const int j = (int)(lane >> 2), r0 = (int)(lane & 3u);
  u64 x[2 * Q];
  auto addr = [&](int s, unsigned) { return src + (size_t)j * 2 * K + 2 * (r0 + 4 * (s >> 1)) + (s & 1); };
  auto valid = [&](int s) { return j < nl && r0 + 4 * (s >> 1) < K; };
  ok = poll<2 * Q>(addr, valid, TagC{tag}, x, e);
  uint64_t q[Q];
#pragma unroll
  for (int i = 0; i < Q; ++i)
    q[i] = valid(2 * i) ? ((uint64_t)(unsigned)x[2 * i] << 32) | (unsigned)x[2 * i + 1] : kCandNone;
  return queue_select<Q>(q, K);
}

__device__ __forceinline__ int s_sample(unsigned char* smem, const PtkPlan& P, const PtkRun& r, int w, unsigned lane,
                                        u64* sl, unsigned tag, bool fin, bool& ok) {
  const int K = r.samp.k, G = P.G, nm = (G + kPtkFan - 1) / kPtkFan;
  u64* merged = sl + 2 * kPtkSampMax * G;
  ok = true;
  if (w < nm) {
    const int l0 = w * kPtkFan;
    const uint64_t key = s_lists(sl + (size_t)l0 * 2 * K, min(kPtkFan, G - l0), K, tag, lane, r.err, ok);
    if ((int)lane < K) {
      ll_st(merged + (size_t)w * 2 * K + 2 * lane, __uint_as_float((unsigned)(key >> 32)), tag);
      ll_st(merged + (size_t)w * 2 * K + 2 * lane + 1, __uint_as_float((unsigned)key), tag);
    }
  }
  if (fin && w != 0) return 0;
  bool ok2 = true;
  const uint64_t key = s_lists(merged, nm, K, tag, lane, r.err, ok2);
  ok = ok && ok2;
  uint64_t* rsp = lds_ptr<uint64_t>(smem, kLdsRng);
  uint64_t rs = *rsp;
  int tok = spec_draw(key, K, r.samp.inv_t, r.samp.top_p, rs);
  if (lane == 0) *rsp = rs;
  if (tok < 0 || tok >= P.vocab) tok = 0;  // a failed wait: token 0
  return tok;
}

template <bool SAMP>
__device__ __forceinline__ bool s_select(unsigned char* smem, const PtkPlan& P, const PtkRun& r, int i, int w,
                                         unsigned lane, u64* hemb, const u64* cand_v, const u64* cand_i, u64* sl,
                                         unsigned tag_prev, unsigned tag, int pos, int& tok) {
  bool ok = true;
  if (i < r.n_feed) {
    tok = __builtin_amdgcn_readfirstlane(glb(r.feed)[i]);
  } else if constexpr (SAMP) {
    tok = s_sample(smem, P, r, w, lane, sl, tag_prev, false, ok);
  } else {
    tok = s_pick(P, lane, cand_v, cand_i, tag_prev, r.err, ok);
  }
  if (w == 0 && lane == 0) P.toklog[pos] = tok;
  // This wave's conv ring and KV cache stores of the previous token are complete before its first
  // publish of this token.  Every workgroup's layer-0 input depends on every workgroup's embedding
  // columns, so any read of those stores in this token happens after them.
  wait_stores();
  int c0, c1;
  even_split(w, P.G, P.H, &c0, &c1);
  for (int col = c0 + (int)lane; col < c1; col += 64) {
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
  return ok;
}

// ------------------------------------------------------------------ reducer phases
//
// The last NR workgroups are reducers: in every layer all their threads form the per-column sums of
// the split-K partials (R0: in-projection, R1: out-projection + residual, R2: SwiGLU of gate/up,
// R3: down + residual).  They stream no weights, so their polls never wait behind a weight stream
// in their CU's memory pipeline, and the GEMV workgroups request their next weights as soon as
// their lookups are done.  wr is the reducer index (0..NR-1); columns are split evenly over them.

// R1 / R3: h_out[c] = h_in[c] + sum_t part[t][c] (term 0 is h_in, then the tiles in order).  Thread
// (j, q) sums terms [q*Q, q*Q+Q) of column j into LDS; thread j then adds the nq slices in order.
template <int QMAX>
__device__ __forceinline__ bool r_resid(unsigned char* smem, bool prior, const PtkPlan& P, int wr, unsigned tid,
                                        const u64* h_in, unsigned tag_h, const u64* part, int np, int64_t ldp,
                                        unsigned tag_p, u64* h_out, unsigned tag, const PtkErr& e) {
  float* slice = lds_ptr<float>(smem, kLdsScratch);  // nq * nc <= 512 floats
  int c0, c1;
  even_split(wr, P.NR, P.H, &c0, &c1);
  const int nc = c1 - c0, K = np + 1;
  const int nq = nc > 0 ? min(kPtkThreads / nc, K) : 1;
  const int Q = (K + nq - 1) / nq;
  const int j = nc > 0 ? (int)tid % nc : 0, q = nc > 0 ? (int)tid / nc : nq;
  const int k0 = q * Q;
  bool ok = prior;
  if (ok && q < nq) {
    u64 x[QMAX];
    auto addr = [&](int sl, unsigned) {
      const int k = k0 + sl;
      return k == 0 ? h_in + c0 + j : part + (size_t)(k - 1) * ldp + c0 + j;
    };
    auto valid = [&](int sl) { return sl < Q && k0 + sl < K; };
    auto tagf = [&](int sl) { return k0 + sl == 0 ? tag_h : tag_p; };
    ok = poll<QMAX>(addr, valid, tagf, x, e);
    float sv = 0.f;
#pragma unroll
    for (int sl = 0; sl < QMAX; ++sl)
      if (valid(sl)) sv += ll_val(x[sl]);
    slice[q * nc + j] = sv;
  }
  if (!wg_ok(smem, ok)) return false;
  if ((int)tid < nc) {
    float tot = 0.f;
    for (int qq = 0; qq < nq; ++qq) tot += slice[qq * nc + (int)tid];
    ll_st(h_out + c0 + tid, tot, tag);
  }
  lds_barrier();  // the slices are reused by the next reducer phase
  return true;
}

// R2: sw[f] = silu(inv * sum_t g[t][f]) * (inv * sum_t u[t][f]) (mlp.rs:28-47), inv from h_mid's tile
// sums of squares.  Items 0..nf-1 are the gate rows of this reducer's channels, nf..2nf-1 the up
// rows; thread tid sums items tid + 512m (m < MF) into LDS, then thread f combines its channel.
template <int NTH, int MF>
__device__ __forceinline__ bool r_swiglu(unsigned char* smem, bool prior, const PtkPlan& P, int wr, unsigned tid,
                                         const u64* sstm, const u64* pgu, unsigned tag_p, u64* sw, unsigned tag,
                                         const PtkErr& e) {
  float* gu = lds_ptr<float>(smem, kLdsScratch);  // 2 nf floats
  float* red = lds_ptr<float>(smem, kLdsRed);
  int f0, f1;
  even_split(wr, P.NR, P.F, &f0, &f1);
  const int nf = f1 - f0;
  const int64_t ldp = (int64_t)P.nrb_gu * kRowBlock;
  const int T = P.nT_h;
  bool ok = prior;
  if (ok) {
    // slot MF*NTH: lane k < T of wave 0 polls the tile sum of squares k (wave 0 sums them)
    constexpr int N = MF * NTH + 1;
    u64 x[N];
    const bool sq_lane = (int)tid < T;
    auto item_row = [&](int it) { return it < nf ? f0 + it : P.F + f0 + (it - nf); };
    auto addr = [&](int sl, unsigned) -> const u64* {
      if (sl >= MF * NTH) return sstm + (sq_lane ? (int)tid : 0);
      return pgu + (size_t)(sl % NTH) * ldp + item_row((int)tid + kPtkThreads * (sl / NTH));
    };
    auto valid = [&](int sl) {
      if (sl >= MF * NTH) return sq_lane;
      return sl % NTH < T && (int)tid + kPtkThreads * (sl / NTH) < 2 * nf;
    };
    ok = poll<N>(addr, valid, TagC{tag_p}, x, e);
#pragma unroll
    for (int m = 0; m < MF; ++m) {
      const int it = (int)tid + kPtkThreads * m;
      if (it < 2 * nf) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < NTH; ++k)
          if (k < T) v += ll_val(x[m * NTH + k]);
        gu[it] = v;
      }
    }
    if (tid < 64) {
      const float ss = wave_sum(sq_lane ? ll_val(x[MF * NTH]) : 0.f);
      if (tid == 0) red[33] = fast_rsq(ss / (float)P.H + P.eps);
    }
  }
  if (!wg_ok(smem, ok)) return false;
  const float inv = red[33];
  for (int f = (int)tid; f < nf; f += kPtkThreads) ll_st(sw + f0 + f, fast_silu(gu[f] * inv) * (gu[nf + f] * inv), tag);
  lds_barrier();
  return true;
}

// R0: in-projection outputs = inv * sum of the tile partials (q|k|v|z|alpha|beta of a DeltaNet layer,
// q|gate|k|v of an attention layer), rows tid + 512m of this reducer's share.  The per-thread
// outcome is agreed on at the next reducer barrier.
template <int NTH, int MR>
__device__ __forceinline__ bool r_qkv(const PtkPlan& P, const PtkLayer& Ly, int wr, unsigned tid, const u64* sst_in,
                                      const u64* pin, unsigned tag_in, u64* qkv, unsigned tag, const PtkErr& e) {
  int r0, r1;
  even_split(wr, P.NR, Ly.rows_in, &r0, &r1);
  const int nr = r1 - r0;
  const int64_t ldp = (int64_t)Ly.nrb_in * kRowBlock;
  const int T = P.nT_h;
  const int lane = (int)(tid & 63u);
  // slot MR*NTH: lane k < T of every wave polls the tile sum of squares k (the wave sums them)
  constexpr int N = MR * NTH + 1;
  u64 x[N];
  auto addr = [&](int sl, unsigned) -> const u64* {
    if (sl >= MR * NTH) return sst_in + (lane < T ? lane : 0);
    return pin + (size_t)(sl % NTH) * ldp + r0 + (int)tid + kPtkThreads * (sl / NTH);
  };
  auto valid = [&](int sl) {
    if (sl >= MR * NTH) return lane < T;
    return sl % NTH < T && (int)tid + kPtkThreads * (sl / NTH) < nr;
  };
  const bool ok = poll<N>(addr, valid, TagC{tag_in}, x, e);
  const float ss = wave_sum(lane < T ? ll_val(x[MR * NTH]) : 0.f);
  const float inv = fast_rsq(ss / (float)P.H + P.eps);
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const int row = (int)tid + kPtkThreads * m;
    if (row < nr && ok) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < NTH; ++k)
        if (k < T) v += ll_val(x[m * NTH + k]);
      ll_st(qkv + r0 + row, v * inv, tag);
    }
  }
  return ok;
}

__device__ __forceinline__ void attn_chunks(const PtkPlan& P, int pos, int* chunk, int* gc) {
  const int ctx = pos + 1;
  int ch = (ctx + P.gmax - 1) / P.gmax;
  if (ch < 16) ch = 16;
  *chunk = ch;
  *gc = (ctx + ch - 1) / ch;
}

// Max over each row of 16 lanes (DPP); every lane gets its row's maximum.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
  return v;
}

// R'': merge the chunk records of each query head and apply the output gate (attention.rs:189-203):
// ao[h*hd + d] = (O/L) * sigmoid(gate), on all waves of a GEMV workgroup.  Output jj of this
// workgroup's share [j0, j1) (<= 32 outputs) is handled by the 16 lanes of row jj; lane s of the row
// holds chunks s, s+16, s+32, s+48 (gmax <= 64), and the row's max and sums are DPP reductions, so no
// barrier is involved.  The per-thread outcome is agreed on at the next barrier.
template <int MO>
__device__ __forceinline__ bool phase_merge(const PtkPlan& P, int w, unsigned tid, int pos, const u64* rec,
                                            unsigned tag_r, const u64* qkv, unsigned tag_q, u64* ao, unsigned tag,
                                            const PtkErr& e) {
  static_assert(MO <= kPtkThreads / 16, "one 16-lane row per attention output");
  constexpr int HD = 256;
  int chunk, gc;
  attn_chunks(P, pos, &chunk, &gc);
  int j0, j1;
  even_split(w, P.Gp, P.nq * HD, &j0, &j1);
  const int jj = (int)(tid >> 4), sub = (int)(tid & 15u);
  const bool act = jj < j1 - j0;
  const int j = j0 + (act ? jj : 0), h = j / HD, d = j % HD;
  // slots 3q + {0, 1, 2} = m, l, o[d] of chunk sub + 16q; slot 12 = the output's gate
  u64 x[13];
  auto addr = [&](int sl, unsigned) -> const u64* {
    if (sl == 12) return qkv + (int64_t)(h * 2 + 1) * HD + d;
    const u64* rc = rec + ((size_t)h * P.gmax + sub + 16 * (sl / 3)) * (2 + HD);
    return sl % 3 == 2 ? rc + 2 + d : rc + sl % 3;
  };
  auto valid = [&](int sl) { return act && (sl == 12 || sub + 16 * (sl / 3) < gc); };
  auto tagf = [&](int sl) { return sl == 12 ? tag_q : tag_r; };
  bool ok = true;
  if (act) ok = poll<13>(addr, valid, tagf, x, e);
  float mv[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) mv[q] = valid(3 * q) ? ll_val(x[3 * q]) : -INFINITY;
  const float M = row16_max(fmaxf(fmaxf(mv[0], mv[1]), fmaxf(mv[2], mv[3])));
  float lp = 0.f, op = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float ex = valid(3 * q) ? __expf(mv[q] - M) : 0.f;
    lp = __builtin_fmaf(valid(3 * q) ? ll_val(x[3 * q + 1]) : 0.f, ex, lp);
    op = __builtin_fmaf(valid(3 * q) ? ll_val(x[3 * q + 2]) : 0.f, ex, op);
  }
  const float L = row16_sum(lp), O = row16_sum(op);
  if (act && sub == 0 && ok) ll_st(ao + j, (O * fast_rcp(L)) * fast_sigmoid(ll_val(x[12])), tag);
  return ok;
}

// ------------------------------------------------------------------ phase B: Gated DeltaNet step

// State rows of a compute thread in the DeltaNet phase: waves 4..7 hold rows quarter*32 + (wave-4)*8
// + (lane >> 3), columns (lane & 7)*16 .. +16 of the v-head's 128x128 state S[i][j].
__device__ __forceinline__ void dn_state_load(const PtkPlan& P, const PtkLayer& Ly, int w, unsigned tid,
                                              float (&s)[16]) {
  // every thread loads: a thread without rows reads 16 distinct words of one cache line, so that no
  // phi forms and no identical loads merge (the register copies either needs would wait for the loads)
  const bool v = !Ly.attn && w < 4 * P.nvh && tid >= 256;
  const int vh = w >> 2, quarter = w & 3;
  const unsigned lane = tid & 63u, w4 = (tid >> 6) - 4, il = lane >> 3, js = lane & 7u;
  const int i = quarter * 32 + (int)(w4 * 8 + il);
  // Row i's 16 columns js*16.. are 64 contiguous bytes (S[vh][i][j]).  Plain loads: within a launch
  // these rows are written only by this thread (the delta rule below), and writes by other kernels
  // are made visible by the launch boundary.
  state_row_load(v ? Ly.state + (size_t)vh * 128 * 128 + (size_t)i * 128 + (size_t)js * 16 : P.output_norm, s);
}

// Workgroup w < 4*nvh: v-head w/4, state rows (w%4)*32 .. +32 (ssm.rs:425-616).  The sync wave takes
// its 322 in-projection channels (q and k of the tiled k-head kh = vh % nkh, this quarter's v and z
// channels, alpha, beta; summed and scaled by 1/rms in phase R0), runs the conv ring + causal conv +
// SiLU, the q/k L2 norms and the gates, and publishes silu(z); waves 4..7 then run the delta rule on
// the state rows held in registers and publish y and per-wave sums of y^2.
// Sum over the 8 lanes of each aligned group of 8 (DPP: xor 1, xor 2, then the half-row mirror
// adds the two quads); every lane of the group gets bitwise the same value.
__device__ __forceinline__ float group8_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  return v;
}

// LDS layout of the DeltaNet phase (scratch): q[128] k[128] v[32] | decay, beta | conv inputs of the
// 288 convolved channels (q 0..127, k 128..255, this quarter's v 256..287): ring history [3][288]
// (t = 0 oldest) and conv weights [4][288] | ssm_a, dt_bias.
constexpr int kDnCh = 288;
constexpr int kDnRing = 128 + 128 + 32 + 4;           // float offset of the ring history
constexpr int kDnConvW = kDnRing + 3 * kDnCh;         // conv weights
constexpr int kDnGate = kDnConvW + 4 * kDnCh;         // ssm_a, dt_bias
static_assert((kDnGate + 2) * 4 <= kLdsScratchBytes, "DeltaNet scratch exceeds the LDS scratch area");

// In-projection row of convolved channel c (0..287) of v-head vh, quarter `quarter`.
__device__ __forceinline__ int64_t dn_conv_row(const PtkPlan& P, int kh, int vh, int quarter, int c) {
  const int64_t kdim = (int64_t)P.nkh * 128;
  return c < 128 ? (int64_t)kh * 128 + c : c < 256 ? kdim + (int64_t)kh * 128 + (c - 128)
                                                   : 2 * kdim + (int64_t)vh * 128 + quarter * 32 + (c - 256);
}

// The conv inputs a compute thread of waves 1..3 brings to the DeltaNet phase: ring history (3) and
// conv weights (4) of channels c = tid-64 and tid-64+192, and (thread 64) ssm_a, dt_bias.  Loaded at
// the start of the layer, long before the phase, so that they are never in the CU's memory pipeline
// ahead of the sync wave's polls.  Every thread loads: one without channels (or in an attention
// layer) reads distinct words of one cache line, so that no phi forms.
struct DnConvIn {
  float rh[2][3], cw[2][4], g[2];
};
__device__ __forceinline__ void dn_conv_load(const PtkPlan& P, const PtkLayer& Ly, int w, unsigned tid, int ring_base,
                                             int pos, DnConvIn& ci) {
  const bool wgv = !Ly.attn && w < 4 * P.nvh && tid >= 64 && tid < 256;
  const int vh = w >> 2, quarter = w & 3, kh = vh % P.nkh;
  const int hb = (ring_base + pos) & 3;
  const int64_t qkvd = P.qkvd;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int c = (int)tid - 64 + 192 * k;
    const bool v = wgv && c < kDnCh;
    const int64_t row = v ? dn_conv_row(P, kh, vh, quarter, c) : 0;
#pragma unroll
    for (int t = 0; t < 3; ++t)
      ci.rh[k][t] = co_ld(v ? Ly.conv + (size_t)((hb + 1 + t) & 3) * qkvd + row : P.output_norm + 7 * k + t);
#pragma unroll
    for (int t = 0; t < 4; ++t) ci.cw[k][t] = v ? Ly.conv_w[(size_t)t * qkvd + row] : P.output_norm[7 * k + 3 + t];
  }
  const bool gv = wgv && tid == 64;
  ci.g[0] = gv ? Ly.ssm_a[vh] : P.output_norm[14];
  ci.g[1] = gv ? Ly.dt_bias[vh] : P.output_norm[15];
}

// Workgroup w < 4*nvh: v-head w/4, state rows (w%4)*32 .. +32 (ssm.rs:425-616).  Compute waves 1..3
// write the conv inputs they loaded at the layer's start into LDS and count themselves in; the sync wave takes
// its in-projection channels (q and k of the tiled k-head kh = vh % nkh, this quarter's v and z
// channels, alpha, beta; summed and scaled by 1/rms in phase R0), runs the conv ring + causal conv +
// SiLU, the q/k L2 norms and the gates, and publishes silu(z); waves 4..7 then run the delta rule on
// the state rows held in registers and publish y and per-wave sums of y^2.  dn_seq counts DeltaNet
// phases (both roles), for the compute waves' LDS arrival count.
template <bool SYNC>
__device__ __forceinline__ bool phase_dn(unsigned char* smem, bool prior, const PtkPlan& P, const PtkLayer& Ly,
                                         int ring_base, int w, unsigned tid, int pos, const u64* qkvz, unsigned tag_in,
                                         u64* y, u64* zs, u64* yss, unsigned tag, const PtkErr& e, float (&s)[16],
                                         const DnConvIn& ci, int dn_seq, const TraceAt& tr) {
  constexpr int HD = 128;
  if (w >= 4 * P.nvh) return wg_ok(smem, SYNC ? prior : true);
  float* qs = lds_ptr<float>(smem, kLdsScratch);
  float* ks = qs + HD;
  float* vs = ks + HD;
  float* sc = vs + 32;  // decay, beta
  float* rl = qs + kDnRing;
  float* cwl = qs + kDnConvW;
  float* gl = qs + kDnGate;
  int* arrivals = reinterpret_cast<int*>(smem + kLdsFlag + 12);
  const int vh = w >> 2, quarter = w & 3, kh = vh % P.nkh;
  const int hb = (ring_base + pos) & 3;
  const int64_t qkvd = P.qkvd;
  bool ok = SYNC ? prior : true;
  if (!SYNC && tid < 256) {
    // waves 1..3: conv inputs of channels c = tid-64 and tid-64+192 (loaded at the layer's start)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int c = (int)tid - 64 + 192 * k;
      if (c < kDnCh) {
#pragma unroll
        for (int t = 0; t < 3; ++t) rl[t * kDnCh + c] = ci.rh[k][t];
#pragma unroll
        for (int t = 0; t < 4; ++t) cwl[t * kDnCh + c] = ci.cw[k][t];
      }
    }
    if (tid == 64) {
      gl[0] = ci.g[0];
      gl[1] = ci.g[1];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS writes are done (lgkmcnt(0))
    if ((tid & 63u) == 0) __hip_atomic_fetch_add(arrivals, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (SYNC && ok) {
    const unsigned lane = tid;
    const bool vlane = lane < 32;  // slot 4: a v channel (convolved) below lane 32, a z channel above
    int64_t row[6];
    row[0] = dn_conv_row(P, kh, vh, quarter, (int)lane);
    row[1] = dn_conv_row(P, kh, vh, quarter, (int)lane + 64);
    row[2] = dn_conv_row(P, kh, vh, quarter, (int)lane + 128);
    row[3] = dn_conv_row(P, kh, vh, quarter, (int)lane + 192);
    row[4] = vlane ? dn_conv_row(P, kh, vh, quarter, 256 + (int)lane) : P.off_z + (int64_t)vh * HD + quarter * 32 + (lane - 32);
    row[5] = lane == 0 ? P.off_a + vh : P.off_b + vh;
    u64 x[6];
    ok = poll<6>([&](int sl, unsigned) { return qkvz + row[sl]; }, [&](int sl) { return sl < 5 || lane < 2; },
                 TagC{tag_in}, x, e);
    float xn[6];
#pragma unroll
    for (int sl = 0; sl < 6; ++sl) xn[sl] = sl < 5 || lane < 2 ? ll_val(x[sl]) : 0.f;
    // the compute waves' conv inputs (bounded wait; they always arrive)
    for (int spin = 0; spin < (1 << 22); ++spin) {
      if (__hip_atomic_load(arrivals, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) - 3 * dn_seq >= 0) break;
      __builtin_amdgcn_s_sleep(1);
    }
    // conv ring + causal conv + SiLU (ssm.rs:467-518): tap 3 is this token
    float c[5];
#pragma unroll
    for (int sl = 0; sl < 5; ++sl) {
      const int ch = sl < 4 ? (int)lane + 64 * sl : 256 + (int)(lane & 31u);
      float o = 0.f;
      o = __builtin_fmaf(rl[0 * kDnCh + ch], cwl[0 * kDnCh + ch], o);
      o = __builtin_fmaf(rl[1 * kDnCh + ch], cwl[1 * kDnCh + ch], o);
      o = __builtin_fmaf(rl[2 * kDnCh + ch], cwl[2 * kDnCh + ch], o);
      o = __builtin_fmaf(xn[sl], cwl[3 * kDnCh + ch], o);
      c[sl] = fast_silu(o);
    }
    if (ok) {
      // silu(z) first (the out-projection waits for it), then the conv ring
      if (!vlane) ll_st(zs + (size_t)vh * HD + quarter * 32 + (lane - 32), fast_silu(xn[4]), tag);
      if (vh < P.nkh && quarter == 0) {
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) co_st(Ly.conv + (size_t)hb * qkvd + row[sl], xn[sl]);
      }
      if (vlane) co_st(Ly.conv + (size_t)hb * qkvd + row[4], xn[4]);
    }
    if (lane == 0) {
      const float xa = xn[5] + gl[1];
      const float sp = xa > 20.0f ? xa : __logf(1.0f + __expf(xa));
      sc[0] = __expf(gl[0] * sp);
    } else if (lane == 1) {
      sc[1] = fast_sigmoid(xn[5]);
    }
    // L2 norms of q and k (ssm.rs:76-135), q *= 1/sqrt(128) (ssm.rs:532-533)
    const float inq = fast_rsq(wave_sum(c[0] * c[0] + c[1] * c[1]) + 1e-6f);
    const float ink = fast_rsq(wave_sum(c[2] * c[2] + c[3] * c[3]) + 1e-6f);
    const float qsc = 1.0f / sqrtf((float)HD);
    qs[lane] = (c[0] * inq) * qsc;
    qs[lane + 64] = (c[1] * inq) * qsc;
    ks[lane] = c[2] * ink;
    ks[lane + 64] = c[3] * ink;
    if (vlane) vs[lane] = c[4];
    tr(tid, 0, 3);
  }
  if (!wg_ok(smem, ok)) return false;
  tr(tid, 256, 1);
  if (!SYNC && tid >= 256) {
    // gated delta rule (ssm_scan_fused_avx2, ssm.rs:378-418) on row i (lane >> 3 within the wave's
    // 8 rows), columns j = js*16 + jj (js = lane & 7); a row's 8 column slices are adjacent lanes
    const unsigned lane = tid & 63u, w4 = (tid >> 6) - 4, il = lane >> 3, js = lane & 7u;
    const int i32 = (int)(w4 * 8 + il), i = quarter * 32 + i32;
    const float decay = sc[0], beta = sc[1];
    float kk[16], qq[16];
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const float4 a4 = *reinterpret_cast<const float4*>(&ks[js * 16 + 4 * v4]);
      const float4 b4 = *reinterpret_cast<const float4*>(&qs[js * 16 + 4 * v4]);
      kk[4 * v4] = a4.x; kk[4 * v4 + 1] = a4.y; kk[4 * v4 + 2] = a4.z; kk[4 * v4 + 3] = a4.w;
      qq[4 * v4] = b4.x; qq[4 * v4 + 1] = b4.y; qq[4 * v4 + 2] = b4.z; qq[4 * v4 + 3] = b4.w;
    }
    const float vi = vs[i32];
    float kvp = 0.f;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      s[jj] *= decay;
      kvp = __builtin_fmaf(s[jj], kk[jj], kvp);
    }
    const float kv = group8_sum(kvp);
    const float d = (vi - kv) * beta;
    float yp = 0.f;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      s[jj] = __builtin_fmaf(d, kk[jj], s[jj]);
      yp = __builtin_fmaf(s[jj], qq[jj], yp);
    }
    const float yy = group8_sum(yp);
    if (js == 0) ll_st(y + (size_t)vh * HD + i, yy, tag);
    const float ys = wave_sum(js == 0 ? yy * yy : 0.f);
    if (lane == 0) ll_st(yss + (size_t)vh * 16 + quarter * 4 + w4, ys, tag);
    lds_gate_arrive(smem, 61, tid);
    // the state rows are stored by dn_state_store after the out-projection's stores
  }
  return true;
}

// Stores the state rows updated by phase_dn (waves 4..7 of workgroups w < 4*nvh).  Called after the
// out-projection's partial stores: the CU's memory pipeline is in order, and 16 KiB of state stores
// issued at the end of the DeltaNet phase sat ahead of the out-projection's input polls.
__device__ __forceinline__ void dn_state_store(const PtkPlan& P, const PtkLayer& Ly, int w, unsigned tid,
                                               const float (&s)[16]) {
  if (w >= 4 * P.nvh || tid < 256) return;
  const int vh = w >> 2, quarter = w & 3;
  const unsigned lane = tid & 63u, w4 = (tid >> 6) - 4, il = lane >> 3, js = lane & 7u;
  const int i = quarter * 32 + (int)(w4 * 8 + il);
  state_row_store(Ly.state + (size_t)vh * 128 * 128 + (size_t)i * 128 + (size_t)js * 16, s);
}

// ------------------------------------------------------------------ phase B': attention chunk

// Workgroup (kv-head, chunk g) of attention.rs:56-208.  The sync wave takes the q/k/v sums of the
// kv-head's GRP query heads, applies the q/k RMSNorm, the reference's +/+ partial RoPE on dims 0..63
// (pairs (i, i+32), rope.rs:187-231) and q *= 1/sqrt(hd), and appends k/v when the chunk holds the
// new position; all waves then run the online softmax over the chunk's positions and publish one
// (m, l, o[hd]) record per query head.  pf() (the out-projection prefetch) runs after the last
// cache read.
template <bool SYNC, int GRP, class Pf>
__device__ __forceinline__ bool phase_attn(unsigned char* smem, bool prior, const PtkPlan& P, const PtkLayer& Ly, int w,
                                           unsigned tid, int pos, const u64* qkv, unsigned tag_q, u64* rec,
                                           unsigned tag, const PtkErr& e, const Pf& pf, const TraceAt& tr) {
  constexpr int HD = 256;
  const int kvh = w / P.gmax, g = w % P.gmax;
  int chunk, gc;
  attn_chunks(P, pos, &chunk, &gc);
  if (kvh >= P.nkv || g >= gc) {
    pf();
    return wg_ok(smem, SYNC ? prior : true);
  }
  const unsigned lane = tid & 63u, wave = tid >> 6;
  const int ctx = pos + 1, p0 = g * chunk, p1 = min(ctx, p0 + chunk);
  const bool has_new = p1 == ctx;
  float* qs = lds_ptr<float>(smem, kLdsScratch);  // [GRP][HD]
  float* kn = qs + GRP * HD;                      // [HD]
  float* vn = kn + HD;                            // [HD]
  float* wm = vn + HD;                            // [8][GRP]
  float* wl = wm + kPtkWaves * GRP;               // [8][GRP]
  float* wo = lds_ptr<float>(smem, 0);            // [8][GRP][HD] in the table area (unused here)
  bool ok = SYNC ? prior : true;
  if (SYNC && ok) {
    const int half = P.rope_dim / 2;  // 32 (checked on the host)
    const float* cs = P.rope + (size_t)pos * P.rope_dim;
    const float cr = cs[lane & 31u], sr = cs[half + (lane & 31u)];
    float qn[4], kw[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      qn[m] = Ly.q_norm[lane + 64 * m];
      kw[m] = Ly.k_norm[lane + 64 * m];
    }
    constexpr int N = GRP * 4 + 8;
    const int64_t kb = (int64_t)P.nq * 2 * HD;
    u64 x[N];
    auto addr = [&](int s, unsigned ln) -> const u64* {
      const int d = (int)ln + 64 * (s & 3);
      if (s < GRP * 4) return qkv + (int64_t)(kvh * GRP + s / 4) * 2 * HD + d;
      if (s < GRP * 4 + 4) return qkv + kb + (int64_t)kvh * HD + d;
      return qkv + kb + (int64_t)P.nkv * HD + (int64_t)kvh * HD + d;
    };
    ok = poll<N>(addr, [](int) { return true; }, TagC{tag_q}, x, e);
    // q/k RMSNorm over 256 dims (attention.rs:101-119), then RoPE: the partner of dim d < 64 is lane ^ 32
#pragma unroll
    for (int gi = 0; gi <= GRP; ++gi) {
      float v[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) v[m] = ll_val(x[gi * 4 + m]);
      const float ss = wave_sum((v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]));
      const float in = fast_rsq(ss / (float)HD + P.eps);
#pragma unroll
      for (int m = 0; m < 4; ++m) v[m] = (v[m] * in) * (gi < GRP ? qn[m] : kw[m]);
      const float o = __shfl_xor(v[0], 32, 64);
      v[0] = __builtin_fmaf(v[0], cr, o * sr);
      float* dst = gi < GRP ? qs + gi * HD : kn;
      const float scl = gi < GRP ? 1.0f / sqrtf((float)HD) : 1.0f;
#pragma unroll
      for (int m = 0; m < 4; ++m) dst[lane + 64 * m] = gi < GRP ? v[m] * scl : v[m];
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) vn[lane + 64 * m] = ll_val(x[GRP * 4 + 4 + m]);
    if (has_new && ok) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        co_st(Ly.kc + ((size_t)kvh * P.max_ctx + pos) * HD + lane + 64 * m, kn[lane + 64 * m]);
        co_st(Ly.vc + ((size_t)kvh * P.max_ctx + pos) * HD + lane + 64 * m, vn[lane + 64 * m]);
      }
    }
    tr(tid, 0, 3);
  }
  const float* kb = Ly.kc + (size_t)kvh * P.max_ctx * HD;
  const float* vb = Ly.vc + (size_t)kvh * P.max_ctx * HD;
  // Cache rows of position pp into slot registers.  Every slot is loaded unconditionally: a position
  // past the chunk or the new one (which comes from LDS) reads the chunk's first row instead, and the
  // value is never used -- a slot that were either loaded or left as it was would become a phi, and
  // the register copies that resolve it wait for the loads.
  auto ldkv = [&](int pp, float4& k4, float4& v4) {
    const int pc = (pp < p1 && pp != pos) ? pp : p0;
    k4 = co_ld4(kb + (size_t)pc * HD + 4 * lane);
    v4 = co_ld4(vb + (size_t)pc * HD + 4 * lane);
  };
  // Each wave keeps its next KD positions in flight: a compute wave requests its first KD while the
  // sync wave runs the prologue, the sync wave after it (its own loads would delay its polls).
  constexpr int NW = kPtkWaves, KD = 4;
  const int p = p0 + (int)wave;
  float4 kq[KD], vq[KD];
  if (!SYNC) {
#pragma unroll
    for (int d = 0; d < KD; ++d) ldkv(p + d * NW, kq[d], vq[d]);
  }
  if (!wg_ok(smem, ok)) return false;
  if (SYNC) {
#pragma unroll
    for (int d = 0; d < KD; ++d) ldkv(p + d * NW, kq[d], vq[d]);
  }
  // online softmax over this wave's positions (attention.rs:149-199); lane holds dims 4*lane..+3
  float m[GRP], l[GRP];
  float4 o[GRP], q4[GRP];
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    m[gi] = -INFINITY;
    l[gi] = 0.f;
    o[gi] = make_float4(0.f, 0.f, 0.f, 0.f);
    q4[gi] = *reinterpret_cast<const float4*>(&qs[gi * HD + 4 * lane]);
  }
  const float4 knew = *reinterpret_cast<const float4*>(&kn[4 * lane]);
  const float4 vnew = *reinterpret_cast<const float4*>(&vn[4 * lane]);
  for (int base = p; base < p1; base += KD * NW) {
#pragma unroll
    for (int d = 0; d < KD; ++d) {
      const int pp = base + d * NW;
      if (pp < p1) {
        const float4 k4 = pp == pos ? knew : kq[d], v4 = pp == pos ? vnew : vq[d];
        float dp[GRP];
#pragma unroll
        for (int gi = 0; gi < GRP; ++gi) {
          float t = q4[gi].x * k4.x;
          t = __builtin_fmaf(q4[gi].y, k4.y, t);
          t = __builtin_fmaf(q4[gi].z, k4.z, t);
          dp[gi] = __builtin_fmaf(q4[gi].w, k4.w, t);
        }
#pragma unroll
        for (int gi = 0; gi < GRP; ++gi) {
          const float score = wave_sum(dp[gi]);
          const float mn = fmaxf(m[gi], score);
          const float al = __expf(m[gi] - mn), be = __expf(score - mn);
          l[gi] = l[gi] * al + be;
          o[gi].x = __builtin_fmaf(be, v4.x, o[gi].x * al);
          o[gi].y = __builtin_fmaf(be, v4.y, o[gi].y * al);
          o[gi].z = __builtin_fmaf(be, v4.z, o[gi].z * al);
          o[gi].w = __builtin_fmaf(be, v4.w, o[gi].w * al);
          m[gi] = mn;
        }
      }
      if (base + KD * NW < p1) ldkv(pp + KD * NW, kq[d], vq[d]);
    }
  }
  tr(tid, 64, 1);
#pragma unroll
  for (int gi = 0; gi < GRP; ++gi) {
    if (lane == 0) {
      wm[wave * GRP + gi] = m[gi];
      wl[wave * GRP + gi] = l[gi];
    }
    *reinterpret_cast<float4*>(&wo[(wave * GRP + gi) * HD + 4 * lane]) = o[gi];
  }
  lds_barrier();
  // merge the 8 waves (a wave without positions has l = 0): the per-(wave, head) rescale factors
  // once, then every output dim, and publish each query head's record
  float* wx = wl + kPtkWaves * GRP;  // [8][GRP] rescale factors, then [GRP] M and [GRP] L
  if (tid < (unsigned)GRP) {
    const int gi = (int)tid;
    float M = -INFINITY;
    for (int wv = 0; wv < kPtkWaves; ++wv) M = fmaxf(M, wm[wv * GRP + gi]);
    float L = 0.f;
    for (int wv = 0; wv < kPtkWaves; ++wv) {
      const float ex = wl[wv * GRP + gi] > 0.f ? __expf(wm[wv * GRP + gi] - M) : 0.f;
      wx[wv * GRP + gi] = ex;
      L = __builtin_fmaf(wl[wv * GRP + gi], ex, L);
    }
    wx[kPtkWaves * GRP + gi] = M;
    wx[kPtkWaves * GRP + GRP + gi] = L;
  }
  lds_barrier();
  for (int idx = (int)tid; idx < GRP * HD; idx += kPtkThreads) {
    const int gi = idx / HD, d = idx % HD;
    float O = 0.f;
    for (int wv = 0; wv < kPtkWaves; ++wv) O = __builtin_fmaf(wo[(wv * GRP + gi) * HD + d], wx[wv * GRP + gi], O);
    u64* rc = rec + ((size_t)(kvh * GRP + gi) * P.gmax + g) * (2 + HD);
    if (d == 0) {
      ll_st(rc, wx[kPtkWaves * GRP + gi], tag);
      ll_st(rc + 1, wx[kPtkWaves * GRP + GRP + gi], tag);
    }
    ll_st(rc + 2 + d, O, tag);
  }
  tr(tid, 64, 2);
  // the out-projection weights, after the record stores (queued behind them, not ahead)
  pf();
  return true;
}

// ------------------------------------------------------------------ phase L: lm_head + argmax

// Full K per workgroup: rows [rb0, rb1) of the vocabulary, tile by tile (one table per tile), on
// weights requested one tile ahead; logits = inv_rms(h) * W (h * output_norm) (forward.rs:332-341).
// The tile loop is unrolled (NTH bounds the tile count), so that no loaded value is carried around a
// loop (a phi, resolved with register copies that wait for the loads).
template <bool SYNC, bool SAMP, int NTH, int U_LM, int U>
__device__ __forceinline__ bool phase_lm(unsigned char* smem, bool prior, const PtkPlan& P, const PtkRun& r, int i, int w,
                                         unsigned tid, const u64* h_fin, unsigned tag_h, WRegs<U>& cur, u64* cand_v,
                                         u64* cand_i, u64* sl, unsigned tag) {
  const PtkErr& e = r.err;
  const unsigned lane = tid & 63u, wave = tid >> 6, cw = wave - 1;
  int rb0, rb1;
  even_split(w, P.G, P.nrb_v, &rb0, &rb1);
  float acc[U_LM];
#pragma unroll
  for (int m = 0; m < U_LM; ++m) acc[m] = 0.f;
  float* lut = lds_ptr<float>(smem, 0);
  float* xs = lds_ptr<float>(smem, kLdsXs);
  float* red = lds_ptr<float>(smem, kLdsRed);
  float ssq = 0.f;  // sync wave: this lane's share of sum(h^2), the output norm's statistics
  bool ok = SYNC ? prior : true;
  if constexpr (!SYNC) gemv_prefetch<U_LM, U, kCW>(P.w_lm, NTH, 0, rb0, rb1, tid, cur);
#pragma unroll
  for (int t = 0; t < NTH; ++t) {  // NTH is the tile count itself (checked on the host)
    if (SYNC && ok) {
      SrcNormedLL src{h_fin, tag_h, P.output_norm, P.H, nullptr};
      float sq;
      ok = src.stage(xs, t, lane, e, sq);
      ssq += sq;
    }
    if (!wg_ok(smem, ok)) return false;
    build_lut<kPtkThreads>(lut, xs, tid);
    lds_barrier();
    if constexpr (!SYNC) {
      unsigned c[16];
      make_pos_consts(lane, c);
#pragma unroll
      for (int m = 0; m < U_LM; ++m) {
        const int rb = rb0 + (int)cw + kCW * m;
        if (rb < rb1) acc[m] += unit_dot(cur.u[m], c);
      }
      // the next tile (after the last one, slots without row-blocks: one cache line)
      gemv_prefetch<U_LM, U, kCW>(P.w_lm, NTH, t + 1 < NTH ? t + 1 : t, rb0, t + 1 < NTH ? rb1 : rb0, tid, cur);
    }
  }
  if constexpr (SYNC) {
    const float s = wave_sum(ssq);
    if (tid == 0) red[32] = 1.0f / sqrtf(s / (float)P.H + P.eps);
  }
  lds_barrier();
  const float inv = red[32];
  float* sv = lds_ptr<float>(smem, kLdsScratch);
  int* si = lds_ptr<int>(smem, kLdsScratch + 64);
  if constexpr (!SYNC) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    // the context's logits: the last token's, or every token's when an EOS pick may end the launch
    // early (the logits of the last token forwarded, as the reference leaves them)
    const bool last = i == r.n_tok - 1 || r.eos >= 0;
#pragma unroll
    for (int m = 0; m < U_LM; ++m) {
      const int rb = rb0 + (int)cw + kCW * m;
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
    if (lane == 0) {
      sv[cw] = bv;
      si[cw] = bi;
    }
    // sampled selection: the wave's samp.k best logits as an ordered list of keys (LDS, in the
    // table's space), from each lane's U_LM keys in descending order
    if constexpr (SAMP) {
      uint64_t q[U_LM];
#pragma unroll
      for (int m = 0; m < U_LM; ++m) {
        const int rb = rb0 + (int)cw + kCW * m;
        const int row = rb * kRowBlock + (int)lane;
        q[m] = rb < rb1 && row < P.vocab ? cand_key(acc[m] * inv, row) : kCandNone;
      }
#pragma unroll
      for (int a = 0; a < U_LM; ++a)
#pragma unroll
        for (int b = U_LM - 1; b > a; --b)
          if (q[b] > q[b - 1]) {
            const uint64_t t = q[b];
            q[b] = q[b - 1];
            q[b - 1] = t;
          }
      const uint64_t mine = queue_select<U_LM>(q, r.samp.k);
      if ((int)lane < r.samp.k) lds_ptr<uint64_t>(smem, 0)[cw * kPtkSampMax + lane] = mine;
    }
  }
  lds_barrier();
  if (SYNC && tid == 0) {
    float bv = sv[0];
    int bi = si[0];
    for (int k = 1; k < kCW; ++k)
      if (am_better(sv[k], si[k], bv, bi)) {
        bv = sv[k];
        bi = si[k];
      }
    ll_st(cand_v + w, bv, tag);
    ll_st(cand_i + w, __int_as_float(bi), tag);
  }
  if constexpr (SYNC && SAMP) {
    // the compute waves' lists merged into the workgroup's list at sl[w]: lane 8j + r holds list j's
    // keys r, r + 8, ... as its queue
    constexpr int Q = kPtkSampMax / 8;
    const int K = r.samp.k, j = (int)(lane >> 3), r0 = (int)(lane & 7u);
    const uint64_t* lst = lds_ptr<uint64_t>(smem, 0);
    uint64_t q[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) q[i] = j < kCW && r0 + 8 * i < K ? lst[j * kPtkSampMax + r0 + 8 * i] : kCandNone;
    const uint64_t mine = queue_select<Q>(q, K);
    if ((int)lane < K) {
      u64* d = sl + (size_t)w * 2 * K + 2 * lane;
      ll_st(d, __uint_as_float((unsigned)(mine >> 32)), tag);
      ll_st(d + 1, __uint_as_float((unsigned)mine), tag);
    }
  }
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


// Template bounds: NTH K tiles of hidden (DeltaNet / q,k,v / SwiGLU sums), GRP query heads per kv
// head, U_* row-block slots per compute wave of the in-proj, out-proj, gate/up, down and lm_head
// phases, QR terms per thread of the reducers' residual sums, MF gate/up items per thread of the
// reducers' SwiGLU sums, MR rows per thread of the reducers' in-projection sums, MO attention outputs
// per workgroup of the chunk merge (all checked on the host).
#define DZ_PTK_TPARAMS int NTH, int GRP, int U_IN, int U_OUT, int U_GU, int U_DN, int U_LM, int QR, int MF, int MR, int MO

// The token loop of one role: SYNC for wave 0, else for a compute wave; SAMP draws the tokens past
// the fed ones (PtkRun::samp) instead of the greedy pick (a kernel instance of its own, so that the
// greedy instance carries none of the sampling code).  Both roles walk the same
// phases and meet at the same barriers (each phase function holds both roles' barriers); a role's
// registers (the sync wave's poll words, a compute wave's weights) exist only in its own copy.  In a
// reducer workgroup both roles run the same reducer code.
template <bool SYNC, bool SAMP, DZ_PTK_TPARAMS>
__device__ __forceinline__ void ptk_role(const PtkRun& r, unsigned char* smem) {
  const PtkPlan P0 = plan_view(r.plan);
  const PtkErr& e = r.err;
  const int w0 = (int)blockIdx.x, G = P0.G;
  const bool reducer = w0 >= P0.Gp;
  const PtkOffsets& O = P0.off;
  const int64_t ld_in_h = (int64_t)P0.nrb_h * kRowBlock;
  const int64_t cand_off = ld_in_h;  // token region: h_emb [ld_in_h], cand_v [G], cand_i [G], sampling lists
  const int64_t samp_off = ptk_samp_off(ld_in_h, G);
  // a compute wave's weight registers: each GEMV phase's weights from the phase that requested them
  // to the phase that uses them
  constexpr int UW = U_IN > U_OUT ? (U_IN > U_GU ? (U_IN > U_DN ? U_IN : U_DN) : (U_GU > U_DN ? U_GU : U_DN))
                                  : (U_OUT > U_GU ? (U_OUT > U_DN ? U_OUT : U_DN) : (U_GU > U_DN ? U_GU : U_DN));
  constexpr int UWL = UW > U_LM ? UW : U_LM;
  WRegs<UWL> wn;
  float sreg[16];  // DeltaNet state rows (waves 4..7), from the layer's start to the DeltaNet phase
  DnConvIn cin;    // DeltaNet conv inputs (waves 1..3), likewise
  // `ok` carries the sync wave's outcome from its poll phases to the next workgroup barrier
  bool ok = true;
  int dn_seq = 0;  // DeltaNet phases passed (the compute waves' conv-input arrivals count 3 per phase)
  int gseq = 0;    // GEMV phases passed (both roles count them)
  bool stopped = false;
  int n_done = r.n_tok;
  for (int i = 0; i < r.n_tok; ++i) {
    const unsigned tb = r.tag0 + (unsigned)i * (unsigned)P0.ppt;
    const int par = (int)((r.tag0 / (unsigned)P0.ppt + (unsigned)i) & 1u);
    const int pos = r.pos0 + i;
    u64* tokreg = ll_region(P0, par, P0.n_layers);
    u64* prev_tok = ll_region(P0, par ^ 1, P0.n_layers);
    int tok = 0;
    if constexpr (SYNC) {
      ok = s_select<SAMP>(smem, P0, r, i, w0, threadIdx.x, tokreg, prev_tok + cand_off, prev_tok + cand_off + G,
                    prev_tok + samp_off, tb - (unsigned)P0.ppt + (unsigned)P0.ph_l, tb, pos, tok);
      ptk_mark(r, P0, i, 0, w0, threadIdx.x, 0);
    }
    // EOS stop (engine.rs:850-871: a sampled eos_token_id ends the loop before it is forwarded).  Every
    // workgroup picks the same token from the same candidates, so all of them stop at the same step;
    // the sync wave hands its decision to the compute waves through LDS.  toklog[pos] already holds
    // the eos id.
    if (r.eos >= 0) {
      int* stopw = lds_ptr<int>(smem, kLdsFlag + 8);
      if constexpr (SYNC) {
        if (threadIdx.x == 0) *stopw = (i >= r.n_feed && tok == r.eos) ? 1 : 0;
      }
      lds_barrier();
      if (*stopw) {
        stopped = true;
        n_done = i;
        break;
      }
    }
    const u64* h_in = tokreg;
    unsigned tag_h = tb;
    for (int l = 0; l < P0.n_layers; ++l) {
      // opaque copies of the thread index, the workgroup index and the plan's dimensions: values
      // derived from them are recomputed in each layer instead of being hoisted out of the loops
      // (and kept live, or spilled, for the whole kernel)
      unsigned tid = threadIdx.x;
      asm volatile("" : "+v"(tid));
      PtkPlan P = P0;
      int w = w0;
#define DZ_OPQ(f) f = opaque_s(f)
      DZ_OPQ(w); DZ_OPQ(P.G); DZ_OPQ(P.Gp); DZ_OPQ(P.NR); DZ_OPQ(P.H); DZ_OPQ(P.F); DZ_OPQ(P.nT_h); DZ_OPQ(P.nT_f);
      DZ_OPQ(P.nrb_h); DZ_OPQ(P.nrb_gu); DZ_OPQ(P.nrb_v); DZ_OPQ(P.gmax); DZ_OPQ(P.max_ctx); DZ_OPQ(P.nkh);
      DZ_OPQ(P.nvh); DZ_OPQ(P.qkvd); DZ_OPQ(P.inner); DZ_OPQ(P.off_z); DZ_OPQ(P.off_a); DZ_OPQ(P.off_b);
      DZ_OPQ(P.nq); DZ_OPQ(P.nkv); DZ_OPQ(P.rope_dim);
#undef DZ_OPQ
      const PtkLayer Ly = layer_at(P, l);
      u64* R = ll_region(P, par, l);
      const unsigned t0 = tb + (unsigned)Ly.ph0;
      const int k = Ly.attn ? 5 : 4;  // R1's phase offset within the layer
      if (reducer) {
        // R0, R1, R2, R3 of this layer (all threads)
        const int wr = w - P.Gp;
        if (ok) ok = r_qkv<NTH, MR>(P, Ly, wr, tid, R + O.sst_in, R + O.pin, t0, R + O.qkv, t0 + 1, e);
        ptk_mark(r, P, i, Ly.ph0 + 1, w, tid, 0);
        const unsigned tag_o = t0 + (unsigned)(k - 1);
        if (!r_resid<QR>(smem, ok, P, wr, tid, h_in, tag_h, R + O.po, Ly.nt_out, ld_in_h, tag_o, R + O.hmid, t0 + k, e))
          return;
        ptk_mark(r, P, i, Ly.ph0 + k, w, tid, 0);
        if (!r_swiglu<NTH, MF>(smem, true, P, wr, tid, R + O.sst_mid, R + O.pgu, t0 + k + 1, R + O.sw, t0 + k + 2, e))
          return;
        ptk_mark(r, P, i, Ly.ph0 + k + 2, w, tid, 0);
        if (!r_resid<QR>(smem, true, P, wr, tid, R + O.hmid, t0 + k, R + O.pd, P.nT_f, ld_in_h, t0 + k + 3, R + O.h,
                         t0 + k + 4, e))
          return;
        ptk_mark(r, P, i, Ly.ph0 + k + 4, w, tid, 0);
      } else {
        const int64_t ld_in = (int64_t)Ly.nrb_in * kRowBlock;
        const Assign a_out = asg_at(smem, 2 + Ly.attn);
        const Assign a_gu = asg_at(smem, 4);
        const Assign a_dn = asg_at(smem, 5);
        // The in-projection weights.  Every prefetch is issued in the block that uses it: a loaded
        // value carried around a loop becomes a phi, resolved with register copies that wait for the
        // loads.
        {
          ptk_mark(r, P, i, Ly.ph0 + 1, w, tid, 64, 1);
          const Assign a = asg_at(smem, Ly.attn);
          gemv_prefetch<U_IN>(Ly.w_in, P.nT_h, a.t, a.rb0, a.rb1, tid, wn);
          ptk_mark(r, P, i, Ly.ph0 + 1, w, tid, 64, 2);
        }
        // A: in-proj of h * attn_norm; tile leaders publish sum(h^2) per tile (1/rms applied downstream).
        // After its stores the compute waves request the DeltaNet conv inputs and state rows (every
        // layer loads: an attention layer reads 16 words of one cache line, so that no phi forms) and
        // then, in a DeltaNet layer, the out-proj weights slot by slot (an attention layer requests
        // them after its cache reads, and here reads one line per slot instead).  Requested at the
        // layer's start, the state rows -- 512 partial-line reads per workgroup -- sat in the CU's
        // memory queue ahead of the sync wave's polls for this phase's inputs.
        {
          const Assign a = asg_at(smem, Ly.attn);
          SrcNormedLL src{h_in, tag_h, Ly.attn_norm, P.H, R + O.sst_in};
          const NextW nx{Ly.w_out, Ly.nt_out, a_out.t, a_out.rb0, Ly.attn ? a_out.rb0 : a_out.rb1};
          const int ring_l = lds_ptr<int>(smem, kLdsRing)[l];
          auto post = [&]() {
            dn_conv_load(P, Ly, w, tid, ring_l, pos, cin);
            dn_state_load(P, Ly, w, tid, sreg);
          };
          if (!gemv_phase<SYNC, U_IN, U_OUT>(smem, ok, src, wn, a, asg_lead(smem, Ly.attn), R + O.pin, ld_in, t0, tid,
                                             e, nx, TraceAt{&r, &P, i, Ly.ph0, w}, gseq, post))
            return;
        }
        if (!Ly.attn) {
          // B: DeltaNet (q/k/v/z/alpha/beta summed by the reducers in R0)
          ++dn_seq;
          if (!phase_dn<SYNC>(smem, true, P, Ly, lds_ptr<int>(smem, kLdsRing)[l], w, tid, pos, R + O.qkv, t0 + 1,
                              R + O.y, R + O.zs, R + O.yss, t0 + 2, e, sreg, cin, dn_seq,
                              TraceAt{&r, &P, i, Ly.ph0 + 2, w}))
            return;
          if constexpr (!SYNC) ptk_mark(r, P, i, Ly.ph0 + 2, w, tid, 256);
          // C: out-proj
          SrcGatedYLL src{R + O.y, R + O.zs, R + O.yss, t0 + 2, Ly.ssm_norm, P.inner};
          auto post = [&]() { dn_state_store(P, Ly, w, tid, sreg); };
          if constexpr (SYNC) {
            if (w < 4 * P.nvh) lds_gate_wait(smem, 61, 4 * dn_seq);
          }
          if (!gemv_phase<SYNC, U_OUT, 0>(smem, true, src, wn, a_out, false, R + O.po, ld_in_h, t0 + 3, tid, e,
                                          NextW{}, TraceAt{&r, &P, i, Ly.ph0 + 3, w}, gseq, post))
            return;
        } else {
          // B': attention chunks (then the out-proj weights, after the cache reads they would delay)
          auto pf_out = [&]() {
            gemv_prefetch<U_OUT>(Ly.w_out, Ly.nt_out, a_out.t, a_out.rb0, a_out.rb1, tid, wn);
          };
          if (!phase_attn<SYNC, GRP>(smem, true, P, Ly, w, tid, pos, R + O.qkv, t0 + 1, R + O.rec, t0 + 2, e, pf_out,
                                     TraceAt{&r, &P, i, Ly.ph0 + 2, w}))
            return;
          if constexpr (!SYNC) ptk_mark(r, P, i, Ly.ph0 + 2, w, tid, 64);
          // R'': chunk merge and output gate (all waves)
          ptk_mark(r, P, i, Ly.ph0 + 3, w, tid, 0, 1);
          ok = phase_merge<MO>(P, w, tid, pos, R + O.rec, t0 + 2, R + O.qkv, t0 + 1, R + O.ao, t0 + 3, e) && ok;
          ptk_mark(r, P, i, Ly.ph0 + 3, w, tid, 0);
          // C': out-proj
          SrcPlainLL src{R + O.ao, t0 + 3, P.nq * 256};
          if (!gemv_phase<SYNC, U_OUT, 0>(smem, ok, src, wn, a_out, false, R + O.po, ld_in_h, t0 + 4, tid, e,
                                          NextW{}, TraceAt{&r, &P, i, Ly.ph0 + 4, w}, gseq))
            return;
        }
        // the gate/up weights (issued once after the layer kinds' branches join, so that no phi of two
        // loads forms); the sync wave's next polls are this GEMV's own inputs (h_mid, from R1)
        gemv_prefetch<U_GU>(Ly.w_gu, P.nT_h, a_gu.t, a_gu.rb0, a_gu.rb1, tid, wn);
        // D: gate/up of h_mid * post_norm; tile leaders publish sum(h_mid^2) per tile
        {
          SrcNormedLL src{R + O.hmid, t0 + k, Ly.post_norm, P.H, R + O.sst_mid};
          const NextW nx_dn{Ly.w_dn, P.nT_f, a_dn.t, a_dn.rb0, a_dn.rb1};
          if (!gemv_phase<SYNC, U_GU, U_DN>(smem, true, src, wn, a_gu, asg_lead(smem, 4), R + O.pgu,
                                            (int64_t)P.nrb_gu * kRowBlock, t0 + k + 1, tid, e, nx_dn,
                                            TraceAt{&r, &P, i, Ly.ph0 + k + 1, w}, gseq))
            return;
        }
        // E: down (its input is R2's SwiGLU)
        {
          SrcPlainLL src{R + O.sw, t0 + k + 2, P.F};
          if (!gemv_phase<SYNC, U_DN, 0>(smem, true, src, wn, a_dn, false, R + O.pd, ld_in_h, t0 + k + 3, tid, e,
                                         NextW{}, TraceAt{&r, &P, i, Ly.ph0 + k + 3, w}, gseq))
            return;
        }
        if constexpr (!SYNC) ptk_mark(r, P, i, Ly.ph0 + k + 4, w, tid, 64, 1);
      }
      h_in = R + O.h;
      tag_h = t0 + k + 4;
    }
    // L: lm_head + argmax candidates (all workgroups)
    if (!phase_lm<SYNC, SAMP, NTH, U_LM>(smem, ok, P0, r, i, w0, threadIdx.x, h_in, tag_h, wn, tokreg + cand_off,
                                   tokreg + cand_off + G, tokreg + samp_off, tb + (unsigned)P0.ph_l))
      return;
    if constexpr (SYNC) ptk_mark(r, P0, i, P0.ph_l, w0, threadIdx.x, 0);
  }
  // tokens forwarded by this launch (fewer than n_tok after an EOS stop), for the host
  if constexpr (SYNC) {
    if (w0 == 0 && threadIdx.x == 0) __hip_atomic_store(glb(e.flag) + 3, n_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // the pick after the last token, published as toklog[pos0 + n_tok]: the greedy pick by workgroup
  // 0, or the draw, with the merging workgroups, and the generator state after it
  if constexpr (SYNC && SAMP) {
    if (!stopped && w0 < (G + kPtkFan - 1) / kPtkFan) {
      const int i = r.n_tok;
      const unsigned tb = r.tag0 + (unsigned)i * (unsigned)P0.ppt;
      const int par = (int)((r.tag0 / (unsigned)P0.ppt + (unsigned)i) & 1u);
      u64* prev_tok = ll_region(P0, par ^ 1, P0.n_layers);
      bool pk = true;
      const int tok = s_sample(smem, P0, r, w0, threadIdx.x, prev_tok + samp_off,
                               tb - (unsigned)P0.ppt + (unsigned)P0.ph_l, true, pk);
      if (w0 == 0 && threadIdx.x == 0 && pk) {
        P0.toklog[r.pos0 + r.n_tok] = tok;
        *glb(r.samp.rng) = *lds_ptr<uint64_t>(smem, kLdsRng);
      }
    }
  } else if constexpr (SYNC) {
    if (w0 == 0 && !stopped) {
      const int i = r.n_tok;
      const unsigned tb = r.tag0 + (unsigned)i * (unsigned)P0.ppt;
      const int par = (int)((r.tag0 / (unsigned)P0.ppt + (unsigned)i) & 1u);
      const u64* prev_tok = ll_region(P0, par ^ 1, P0.n_layers);
      bool pk = true;
      const int tok = s_pick(P0, threadIdx.x, prev_tok + cand_off, prev_tok + cand_off + G,
                             tb - (unsigned)P0.ppt + (unsigned)P0.ph_l, e, pk);
      if (threadIdx.x == 0 && pk) P0.toklog[r.pos0 + r.n_tok] = tok;
    }
  }
}

template <bool SAMP, DZ_PTK_TPARAMS>
__device__ __forceinline__ void ptk_body(const PtkRun& r) {
  extern __shared__ __align__(16) unsigned char smem[];
  const PtkPlan P = plan_view(r.plan);
  const unsigned tid = threadIdx.x;
  const int w = (int)blockIdx.x, G = P.G;
  if (tid < 4) lds_ptr<int>(smem, kLdsFlag)[tid] = 0;
  if (SAMP && tid == 0) *lds_ptr<uint64_t>(smem, kLdsRng) = *glb(r.samp.rng);
  if (tid < 2) lds_ptr<int>(smem, kLdsRed)[60 + tid] = 0;
  // this workgroup's GEMV assignments per matrix kind (0/1: in-proj of a DeltaNet/attention layer,
  // 2/3: out-proj, 4: gate/up, 5: down) and the conv ring bases, fixed for the launch
  if (tid < 6) {
    const int k = (int)tid;
    // (selects, not indexing: a thread-dependent index into the plan would put it in scratch memory)
    const int T = k < 2 ? P.nT_h : k == 2 ? P.nt_out_k[0] : k == 3 ? P.nt_out_k[1] : k == 4 ? P.nT_h : P.nT_f;
    const int nrb = k == 0 ? P.nrb_in_k[0] : k == 1 ? P.nrb_in_k[1] : k < 4 ? P.nrb_h : k == 4 ? P.nrb_gu : P.nrb_h;
    const int Gp = P.Gp, wg = w < Gp ? w : 0;  // a reducer's assignment is never used
    const Assign a = gemv_assign(wg, Gp, T, nrb);
    int* q = lds_ptr<int>(smem, kLdsAsg) + 4 * k;
    q[0] = a.t;
    q[1] = a.rb0;
    q[2] = a.rb1;
    q[3] = w < Gp && w == tile_first_wg(a.t, T, Gp);
  }
  for (int l = (int)tid; l < P.n_layers; l += kPtkThreads) {
    const DZ_AS_CONST PtkLayer* t = (const DZ_AS_CONST PtkLayer*)P.L + l;
    lds_ptr<int>(smem, kLdsRing)[l] = t->attn ? 0 : *glb(t->ring_base);
  }
  lds_barrier();
  // one wave-uniform branch into the two roles
  if (__builtin_amdgcn_readfirstlane(tid >> 6) == 0)
    ptk_role<true, SAMP, NTH, GRP, U_IN, U_OUT, U_GU, U_DN, U_LM, QR, MF, MR, MO>(r, smem);
  else
    ptk_role<false, SAMP, NTH, GRP, U_IN, U_OUT, U_GU, U_DN, U_LM, QR, MF, MR, MO>(r, smem);
}

// The greedy kernel (instantiated in model.hip) and the sampled one (ptk_samp.hip, a code object of
// its own: the greedy kernel's place in model.hip's code object, by which the instruction cache maps
// its hot loops, does not move with it); with DZ_PTK_TRACE, the same two with the trace stamps.
#ifdef DZ_PTK_TRACE
template <DZ_PTK_TPARAMS>
__global__ __launch_bounds__(kPtkThreads) void ptk_kernel_trace(const PtkRun r) {
  ptk_body<false, NTH, GRP, U_IN, U_OUT, U_GU, U_DN, U_LM, QR, MF, MR, MO>(r);
}
template <DZ_PTK_TPARAMS>
__global__ __launch_bounds__(kPtkThreads) void ptk_kernel_samp_trace(const PtkRun r) {
  ptk_body<true, NTH, GRP, U_IN, U_OUT, U_GU, U_DN, U_LM, QR, MF, MR, MO>(r);
}
#else
template <DZ_PTK_TPARAMS>
__global__ __launch_bounds__(kPtkThreads) void ptk_kernel(const PtkRun r) {
  ptk_body<false, NTH, GRP, U_IN, U_OUT, U_GU, U_DN, U_LM, QR, MF, MR, MO>(r);
}
template <DZ_PTK_TPARAMS>
__global__ __launch_bounds__(kPtkThreads) void ptk_kernel_samp(const PtkRun r) {
  ptk_body<true, NTH, GRP, U_IN, U_OUT, U_GU, U_DN, U_LM, QR, MF, MR, MO>(r);
}
#endif
#undef DZ_PTK_TPARAMS

}  // namespace dz
