// spec.hip — speculative verify around the device's n-token verify forward:
// the reference's verify loop (Daiza-runtime/src/engine.rs:1255-1470) with Leviathan acceptance
// (leviathan_check, engine.rs:1791-1819), bonus sampling from the residual distribution
// (sample_bonus, engine.rs:1833-1866), temperature/top-k/top-p sampling
// (sample_top_k_top_p_into, Daiza-engine/src/math/sampling.rs:144-247) and its LcgRng
// (sampling.rs:9-19).  The reference forwards each accepted draft one at a time; here all k drafts
// run in one forward (dz_verify_forward) and the accepted prefix is kept (dz_verify_commit).
// The vocabulary-wide work (softmax statistics, the draft token's probabilities, top-k candidates of
// the row or of the residual distribution) runs on the device (spec_kernels.h); the acceptance
// draws and the final temperature / top-p draw over the k candidates run on the host, in the
// reference's order.  The sampled decode loop (dz_decode_sample) runs on the device: one token-kernel
// launch per token, then the top-k and the draw, which feeds the next launch.
#include "runtime.h"
#include "spec_kernels.h"

#include <algorithm>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <numeric>
#include <vector>

namespace dz {

// LcgRng::next_f32 (sampling.rs:14-18).
static float lcg_next(uint64_t* st) {
  *st = *st * 6364136223846793005ull + 1442695040888963407ull;
  return (float)(uint32_t)((*st >> 40) & 0xFFFFFFu) / (float)0x1000000;
}

// argmax_avx2 (simd_exp.rs:551-598): strict >, so the lowest index wins ties.
static size_t argmax_of(const float* x, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return best;
}

// softmax_inplace (math/softmax.rs:15-80): e = exp(x - max), x = e * (1 / sum).
static void softmax_into(const float* x, size_t n, float* out) {
  float mx = x[0];
  for (size_t i = 1; i < n; ++i)
    if (x[i] > mx) mx = x[i];
  float sum = 0.f;
  for (size_t i = 0; i < n; ++i) {
    out[i] = expf(x[i] - mx);
    sum += out[i];
  }
  const float inv = 1.0f / sum;
  for (size_t i = 0; i < n; ++i) out[i] *= inv;
}

// softmax_pair_single_avx2 (simd_exp.rs:656-767): softmax(target)[idx], softmax(draft)[idx].
static void softmax_pair_single(const float* t, const float* d, size_t n, size_t idx, float* p, float* q) {
  float tm = t[0], dm = d[0];
  for (size_t i = 1; i < n; ++i) {
    if (t[i] > tm) tm = t[i];
    if (d[i] > dm) dm = d[i];
  }
  float ts = 0.f, ds = 0.f, te_i = 0.f, de_i = 0.f;
  for (size_t i = 0; i < n; ++i) {
    const float te = expf(t[i] - tm), de = expf(d[i] - dm);
    ts += te;
    ds += de;
    if (i == idx) {
      te_i = te;
      de_i = de;
    }
  }
  if (ts <= 0.f) ts = 1.f;
  if (ds <= 0.f) ds = 1.f;
  *p = te_i / ts;
  *q = de_i / ds;
}

struct Sampler {
  std::vector<float> scaled, p, q, residual;
  std::vector<uint32_t> idx;
  std::vector<std::pair<uint32_t, float>> probs;

  // sample_top_k_top_p_into (sampling.rs:144-247).
  uint32_t top_k_top_p(const float* logits, size_t n, const dz_sampling& sp, uint64_t* rng) {
    if (sp.temperature <= 0.f) return (uint32_t)argmax_of(logits, n);
    const float inv_t = 1.0f / sp.temperature;
    scaled.resize(n);
    for (size_t i = 0; i < n; ++i) scaled[i] = logits[i] * inv_t;
    const size_t k = std::min((size_t)sp.top_k, n);
    idx.resize(n);
    std::iota(idx.begin(), idx.end(), 0u);
    // larger value first, the lower index first among equal values: a strict total order, so the k
    // kept and their order are fixed (the device top-k ranks the same way; the reference's
    // select_nth_unstable_by leaves the order of exact ties to its partition steps)
    auto desc = [&](uint32_t a, uint32_t b) { return scaled[a] > scaled[b] || (scaled[a] == scaled[b] && a < b); };
    std::nth_element(idx.begin(), idx.begin() + (k - 1), idx.end(), desc);
    std::sort(idx.begin(), idx.begin() + k, desc);
    float mx = -INFINITY;
    for (size_t j = 0; j < k; ++j) mx = std::max(mx, scaled[idx[j]]);
    probs.clear();
    float sum = 0.f;
    for (size_t j = 0; j < k; ++j) {
      const float e = expf(scaled[idx[j]] - mx);
      probs.emplace_back(idx[j], e);
    }
    for (auto& pr : probs) sum += pr.second;
    const float inv_sum = 1.0f / sum;
    for (auto& pr : probs) pr.second *= inv_sum;
    float cum = 0.f;
    size_t cutoff = probs.size();
    for (size_t j = 0; j < probs.size(); ++j) {
      cum += probs[j].second;
      if (cum >= sp.top_p) {
        cutoff = j + 1;
        break;
      }
    }
    probs.resize(cutoff);
    float new_sum = 0.f;
    for (auto& pr : probs) new_sum += pr.second;
    const float new_inv = 1.0f / new_sum;
    for (auto& pr : probs) pr.second *= new_inv;
    const float r = lcg_next(rng);
    float acc = 0.f;
    uint32_t chosen = probs[0].first;
    for (auto& pr : probs) {
      acc += pr.second;
      if (r <= acc) {
        chosen = pr.first;
        break;
      }
    }
    return chosen;
  }

  // sample_bonus (engine.rs:1833-1866): from norm(max(0, p - q)) as log-probabilities, or from the
  // target when the residual has no mass.
  uint32_t bonus(const float* target, const float* draft, size_t n, const dz_sampling& sp, uint64_t* rng) {
    p.resize(n);
    q.resize(n);
    residual.resize(n);
    softmax_into(target, n, p.data());
    softmax_into(draft, n, q.data());
    float sum = 0.f;
    for (size_t i = 0; i < n; ++i) {  // residual_max_zero_sum_avx2 (simd_exp.rs:605-642)
      const float r = std::max(p[i] - q[i], 0.0f);
      residual[i] = r;
      sum += r;
    }
    if (sum <= 1e-12f) return top_k_top_p(target, n, sp, rng);
    const float inv = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) residual[i] = logf(residual[i] * inv);
    return top_k_top_p(residual.data(), n, sp, rng);
  }
};

// The end of sample_top_k_top_p_into (sampling.rs:162-246) over the row's top-k candidates, given in
// order (value descending, lower index first): for mode 1 the values are residual masses r, turned
// into log-probabilities ln(r · 1/mass) as sample_bonus does; then scaled = value · (1/T), softmax
// over the candidates, top-p cut, renormalisation and the draw.
static uint32_t sample_candidates(const SpecCand* c, int K, int mode, float mass, const dz_sampling& sp,
                                  uint64_t* rng) {
  const float inv_t = 1.0f / sp.temperature;
  const float inv_m = mode == 1 ? 1.0f / mass : 1.0f;
  std::vector<float> scaled((size_t)K);
  for (int j = 0; j < K; ++j) scaled[(size_t)j] = (mode == 1 ? logf(c[j].v * inv_m) : c[j].v) * inv_t;
  float mx = -INFINITY;
  for (int j = 0; j < K; ++j) mx = std::max(mx, scaled[(size_t)j]);
  std::vector<float> pr((size_t)K);
  float sum = 0.f;
  for (int j = 0; j < K; ++j) pr[(size_t)j] = expf(scaled[(size_t)j] - mx);
  for (int j = 0; j < K; ++j) sum += pr[(size_t)j];
  const float inv_sum = 1.0f / sum;
  for (int j = 0; j < K; ++j) pr[(size_t)j] *= inv_sum;
  float cum = 0.f;
  int cut = K;
  for (int j = 0; j < K; ++j) {
    cum += pr[(size_t)j];
    if (cum >= sp.top_p) {
      cut = j + 1;
      break;
    }
  }
  float ns = 0.f;
  for (int j = 0; j < cut; ++j) ns += pr[(size_t)j];
  const float ninv = 1.0f / ns;
  for (int j = 0; j < cut; ++j) pr[(size_t)j] *= ninv;
  const float r = lcg_next(rng);
  float acc = 0.f;
  uint32_t chosen = (uint32_t)c[0].i;
  for (int j = 0; j < cut; ++j) {
    acc += pr[(size_t)j];
    if (r <= acc) {
      chosen = (uint32_t)c[j].i;
      break;
    }
  }
  return chosen;
}

static int check_sampling(const dz_sampling* sp) {
  if (!sp) return set_error(DZ_ERR_TENSOR, "sampling: null parameters");
  if (sp->temperature > 0.f && (sp->top_k < 1 || !(sp->top_p > 0.f)))
    return set_error(DZ_ERR_TENSOR, "sampling: top_k %d, top_p %g", sp->top_k, (double)sp->top_p);
  return DZ_OK;
}

// The stream that uploads draft logits beside a verify forward (default priority, non-blocking) and
// the event that marks the upload's end, created once per process.
static int upload_stream(hipStream_t* s, hipEvent_t* e) {
  static hipStream_t side = nullptr;
  static hipEvent_t done = nullptr;
  if (!side) DZ_HIP_CHECK(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
  if (!done) DZ_HIP_CHECK(hipEventCreateWithFlags(&done, hipEventDisableTiming));
  *s = side;
  *e = done;
  return DZ_OK;
}

}  // namespace dz

using namespace dz;

extern "C" {

float dz_lcg_next(uint64_t* state) { return state ? lcg_next(state) : 0.f; }

int dz_decode_sample(dz_ctx* c, uint32_t first_token, int n, const dz_sampling* sp, uint64_t* rng_state,
                     uint32_t* out_tokens) {
  if (!c || !rng_state || !out_tokens) return set_error(DZ_ERR_MODEL, "null argument");
  int rc = check_sampling(sp);
  if (rc) return rc;
  if (n < 1) return DZ_OK;
  // temperature <= 0 is the argmax with no draw (sample_top_k_top_p_into's greedy branch)
  if (sp->temperature <= 0.f) return dz_decode_greedy(c, first_token, n, out_tokens);
  const int vocab = ctx_config(c)->vocab;
  if (first_token >= (uint32_t)vocab) return set_error(DZ_ERR_TENSOR, "token id %u >= vocab %d", first_token, vocab);
  const int K = std::min(sp->top_k, vocab);
  // one token-kernel launch that draws inside the kernel (DAIZA_PTK_SAMPLE=0: a launch per token
  // with the top-k and the draw in kernels of their own between the launches)
  const char* ev = getenv("DAIZA_PTK_SAMPLE");
  if (!(ev && ev[0] == '0')) {
    rc = ctx_sample_decode(c, first_token, n, K, 1.0f / sp->temperature, sp->top_p, rng_state, out_tokens);
    if (rc != DZ_ERR_UNSUPPORTED) return rc;
  }
  uint32_t* feed = nullptr;
  const float* logits = nullptr;
  hipStream_t st = nullptr;
  Scratch* scr = nullptr;
  const size_t merge_lds = spec_merge_shmem(spec_slices(vocab), K);
  rc = K <= kSpecMaxK && merge_lds ? ctx_sample_begin(c, first_token, n, &feed, &logits, &st, &scr)
                                   : DZ_ERR_UNSUPPORTED;
  if (rc == DZ_ERR_UNSUPPORTED) {
    // the graph path, or a top_k beyond the device top-k: each forward's logits to the host and the
    // reference's sampler there
    std::vector<float> lg((size_t)vocab);
    Sampler smp;
    uint32_t tok = first_token;
    for (int i = 0; i < n; ++i) {
      if ((rc = dz_forward_token(c, tok, lg.data(), nullptr))) return rc;
      tok = smp.top_k_top_p(lg.data(), (size_t)vocab, *sp, rng_state);
      out_tokens[i] = tok;
    }
    return DZ_OK;
  }
  if (rc) return rc;
  // scratch: slice candidates | masses | top-k | total | statistics (unused by mode 0) | generator state
  const int nsl = spec_slices(vocab);
  const size_t off_mass = (size_t)nsl * kSpecMaxK * sizeof(uint64_t);
  const size_t off_top = off_mass + 256 * ((nsl * 4 + 255) / 256);
  const size_t off_tot = off_top + kSpecMaxK * sizeof(SpecCand);
  const size_t off_st = off_tot + 256;
  const size_t off_rng = off_st + 256 * ((sizeof(SpecRowStats) + 255) / 256);
  if ((rc = scr->reserve(off_rng + 256))) return rc;
  char* base = static_cast<char*>(scr->ptr);
  uint64_t* cand_dev = reinterpret_cast<uint64_t*>(base);
  float* mass_dev = reinterpret_cast<float*>(base + off_mass);
  SpecCand* top_dev = reinterpret_cast<SpecCand*>(base + off_top);
  float* tot_dev = reinterpret_cast<float*>(base + off_tot);
  SpecRowStats* st_dev = reinterpret_cast<SpecRowStats*>(base + off_st);
  uint64_t* rng_dev = reinterpret_cast<uint64_t*>(base + off_rng);
  DZ_HIP_CHECK(hipMemsetAsync(st_dev, 0, sizeof(SpecRowStats), st));
  DZ_HIP_CHECK(hipMemcpyAsync(rng_dev, rng_state, 8, hipMemcpyHostToDevice, st));
  const float inv_t = 1.0f / sp->temperature;
  for (int i = 0; i < n; ++i) {
    if ((rc = ctx_sample_launch(c, i))) return rc;
    hipLaunchKernelGGL(spec_topk_slice_kernel, dim3((unsigned)nsl), dim3(256), 0, st, logits, (const float*)nullptr,
                       vocab, 0, (const SpecRowStats*)st_dev, K, cand_dev, mass_dev);
    DZ_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(spec_topk_merge_kernel, dim3(1), dim3(256), merge_lds, st, (const uint64_t*)cand_dev, nsl, K,
                       (const float*)mass_dev, top_dev, tot_dev, SpecDraw{inv_t, sp->top_p, rng_dev, feed + i + 1});
    DZ_HIP_CHECK(hipGetLastError());
  }
  if ((rc = ctx_sample_end(c, n))) return rc;
  DZ_HIP_CHECK(hipMemcpyAsync(out_tokens, feed + 1, (size_t)n * 4, hipMemcpyDeviceToHost, st));
  DZ_HIP_CHECK(hipMemcpyAsync(rng_state, rng_dev, 8, hipMemcpyDeviceToHost, st));
  DZ_HIP_CHECK(hipStreamSynchronize(st));
  return DZ_OK;
}

int dz_sample(const float* logits, int n, const dz_sampling* sp, uint64_t* rng_state, uint32_t* out) {
  if (!logits || !rng_state || !out || n < 1) return set_error(DZ_ERR_TENSOR, "sample: bad arguments");
  int rc = check_sampling(sp);
  if (rc) return rc;
  Sampler s;
  *out = s.top_k_top_p(logits, (size_t)n, *sp, rng_state);
  return DZ_OK;
}

int dz_leviathan_check(const float* target, const float* draft, int n, uint32_t token, const dz_sampling* sp,
                       uint64_t* rng_state, int* accepted) {
  if (!target || !accepted || n < 1 || token >= (uint32_t)n) return set_error(DZ_ERR_TENSOR, "leviathan: bad arguments");
  int rc = check_sampling(sp);
  if (rc) return rc;
  if (sp->temperature <= 0.f) {
    *accepted = argmax_of(target, (size_t)n) == token;
    return DZ_OK;
  }
  if (!draft || !rng_state) return set_error(DZ_ERR_TENSOR, "leviathan: draft logits and rng needed");
  float p, q;
  softmax_pair_single(target, draft, (size_t)n, token, &p, &q);
  const float r = q > 1e-12f ? p / q : 0.f;
  *accepted = lcg_next(rng_state) < r;
  return DZ_OK;
}

int dz_sample_bonus(const float* target, const float* draft, int n, const dz_sampling* sp, uint64_t* rng_state,
                    uint32_t* out) {
  if (!target || !draft || !rng_state || !out || n < 1) return set_error(DZ_ERR_TENSOR, "bonus: bad arguments");
  int rc = check_sampling(sp);
  if (rc) return rc;
  Sampler s;
  *out = s.bonus(target, draft, (size_t)n, *sp, rng_state);
  return DZ_OK;
}

int dz_spec_verify(dz_ctx* c, const uint32_t* draft, int k, const float* draft_logits, const dz_sampling* sp,
                   int32_t eos_id, uint64_t* rng_state, int* n_accepted, uint32_t* bonus) {
  if (!c || !draft || !n_accepted || !bonus || k < 1) return set_error(DZ_ERR_TENSOR, "spec_verify: bad arguments");
  int rc = check_sampling(sp);
  if (rc) return rc;
  const bool greedy = sp->temperature <= 0.f;
  if (!greedy && (!draft_logits || !rng_state)) return set_error(DZ_ERR_TENSOR, "spec_verify: draft logits and rng needed");
  int vocab = 0;
  if ((rc = dz_ctx_vocab(c, &vocab))) return rc;
  const size_t V = (size_t)vocab;
  const int K = greedy ? 1 : std::min(sp->top_k, vocab);
  if (K > kSpecMaxK || !spec_merge_shmem(spec_slices(vocab), K)) {
    // a top-k beyond what the device pass keeps (or a vocabulary beyond its merge): every row to the
    // host, the sampler of dz_sample
    std::vector<float> rows((size_t)(k + 1) * V);
    if ((rc = dz_ctx_logits(c, rows.data()))) return rc;
    if ((rc = dz_verify_forward(c, draft, k, rows.data() + V))) return rc;
    Sampler s;
    int acc = 0;
    bool eos = false, have = false;
    uint32_t b = 0;
    for (int i = 0; i < k && !have && !eos; ++i) {
      const float* tl = rows.data() + (size_t)i * V;
      const float* dl = draft_logits + (size_t)i * V;
      float p, q;
      softmax_pair_single(tl, dl, V, draft[i], &p, &q);
      const float r = q > 1e-12f ? p / q : 0.f;
      if (!(lcg_next(rng_state) < r)) {
        b = s.bonus(tl, dl, V, *sp, rng_state);
        have = true;
      } else {
        ++acc;
        eos = eos_id >= 0 && draft[i] == (uint32_t)eos_id;
      }
    }
    if (!have && !eos) b = s.top_k_top_p(rows.data() + (size_t)k * V, V, *sp, rng_state);
    if ((rc = dz_verify_commit(c, eos ? acc - 1 : acc))) return rc;
    *n_accepted = acc;
    *bonus = eos ? 0xFFFFFFFFu : b;
    return DZ_OK;
  }
  // the forward is enqueued without a wait, so that the draft logits' upload (a side stream, joined by
  // an event before the statistics) runs while it computes
  if ((rc = ctx_verify_enqueue(c, draft, k))) return rc;
  const float *row0, *rows;
  hipStream_t st;
  Scratch* scr;
  if ((rc = ctx_verify_view(c, &row0, &rows, &st, &scr))) return rc;
  // scratch: draft logits [k][V] | tokens [k] | stats [k+1] | slice candidates | masses | top-k | total |
  // per-slice statistics [k+1][nsl]
  const int nsl = spec_slices(vocab);
  const size_t off_tok = greedy ? 0 : (size_t)k * V * 4, off_st = off_tok + 256 * ((k * 4 + 255) / 256);
  const size_t off_cand = off_st + 256 * (((size_t)(k + 1) * sizeof(SpecRowStats) + 255) / 256);
  const size_t off_mass = off_cand + (size_t)nsl * kSpecMaxK * sizeof(uint64_t);
  const size_t off_top = off_mass + 256 * ((nsl * 4 + 255) / 256);
  const size_t off_tot = off_top + kSpecMaxK * sizeof(SpecCand);
  const size_t off_part = off_tot + 256;
  if ((rc = scr->reserve(off_part + (size_t)(k + 1) * nsl * sizeof(SpecPart)))) return rc;
  char* base = static_cast<char*>(scr->ptr);
  float* dl_dev = greedy ? nullptr : reinterpret_cast<float*>(base);
  uint32_t* tok_dev = reinterpret_cast<uint32_t*>(base + off_tok);
  SpecRowStats* st_dev = reinterpret_cast<SpecRowStats*>(base + off_st);
  uint64_t* cand_dev = reinterpret_cast<uint64_t*>(base + off_cand);
  float* mass_dev = reinterpret_cast<float*>(base + off_mass);
  SpecCand* top_dev = reinterpret_cast<SpecCand*>(base + off_top);
  float* tot_dev = reinterpret_cast<float*>(base + off_tot);
  SpecPart* part_dev = reinterpret_cast<SpecPart*>(base + off_part);
  if (!greedy) {
    hipStream_t side;
    hipEvent_t up;
    if ((rc = upload_stream(&side, &up))) return rc;
    DZ_HIP_CHECK(hipMemcpyAsync(dl_dev, draft_logits, (size_t)k * V * 4, hipMemcpyHostToDevice, side));
    DZ_HIP_CHECK(hipEventRecord(up, side));
    DZ_HIP_CHECK(hipStreamWaitEvent(st, up, 0));
  }
  DZ_HIP_CHECK(hipMemcpyAsync(tok_dev, draft, (size_t)k * 4, hipMemcpyHostToDevice, st));
  // per-row statistics over the vocabulary in nsl slices per row, then one merge per row
  hipLaunchKernelGGL(spec_stats_part_kernel, dim3((unsigned)(k + 1), (unsigned)nsl), dim3(256), 0, st, row0, rows,
                     (const float*)dl_dev, k, vocab, part_dev);
  DZ_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(spec_stats_merge_kernel, dim3((unsigned)(k + 1)), dim3(64), 0, st, row0, rows,
                     (const float*)dl_dev, k, vocab, nsl, (const SpecPart*)part_dev, (const uint32_t*)tok_dev, st_dev);
  DZ_HIP_CHECK(hipGetLastError());
  std::vector<SpecRowStats> stats((size_t)k + 1);
  DZ_HIP_CHECK(hipMemcpyAsync(stats.data(), st_dev, stats.size() * sizeof(SpecRowStats), hipMemcpyDeviceToHost, st));
  DZ_HIP_CHECK(hipStreamSynchronize(st));
  // the row (target, draft) and mode the bonus is drawn from: -1 when there is none
  auto row_ptr = [&](int r) { return r == 0 ? row0 : rows + (size_t)(r - 1) * V; };
  auto topk = [&](int r, int mode, std::vector<SpecCand>& out, float* mass) -> int {
    hipLaunchKernelGGL(spec_topk_slice_kernel, dim3((unsigned)nsl), dim3(256), 0, st, row_ptr(r),
                       (const float*)(dl_dev ? dl_dev + (size_t)r * V : nullptr), vocab, mode,
                       (const SpecRowStats*)(st_dev + r), K, cand_dev, mass_dev);
    DZ_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(spec_topk_merge_kernel, dim3(1), dim3(256), spec_merge_shmem(nsl, K), st,
                       (const uint64_t*)cand_dev, nsl, K, (const float*)mass_dev, top_dev, tot_dev,
                       SpecDraw{0.f, 0.f, nullptr, nullptr});
    DZ_HIP_CHECK(hipGetLastError());
    out.resize((size_t)K);
    DZ_HIP_CHECK(hipMemcpyAsync(out.data(), top_dev, (size_t)K * sizeof(SpecCand), hipMemcpyDeviceToHost, st));
    DZ_HIP_CHECK(hipMemcpyAsync(mass, tot_dev, 4, hipMemcpyDeviceToHost, st));
    DZ_HIP_CHECK(hipStreamSynchronize(st));
    return DZ_OK;
  };
  int acc = 0;
  bool eos = false, have = false;
  uint32_t b = 0;
  std::vector<SpecCand> cands;
  for (int i = 0; i < k && !have && !eos; ++i) {
    const SpecRowStats& s = stats[(size_t)i];
    bool ok;
    if (greedy) {
      ok = (uint32_t)s.argmax == draft[i];
    } else {
      const float r = s.q > 1e-12f ? s.p / s.q : 0.f;
      ok = lcg_next(rng_state) < r;
    }
    if (!ok) {
      have = true;
      if (greedy) {
        b = (uint32_t)s.argmax;
      } else {
        float mass = 0.f;
        if ((rc = topk(i, 1, cands, &mass))) return rc;
        if (mass <= 1e-12f) {  // no residual mass: sample the target itself
          if ((rc = topk(i, 0, cands, &mass))) return rc;
          b = sample_candidates(cands.data(), K, 0, 0.f, *sp, rng_state);
        } else {
          b = sample_candidates(cands.data(), K, 1, mass, *sp, rng_state);
        }
      }
    } else {
      ++acc;
      eos = eos_id >= 0 && draft[i] == (uint32_t)eos_id;  // an accepted EOS ends generation unforwarded
    }
  }
  if (!have && !eos) {
    if (greedy) {
      b = (uint32_t)stats[(size_t)k].argmax;
    } else {
      float mass = 0.f;
      if ((rc = topk(k, 0, cands, &mass))) return rc;
      b = sample_candidates(cands.data(), K, 0, 0.f, *sp, rng_state);
    }
  }
  if ((rc = dz_verify_commit(c, eos ? acc - 1 : acc))) return rc;
  *n_accepted = acc;
  *bonus = eos ? 0xFFFFFFFFu : b;
  return DZ_OK;
}

}  // extern "C"
