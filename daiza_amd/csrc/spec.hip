// spec.hip — speculative verify around the device's n-token verify forward:
// the reference's verify loop (Daiza-runtime/src/engine.rs:1255-1470) with Leviathan acceptance
// (leviathan_check, engine.rs:1791-1819), bonus sampling from the residual distribution
// (sample_bonus, engine.rs:1833-1866), temperature/top-k/top-p sampling
// (sample_top_k_top_p_into, Daiza-engine/src/math/sampling.rs:144-247) and its LcgRng
// (sampling.rs:9-19).  The reference forwards each accepted draft one at a time; here all k drafts
// run in one forward (dz_verify_forward) and the accepted prefix is kept (dz_verify_commit).
// Sampling runs on the host over the logits rows, as in the reference.
#include "runtime.h"

#include <algorithm>
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
    auto desc = [&](uint32_t a, uint32_t b) { return scaled[a] > scaled[b]; };
    std::nth_element(idx.begin(), idx.begin() + (k - 1), idx.end(), desc);
    std::stable_sort(idx.begin(), idx.begin() + k, desc);
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

static int check_sampling(const dz_sampling* sp) {
  if (!sp) return set_error(DZ_ERR_TENSOR, "sampling: null parameters");
  if (sp->temperature > 0.f && (sp->top_k < 1 || !(sp->top_p > 0.f)))
    return set_error(DZ_ERR_TENSOR, "sampling: top_k %d, top_p %g", sp->top_k, (double)sp->top_p);
  return DZ_OK;
}

}  // namespace dz

using namespace dz;

extern "C" {

float dz_lcg_next(uint64_t* state) { return state ? lcg_next(state) : 0.f; }

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
  // rows[0]: the context's logits (predict draft[0]); rows[i + 1]: after draft[i]
  std::vector<float> rows((size_t)(k + 1) * V);
  if ((rc = dz_ctx_logits(c, rows.data()))) return rc;
  if ((rc = dz_verify_forward(c, draft, k, rows.data() + V))) return rc;
  Sampler s;
  int acc = 0;
  bool eos = false;
  uint32_t b = 0;
  bool have_bonus = false;
  for (int i = 0; i < k; ++i) {
    const float* tl = rows.data() + (size_t)i * V;
    const float* dl = greedy ? nullptr : draft_logits + (size_t)i * V;
    int ok;
    if (greedy) {
      ok = argmax_of(tl, V) == draft[i];
    } else {
      float p, q;
      softmax_pair_single(tl, dl, V, draft[i], &p, &q);
      const float r = q > 1e-12f ? p / q : 0.f;
      ok = lcg_next(rng_state) < r;
    }
    if (!ok) {
      b = greedy ? (uint32_t)argmax_of(tl, V) : s.bonus(tl, dl, V, *sp, rng_state);
      have_bonus = true;
      break;
    }
    ++acc;
    if (eos_id >= 0 && draft[i] == (uint32_t)eos_id) {  // an accepted EOS ends generation unforwarded
      eos = true;
      break;
    }
  }
  if (!have_bonus && !eos) b = s.top_k_top_p(rows.data() + (size_t)k * V, V, *sp, rng_state);
  if ((rc = dz_verify_commit(c, eos ? acc - 1 : acc))) return rc;
  *n_accepted = acc;
  *bonus = eos ? 0xFFFFFFFFu : b;
  return DZ_OK;
}

}  // extern "C"
