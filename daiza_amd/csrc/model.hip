// model.hip — the batch-1 decode loop on one gfx950 device: weights, context state, the
// per-token kernel sequence (captured once as a hipGraph) and the model-level C ABI
// (forward_single_token / forward_batch / ModelState, Daiza-engine/src/model/forward.rs).
#include "runtime.h"
#include "model_kernels.h"
#include "ptk_kernel.h"
#include "batch_kernels.h"
#include "daiza_synth.h"

#include <cmath>
#include <cstdio>
#include <functional>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

using namespace dz;

namespace dz {

struct LayerDev {
  bool attn = false;
  int kind_idx = 0;                  // index among SSM layers or among attention layers
  float* attn_norm = nullptr;
  float* post_norm = nullptr;
  Q1Dev in_proj, out_proj, gate_up, down;  // in_proj: SSM [qkv|z|alpha|beta], attention [q|k|v]
  float* conv_w = nullptr;           // [4][qkvd], tap 3 newest
  float* ssm_a = nullptr;
  float* dt_bias = nullptr;
  float* ssm_norm = nullptr;
  float* q_norm = nullptr;
  float* k_norm = nullptr;
};

}  // namespace dz

struct dz_model {
  dz_config cfg;
  std::vector<LayerDev> L;
  Q1Dev lm_head;
  float* output_norm = nullptr;
  uint16_t* emb_f16 = nullptr;
  Q1Dev emb_q1;
  uint64_t q1_bytes = 0;
  int n_ssm = 0, n_attn = 0;
  std::vector<void*> allocs;
};

struct dz_ctx {
  dz_model* m = nullptr;
  hipStream_t s = nullptr;
  TokState* st = nullptr;
  int* feed = nullptr;
  int feed_cap = 0;
  int* toklog = nullptr;
  float* emb_row = nullptr;
  float* h[2] = {nullptr, nullptr};
  float* ss[2] = {nullptr, nullptr};
  float *p_in = nullptr, *p_o = nullptr, *p_gu = nullptr, *p_down = nullptr;
  float *y = nullptr, *zs = nullptr, *apart = nullptr, *attn_u = nullptr;
  float *h_fin = nullptr, *ss_fin = nullptr, *logits = nullptr, *am_val = nullptr;
  int* am_idx = nullptr;
  int n_am = 0;
  float* ssm_state = nullptr;  // [n_ssm][nvh][128 i][128 j] (row-major S[i][j], as the API)
  float* conv = nullptr;       // [n_ssm][4][qkvd]
  float* kv = nullptr;         // [n_attn][2][nkv][max_ctx][hd]
  float* rope = nullptr;       // [max_ctx][rope_dim]
  std::vector<int> ring_base;  // per SSM layer
  int* ring_base_dev = nullptr;
  int gmax = 128;  // graph path: attention chunks per kv head (<= 128, attn_merge_kernel's bound)
  int pos_host = 0;            // mirror of TokState::pos_next
  // Set when a token-kernel launch gave up on a bounded wait: the launch may have stored part of a
  // token's state (DeltaNet rows, KV, conv rows) without the position moving, so every forward is
  // refused until dz_ctx_reset (or a full-state restore) makes the state consistent again.
  bool poisoned = false;
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  // persistent token kernel (used by forward_token / forward_batch / decode_greedy when enabled)
  struct {
    bool on = false;
    dz::PtkPlan plan{};
    dz::PtkLayer* layers_d = nullptr;
    int* err = nullptr;           // [4]
    uint64_t* rng = nullptr;      // the sampled selection's generator state
    float* logits_all = nullptr;  // [chunk][vocab]
    int chunk = 32;
    uint64_t gti = 0;             // index of the next token for tags and parity
    const void* kfn = nullptr;    // the greedy instance
    const void* kfn_s = nullptr;  // the sampled instance (null: sampled decode takes the per-token launches)
    const void* kfn_t[2] = {nullptr, nullptr};  // the traced greedy / sampled instances (DAIZA_PTK_TRACE)
  } ptk;
  // n-token forward (prefill, speculative verify): activations [cap][width], grown on demand
  struct {
    int cap = 0;
    std::vector<void*> allocs;
    int* ids = nullptr;
    float *h = nullptr, *yin = nullptr, *cout = nullptr, *qk = nullptr, *ys = nullptr, *gy = nullptr;
    float *ygu = nullptr, *sw = nullptr, *qb = nullptr, *gate = nullptr;
    float* logits = nullptr;  // [logits_rows][vocab]
    int logits_rows = 0;
    dz::Scratch pack, split, arec, spec;
    // verify records per DeltaNet layer: conv inputs [kv][qkvd] and the scan's rollback record
    int kv_cap = 0;
    std::vector<float*> rx;
    std::vector<dz::DnRecord> rec;
    int pending = 0;          // tokens of the last verify forward (0: none)
    std::vector<uint32_t> pending_ids;
  } bt;
  std::vector<void*> allocs;
};

namespace dz {

static int alloc_dev(std::vector<void*>& owner, void** p, size_t bytes) {
  if (bytes == 0) bytes = 16;
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return set_error(DZ_ERR_DEVICE, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  owner.push_back(*p);
  return DZ_OK;
}

template <class T>
static int alloc_t(std::vector<void*>& owner, T** p, size_t n) {
  return alloc_dev(owner, reinterpret_cast<void**>(p), n * sizeof(T));
}

static int upload_f32(std::vector<void*>& owner, float** dst, const float* src, size_t n) {
  int rc = alloc_t(owner, dst, n);
  if (rc) return rc;
  DZ_HIP_CHECK(hipMemcpy(*dst, src, n * 4, hipMemcpyHostToDevice));
  return DZ_OK;
}

// Repacks AoS Q1_0 bytes (host) into the GEMV layout (device); the matrix API does the same.
int upload_q1_host(const uint8_t* aos, int64_t rows, int64_t cols, Q1Dev* out, std::vector<void*>& owner);

static int cfg_check(const dz_config* c) {
  if (!c) return set_error(DZ_ERR_MODEL, "null config");
  if (c->n_layers < 1 || c->hidden < 128 || c->hidden % 128 || c->ffn % 128 || c->vocab < 1)
    return set_error(DZ_ERR_MODEL, "config: bad dimensions");
  if (c->head_dim != 256) return set_error(DZ_ERR_UNSUPPORTED, "head_dim %d (this build: 256)", c->head_dim);
  if (c->ssm_state != 128) return set_error(DZ_ERR_UNSUPPORTED, "ssm_state %d (this build: 128)", c->ssm_state);
  if (c->ssm_conv_kernel != 4) return set_error(DZ_ERR_UNSUPPORTED, "ssm_conv_kernel %d (this build: 4)", c->ssm_conv_kernel);
  if (c->n_head_kv < 1 || c->n_head % c->n_head_kv) return set_error(DZ_ERR_MODEL, "n_head %% n_head_kv != 0");
  const int grp = c->n_head / c->n_head_kv;
  if (grp != 1 && grp != 2 && grp != 3 && grp != 4 && grp != 6 && grp != 8)
    return set_error(DZ_ERR_UNSUPPORTED, "GQA group %d (this build: 1,2,3,4,6,8)", grp);
  if (c->rope_dim < 2 || c->rope_dim > c->head_dim || c->rope_dim % 2) return set_error(DZ_ERR_MODEL, "rope_dim %d", c->rope_dim);
  if (c->ssm_k_heads < 1 || c->ssm_v_heads % c->ssm_k_heads) return set_error(DZ_ERR_MODEL, "ssm heads");
  if (c->max_ctx < 1) return set_error(DZ_ERR_MODEL, "max_ctx %d", c->max_ctx);
  const int64_t kout = std::max<int64_t>((int64_t)c->ssm_v_heads * c->ssm_state, (int64_t)c->n_head * c->head_dim);
  if ((c->hidden + kTileCols - 1) / kTileCols > kMaxTilesH)
    return set_error(DZ_ERR_UNSUPPORTED, "hidden %d > %d", c->hidden, kMaxTilesH * kTileCols);
  if ((c->ffn + kTileCols - 1) / kTileCols > kMaxTilesF || (kout + kTileCols - 1) / kTileCols > kMaxTilesF)
    return set_error(DZ_ERR_UNSUPPORTED, "ffn or mixer width > %d", kMaxTilesF * kTileCols);
  return DZ_OK;
}

static bool is_attn_layer(const dz_config* c, int i) {
  if (c->full_attn_interval == 0) return true;
  return i % c->full_attn_interval == c->full_attn_interval - 1;
}

// ---------------------------------------------------------------- synthetic weights (daiza_synth.h)

static void par_rows(int64_t rows, const std::function<void(int64_t, int64_t)>& fn) {
  unsigned nt = std::thread::hardware_concurrency();
  if (nt < 1) nt = 1;
  if (nt > 16) nt = 16;
  if (rows < 256) nt = 1;
  std::vector<std::thread> th;
  const int64_t per = (rows + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    const int64_t a = t * per, b = std::min<int64_t>(rows, a + per);
    if (a >= b) break;
    th.emplace_back(fn, a, b);
  }
  for (auto& x : th) x.join();
}

// AoS bytes of the synthetic matrix (kind, layer) rows [0, rows) appended to `buf`.
static void synth_q1_append(std::vector<uint8_t>& buf, uint64_t seed, int kind, int layer, int64_t rows, int64_t cols) {
  const size_t rb = (size_t)(cols / kGroup) * kBlockBytes;
  const size_t off = buf.size();
  buf.resize(off + (size_t)rows * rb);
  const uint64_t key = dz_key(seed, (uint32_t)kind, (uint32_t)layer);
  uint8_t* base = buf.data() + off;
  par_rows(rows, [&](int64_t a, int64_t b) { dz_synth_q1_0_rows(key, (uint64_t)cols, (uint64_t)a, (uint64_t)b, base + a * rb); });
}

__global__ void synth_embd_kernel(uint64_t key, int64_t n, uint16_t* out) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) out[i] = dz_f32_to_f16(dz_uniform_f32(key, (uint64_t)i, -1.0f, 1.0f));
}

}  // namespace dz

// ---------------------------------------------------------------- model creation

static int model_finish_common(dz_model* m) {
  const dz_config& c = m->cfg;
  int nssm = 0, nattn = 0;
  for (int i = 0; i < c.n_layers; ++i) {
    LayerDev& l = m->L[i];
    l.kind_idx = l.attn ? nattn++ : nssm++;
  }
  m->n_ssm = nssm;
  m->n_attn = nattn;
  uint64_t b = 0;
  auto q1b = [](const Q1Dev& q) { return (uint64_t)q.rows * (uint64_t)(q.cols / kGroup) * kBlockBytes; };
  for (auto& l : m->L) b += q1b(l.in_proj) + q1b(l.out_proj) + q1b(l.gate_up) + q1b(l.down);
  b += q1b(m->lm_head);
  m->q1_bytes = b;
  return DZ_OK;
}

static void model_release(dz_model* m) {
  if (!m) return;
  for (void* p : m->allocs) (void)hipFree(p);
  delete m;
}

extern "C" int dz_model_create_synth(const dz_config* cfg, uint64_t seed, dz_model** out) {
  int rc = cfg_check(cfg);
  if (rc) return rc;
  if (!out) return set_error(DZ_ERR_MODEL, "null output");
  rc = ensure_device();
  if (rc) return rc;
  dz_model* m = new dz_model();
  m->cfg = *cfg;
  const dz_config& c = *cfg;
  const int64_t H = c.hidden, F = c.ffn, hd = c.ssm_state;
  const int64_t kdim = (int64_t)c.ssm_k_heads * hd, inner = (int64_t)c.ssm_v_heads * hd, qkvd = 2 * kdim + inner;
  const int64_t qdim = (int64_t)c.n_head * c.head_dim, kvdim = (int64_t)c.n_head_kv * c.head_dim;
  m->L.resize(c.n_layers);
  auto fail = [&](int code) { model_release(m); return code; };
  std::vector<uint8_t> buf;
  std::vector<float> fbuf;
  auto uni = [&](int kind, int layer, int64_t n, float lo, float hi, float** dst) {
    fbuf.resize(n);
    dz_synth_uniform_f32(dz_key(seed, (uint32_t)kind, (uint32_t)layer), 0, (uint64_t)n, lo, hi, fbuf.data());
    return upload_f32(m->allocs, dst, fbuf.data(), (size_t)n);
  };
  for (int i = 0; i < c.n_layers; ++i) {
    LayerDev& l = m->L[i];
    l.attn = is_attn_layer(&c, i);
    if ((rc = uni(DZ_K_ATTN_NORM, i, H, 0.8f, 1.2f, &l.attn_norm))) return fail(rc);
    if ((rc = uni(DZ_K_POST_NORM, i, H, 0.8f, 1.2f, &l.post_norm))) return fail(rc);
    buf.clear();
    synth_q1_append(buf, seed, DZ_K_FFN_GATE, i, F, H);
    synth_q1_append(buf, seed, DZ_K_FFN_UP, i, F, H);
    if ((rc = upload_q1_host(buf.data(), 2 * F, H, &l.gate_up, m->allocs))) return fail(rc);
    buf.clear();
    synth_q1_append(buf, seed, DZ_K_FFN_DOWN, i, H, F);
    if ((rc = upload_q1_host(buf.data(), H, F, &l.down, m->allocs))) return fail(rc);
    if (!l.attn) {
      buf.clear();
      synth_q1_append(buf, seed, DZ_K_SSM_QKV, i, qkvd, H);
      synth_q1_append(buf, seed, DZ_K_SSM_Z, i, inner, H);
      synth_q1_append(buf, seed, DZ_K_SSM_ALPHA, i, c.ssm_v_heads, H);
      synth_q1_append(buf, seed, DZ_K_SSM_BETA, i, c.ssm_v_heads, H);
      if ((rc = upload_q1_host(buf.data(), qkvd + inner + 2 * c.ssm_v_heads, H, &l.in_proj, m->allocs))) return fail(rc);
      buf.clear();
      synth_q1_append(buf, seed, DZ_K_SSM_OUT, i, H, inner);
      if ((rc = upload_q1_host(buf.data(), H, inner, &l.out_proj, m->allocs))) return fail(rc);
      // conv1d: GGUF order [qkvd][4], stored tap-major (weights.rs:1339-1356)
      const int64_t ck = c.ssm_conv_kernel;
      std::vector<float> raw((size_t)(qkvd * ck)), tr((size_t)(qkvd * ck));
      dz_synth_normal_f32(dz_key(seed, DZ_K_SSM_CONV, (uint32_t)i), 0, (uint64_t)(qkvd * ck), 0.0, 0.25, raw.data());
      for (int64_t ch = 0; ch < qkvd; ++ch)
        for (int64_t t = 0; t < ck; ++t) tr[(size_t)(t * qkvd + ch)] = raw[(size_t)(ch * ck + t)];
      if ((rc = upload_f32(m->allocs, &l.conv_w, tr.data(), tr.size()))) return fail(rc);
      std::vector<float> v((size_t)c.ssm_v_heads);
      dz_synth_ssm_a(dz_key(seed, DZ_K_SSM_A, (uint32_t)i), (uint64_t)c.ssm_v_heads, v.data());
      if ((rc = upload_f32(m->allocs, &l.ssm_a, v.data(), v.size()))) return fail(rc);
      dz_synth_normal_f32(dz_key(seed, DZ_K_SSM_DT, (uint32_t)i), 0, (uint64_t)c.ssm_v_heads, 0.0, 0.1, v.data());
      if ((rc = upload_f32(m->allocs, &l.dt_bias, v.data(), v.size()))) return fail(rc);
      if ((rc = uni(DZ_K_SSM_NORM, i, hd, 0.8f, 1.2f, &l.ssm_norm))) return fail(rc);
    } else {
      buf.clear();
      synth_q1_append(buf, seed, DZ_K_ATT_Q, i, 2 * qdim, H);
      synth_q1_append(buf, seed, DZ_K_ATT_K, i, kvdim, H);
      synth_q1_append(buf, seed, DZ_K_ATT_V, i, kvdim, H);
      if ((rc = upload_q1_host(buf.data(), 2 * qdim + 2 * kvdim, H, &l.in_proj, m->allocs))) return fail(rc);
      buf.clear();
      synth_q1_append(buf, seed, DZ_K_ATT_O, i, H, qdim);
      if ((rc = upload_q1_host(buf.data(), H, qdim, &l.out_proj, m->allocs))) return fail(rc);
      if ((rc = uni(DZ_K_ATT_QNORM, i, c.head_dim, 0.8f, 1.2f, &l.q_norm))) return fail(rc);
      if ((rc = uni(DZ_K_ATT_KNORM, i, c.head_dim, 0.8f, 1.2f, &l.k_norm))) return fail(rc);
    }
  }
  if ((rc = uni(DZ_K_OUTPUT_NORM, -1, H, 0.8f, 1.2f, &m->output_norm))) return fail(rc);
  buf.clear();
  synth_q1_append(buf, seed, DZ_K_OUTPUT, -1, c.vocab, H);
  if ((rc = upload_q1_host(buf.data(), c.vocab, H, &m->lm_head, m->allocs))) return fail(rc);
  buf.clear();
  buf.shrink_to_fit();
  if (c.embd_f16) {
    const int64_t n = (int64_t)c.vocab * H;
    if ((rc = alloc_t(m->allocs, &m->emb_f16, (size_t)n))) return fail(rc);
    hipLaunchKernelGGL(synth_embd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, lib_stream(),
                       dz_key(seed, DZ_K_EMBD, (uint32_t)-1), n, m->emb_f16);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(lib_stream());
    if (e != hipSuccess) return fail(set_error(DZ_ERR_DEVICE, "embedding synth: %s", hipGetErrorString(e)));
  } else {
    std::vector<uint8_t> eb;
    synth_q1_append(eb, seed, DZ_K_EMBD, -1, c.vocab, H);
    if ((rc = upload_q1_host(eb.data(), c.vocab, H, &m->emb_q1, m->allocs))) return fail(rc);
  }
  model_finish_common(m);
  *out = m;
  return DZ_OK;
}

// GGUF-named host tensors (LoadedWeights::load_all, weights.rs:1308-1379).
extern "C" int dz_model_create(const dz_config* cfg, const dz_tensor* tensors, int n_tensors, dz_model** out) {
  int rc = cfg_check(cfg);
  if (rc) return rc;
  if (!out || (!tensors && n_tensors)) return set_error(DZ_ERR_MODEL, "null argument");
  rc = ensure_device();
  if (rc) return rc;
  std::unordered_map<std::string, const dz_tensor*> byname;
  for (int i = 0; i < n_tensors; ++i) byname[tensors[i].name] = &tensors[i];
  dz_model* m = new dz_model();
  m->cfg = *cfg;
  const dz_config& c = *cfg;
  const int64_t H = c.hidden, F = c.ffn, hd = c.ssm_state;
  const int64_t kdim = (int64_t)c.ssm_k_heads * hd, inner = (int64_t)c.ssm_v_heads * hd, qkvd = 2 * kdim + inner;
  const int64_t qdim = (int64_t)c.n_head * c.head_dim, kvdim = (int64_t)c.n_head_kv * c.head_dim;
  auto fail = [&](int code) { model_release(m); return code; };
  auto find = [&](const std::string& name, int type, size_t bytes, const dz_tensor** t) {
    auto it = byname.find(name);
    if (it == byname.end()) return set_error(DZ_ERR_MODEL, "tensor %s not found", name.c_str());
    if (it->second->type != type) return set_error(DZ_ERR_MODEL, "tensor %s: type %d, expected %d", name.c_str(), it->second->type, type);
    if (it->second->n_bytes != bytes)
      return set_error(DZ_ERR_TENSOR, "tensor %s: %zu bytes, expected %zu", name.c_str(), it->second->n_bytes, bytes);
    *t = it->second;
    return DZ_OK;
  };
  auto q1bytes = [](int64_t r, int64_t k) { return (size_t)r * (size_t)(k / kGroup) * kBlockBytes; };
  std::vector<uint8_t> buf;
  auto cat_q1 = [&](const std::string& name, int64_t rows, int64_t cols) {
    const dz_tensor* t;
    int r = find(name, 41, q1bytes(rows, cols), &t);
    if (r) return r;
    const uint8_t* p = static_cast<const uint8_t*>(t->data);
    buf.insert(buf.end(), p, p + t->n_bytes);
    return DZ_OK;
  };
  auto f32 = [&](const std::string& name, int64_t n, float** dst) {
    const dz_tensor* t;
    int r = find(name, 0, (size_t)n * 4, &t);
    if (r) return r;
    return upload_f32(m->allocs, dst, static_cast<const float*>(t->data), (size_t)n);
  };
  m->L.resize(c.n_layers);
  for (int i = 0; i < c.n_layers; ++i) {
    LayerDev& l = m->L[i];
    l.attn = is_attn_layer(&c, i);
    const std::string b = "blk." + std::to_string(i) + ".";
    if ((rc = f32(b + "attn_norm.weight", H, &l.attn_norm))) return fail(rc);
    if ((rc = f32(b + "post_attention_norm.weight", H, &l.post_norm))) return fail(rc);
    buf.clear();
    if ((rc = cat_q1(b + "ffn_gate.weight", F, H)) || (rc = cat_q1(b + "ffn_up.weight", F, H))) return fail(rc);
    if ((rc = upload_q1_host(buf.data(), 2 * F, H, &l.gate_up, m->allocs))) return fail(rc);
    buf.clear();
    if ((rc = cat_q1(b + "ffn_down.weight", H, F))) return fail(rc);
    if ((rc = upload_q1_host(buf.data(), H, F, &l.down, m->allocs))) return fail(rc);
    if (!l.attn) {
      buf.clear();
      if ((rc = cat_q1(b + "attn_qkv.weight", qkvd, H)) || (rc = cat_q1(b + "attn_gate.weight", inner, H)) ||
          (rc = cat_q1(b + "ssm_alpha.weight", c.ssm_v_heads, H)) || (rc = cat_q1(b + "ssm_beta.weight", c.ssm_v_heads, H)))
        return fail(rc);
      if ((rc = upload_q1_host(buf.data(), qkvd + inner + 2 * c.ssm_v_heads, H, &l.in_proj, m->allocs))) return fail(rc);
      buf.clear();
      if ((rc = cat_q1(b + "ssm_out.weight", H, inner))) return fail(rc);
      if ((rc = upload_q1_host(buf.data(), H, inner, &l.out_proj, m->allocs))) return fail(rc);
      const dz_tensor* t;
      const int64_t ck = c.ssm_conv_kernel;
      if ((rc = find(b + "ssm_conv1d.weight", 0, (size_t)(qkvd * ck) * 4, &t))) return fail(rc);
      const float* raw = static_cast<const float*>(t->data);
      std::vector<float> tr((size_t)(qkvd * ck));
      for (int64_t ch = 0; ch < qkvd; ++ch)
        for (int64_t k = 0; k < ck; ++k) tr[(size_t)(k * qkvd + ch)] = raw[(size_t)(ch * ck + k)];
      if ((rc = upload_f32(m->allocs, &l.conv_w, tr.data(), tr.size()))) return fail(rc);
      if ((rc = f32(b + "ssm_a", c.ssm_v_heads, &l.ssm_a))) return fail(rc);
      if ((rc = f32(b + "ssm_dt.bias", c.ssm_v_heads, &l.dt_bias))) return fail(rc);
      if ((rc = f32(b + "ssm_norm.weight", hd, &l.ssm_norm))) return fail(rc);
    } else {
      buf.clear();
      if ((rc = cat_q1(b + "attn_q.weight", 2 * qdim, H)) || (rc = cat_q1(b + "attn_k.weight", kvdim, H)) ||
          (rc = cat_q1(b + "attn_v.weight", kvdim, H)))
        return fail(rc);
      if ((rc = upload_q1_host(buf.data(), 2 * qdim + 2 * kvdim, H, &l.in_proj, m->allocs))) return fail(rc);
      buf.clear();
      if ((rc = cat_q1(b + "attn_output.weight", H, qdim))) return fail(rc);
      if ((rc = upload_q1_host(buf.data(), H, qdim, &l.out_proj, m->allocs))) return fail(rc);
      if ((rc = f32(b + "attn_q_norm.weight", c.head_dim, &l.q_norm))) return fail(rc);
      if ((rc = f32(b + "attn_k_norm.weight", c.head_dim, &l.k_norm))) return fail(rc);
    }
  }
  if ((rc = f32("output_norm.weight", H, &m->output_norm))) return fail(rc);
  buf.clear();
  if ((rc = cat_q1("output.weight", c.vocab, H))) return fail(rc);
  if ((rc = upload_q1_host(buf.data(), c.vocab, H, &m->lm_head, m->allocs))) return fail(rc);
  buf.clear();
  if (c.embd_f16) {
    const dz_tensor* t;
    if ((rc = find("token_embd.weight", 1, (size_t)c.vocab * H * 2, &t))) return fail(rc);
    if ((rc = alloc_t(m->allocs, &m->emb_f16, (size_t)c.vocab * H))) return fail(rc);
    DZ_HIP_CHECK(hipMemcpy(m->emb_f16, t->data, t->n_bytes, hipMemcpyHostToDevice));
  } else {
    if ((rc = cat_q1("token_embd.weight", c.vocab, H))) return fail(rc);
    if ((rc = upload_q1_host(buf.data(), c.vocab, H, &m->emb_q1, m->allocs))) return fail(rc);
  }
  model_finish_common(m);
  *out = m;
  return DZ_OK;
}

extern "C" int dz_model_free(dz_model* m) {
  model_release(m);
  return DZ_OK;
}

extern "C" int dz_model_weight_bytes(const dz_model* m, uint64_t* q1_bytes) {
  if (!m || !q1_bytes) return set_error(DZ_ERR_MODEL, "null argument");
  *q1_bytes = m->q1_bytes;
  return DZ_OK;
}

// ---------------------------------------------------------------- context

namespace dz {

static int ctx_dims(const dz_model* m, int64_t* ld_in, int64_t* ld_h, int64_t* ld_gu, int* th, int* to, int* tf) {
  const dz_config& c = m->cfg;
  int64_t mx = 0;
  for (auto& l : m->L) mx = std::max<int64_t>(mx, l.in_proj.nrb * kRowBlock);
  *ld_in = mx;
  *ld_h = ((int64_t)c.hidden + kRowBlock - 1) / kRowBlock * kRowBlock;
  *ld_gu = (2 * (int64_t)c.ffn + kRowBlock - 1) / kRowBlock * kRowBlock;
  *th = (int)((c.hidden + kTileCols - 1) / kTileCols);
  int64_t ko = std::max<int64_t>((int64_t)c.ssm_v_heads * c.ssm_state, (int64_t)c.n_head * c.head_dim);
  *to = (int)((ko + kTileCols - 1) / kTileCols);
  *tf = (int)((c.ffn + kTileCols - 1) / kTileCols);
  return DZ_OK;
}

static void rope_table(const dz_config& c, std::vector<float>& out) {
  // rope.rs:27-38 and 82-101: freq_i = 1 / base^(2i/d); theta = (pos as f32) * freq_i
  const int half = c.rope_dim / 2;
  std::vector<float> fr(half);
  for (int i = 0; i < half; ++i) fr[i] = 1.0f / powf(c.rope_base, (float)(2 * i) / (float)c.rope_dim);
  out.resize((size_t)c.max_ctx * c.rope_dim);
  for (int p = 0; p < c.max_ctx; ++p)
    for (int i = 0; i < half; ++i) {
      const float th = (float)p * fr[i];
      out[(size_t)p * c.rope_dim + i] = cosf(th);
      out[(size_t)p * c.rope_dim + half + i] = sinf(th);
    }
}

template <class Src, class Dst>
static int gemv(const Q1Dev& mat, int tpw, const Src& src, const Dst& dst, hipStream_t s, int64_t* ld = nullptr) {
  const Q1Dev* ms[1] = {&mat};
  GemvPlan p;
  int rc = plan_gemv(ms, 1, tpw, &p);
  if (rc) return rc;
  if (ld) *ld = p.ld;
  DZ_HIP_CHECK(launch_gemv(p, src, dst, s));
  return DZ_OK;
}

static int launch_attention(int grp, dim3 grid, const AttnArgs& a, hipStream_t s) {
  return with_np_bucket(a.np, [&](auto B) -> int {
    constexpr int NB = decltype(B)::value;
    switch (grp) {
      case 1: hipLaunchKernelGGL((attention_kernel<1, NB>), grid, dim3(256), 0, s, a); break;
      case 2: hipLaunchKernelGGL((attention_kernel<2, NB>), grid, dim3(256), 0, s, a); break;
      case 3: hipLaunchKernelGGL((attention_kernel<3, NB>), grid, dim3(256), 0, s, a); break;
      case 4: hipLaunchKernelGGL((attention_kernel<4, NB>), grid, dim3(256), 0, s, a); break;
      case 6: hipLaunchKernelGGL((attention_kernel<6, NB>), grid, dim3(256), 0, s, a); break;
      case 8: hipLaunchKernelGGL((attention_kernel<8, NB>), grid, dim3(256), 0, s, a); break;
      default: return set_error(DZ_ERR_UNSUPPORTED, "GQA group %d", grp);
    }
    DZ_HIP_CHECK(hipGetLastError());
    return DZ_OK;
  });
}

// The mixer of one layer on the residual held in (h_in + parts): norm + in-proj GEMV, then the
// DeltaNet or attention kernel, then the out-projection GEMV into p_o.  `h_mid` receives the
// materialised layer input with its tile sums of squares in `ss_mid`.
static int enqueue_mixer(dz_ctx* x, int li, const float* h_in, const float* parts, int np, int64_t ldp, float* h_mid,
                         float* ss_mid, hipStream_t s, int pos = -1) {
  dz_model* m = x->m;
  const dz_config& c = m->cfg;
  LayerDev& l = m->L[li];
  int64_t ld_in, ld_h, ld_gu;
  int th, to, tf;
  ctx_dims(m, &ld_in, &ld_h, &ld_gu, &th, &to, &tf);
  const int64_t H = c.hidden, hd = c.ssm_state;
  const int64_t kdim = (int64_t)c.ssm_k_heads * hd, inner = (int64_t)c.ssm_v_heads * hd, qkvd = 2 * kdim + inner;
  int rc;
  int64_t ld_l = 0;
  rc = with_np_bucket(np, [&](auto B) -> int {
    ResidSrc<decltype(B)::value> src{h_in, parts, np, ldp, l.attn_norm, h_mid, ss_mid, H};
    PartialDst dst{x->p_in, l.in_proj.nrb * kRowBlock};
    return gemv(l.in_proj, 1, src, dst, s, &ld_l);
  });
  if (rc) return rc;
  const int nin = (int)l.in_proj.ntiles;
  if (!l.attn) {
    DeltaArgs a;
    a.st = x->st;
    a.pos = pos;
    a.p_in = x->p_in;
    a.np = nin;
    a.ldp = ld_l;
    a.ss = ss_mid;
    a.nss = th;
    a.H = H;
    a.rms_eps = c.rms_eps;
    a.conv = x->conv + (size_t)l.kind_idx * 4 * qkvd;
    a.conv_w = l.conv_w;
    a.ssm_a = l.ssm_a;
    a.dt_bias = l.dt_bias;
    a.state = x->ssm_state + (size_t)l.kind_idx * c.ssm_v_heads * hd * hd;
    a.y = x->y;
    a.zs = x->zs;
    a.nkh = c.ssm_k_heads;
    a.nvh = c.ssm_v_heads;
    a.qkvd = qkvd;
    a.off_z = qkvd;
    a.off_a = qkvd + inner;
    a.off_b = qkvd + inner + c.ssm_v_heads;
    a.ring_base_ptr = x->ring_base_dev + l.kind_idx;
    rc = with_np_bucket(nin, [&](auto B) -> int {
      hipLaunchKernelGGL(deltanet_kernel<decltype(B)::value>, dim3((unsigned)(c.ssm_v_heads * 4)), dim3(256), 0, s, a);
      DZ_HIP_CHECK(hipGetLastError());
      return DZ_OK;
    });
    if (rc) return rc;
    GatedYSrc src{x->y, x->zs, l.ssm_norm, inner, 1e-6f};
    PartialDst dst{x->p_o, ld_h};
    if ((rc = gemv(l.out_proj, 1, src, dst, s))) return rc;
  } else {
    AttnArgs a;
    a.st = x->st;
    a.pos = pos;
    a.p_in = x->p_in;
    a.np = nin;
    a.ldp = ld_l;
    a.ss = ss_mid;
    a.nss = th;
    a.H = H;
    a.eps = c.rms_eps;
    a.q_norm = l.q_norm;
    a.k_norm = l.k_norm;
    a.rope = x->rope;
    a.rope_dim = c.rope_dim;
    const size_t kvsz = (size_t)c.n_head_kv * c.max_ctx * c.head_dim;
    a.kcache = x->kv + (size_t)l.kind_idx * 2 * kvsz;
    a.vcache = a.kcache + kvsz;
    a.max_ctx = c.max_ctx;
    a.apart = x->apart;
    a.gmax = x->gmax;
    a.nq = c.n_head;
    a.nkv = c.n_head_kv;
    if ((rc = launch_attention(c.n_head / c.n_head_kv, dim3((unsigned)(c.n_head_kv * x->gmax)), a, s))) return rc;
    // merge the chunks and gate once, then the out-projection reads the result as a plain vector
    AttnMergeArgs ma{x->apart, x->gmax, c.head_dim, x->st, pos, x->p_in, nin, ld_l, ss_mid, th, H, c.rms_eps, x->attn_u};
    rc = with_np_bucket(nin, [&](auto B) -> int {
      hipLaunchKernelGGL(attn_merge_kernel<decltype(B)::value>, dim3((unsigned)(c.n_head * (c.head_dim / 64))),
                         dim3(256), 0, s, ma);
      DZ_HIP_CHECK(hipGetLastError());
      return DZ_OK;
    });
    if (rc) return rc;
    PlainSrc src{x->attn_u, (int64_t)c.n_head * c.head_dim};
    PartialDst dst{x->p_o, ld_h};
    if ((rc = gemv(l.out_proj, 1, src, dst, s))) return rc;
  }
  return DZ_OK;
}

// One token (forward_single_token): select/embed, all blocks, final norm, lm_head.
static int enqueue_token(dz_ctx* x, hipStream_t s) {
  dz_model* m = x->m;
  const dz_config& c = m->cfg;
  int64_t ld_in, ld_h, ld_gu;
  int th, to, tf;
  ctx_dims(m, &ld_in, &ld_h, &ld_gu, &th, &to, &tf);
  const int64_t H = c.hidden, F = c.ffn;
  int rc;
  SelectArgs sa;
  sa.st = x->st;
  sa.feed = x->feed;
  sa.am_val = x->am_val;
  sa.am_idx = x->am_idx;
  sa.n_am = x->n_am;
  sa.toklog = x->toklog;
  sa.emb_f16 = m->emb_f16;
  sa.emb_q1 = m->emb_q1.data;
  sa.emb_ntiles = m->emb_q1.ntiles;
  sa.H = H;
  sa.emb_out = x->emb_row;
  sa.commit = 1;
  hipLaunchKernelGGL(select_token_kernel, dim3(1), dim3(1024), 0, s, sa);
  DZ_HIP_CHECK(hipGetLastError());
  for (int li = 0; li < c.n_layers; ++li) {
    LayerDev& l = m->L[li];
    const float* h_in = li == 0 ? x->emb_row : x->h[1];
    const int np = li == 0 ? 0 : (int)m->L[li - 1].down.ntiles;
    if ((rc = enqueue_mixer(x, li, h_in, x->p_down, np, ld_h, x->h[0], x->ss[0], s))) return rc;
    // post-attention norm + gate/up (block.rs:101-120, mlp.rs:28-47)
    rc = with_np_bucket((int)l.out_proj.ntiles, [&](auto B) -> int {
      ResidSrc<decltype(B)::value> src{x->h[0], x->p_o, (int)l.out_proj.ntiles, ld_h, l.post_norm, x->h[1], x->ss[1], H};
      PartialDst dst{x->p_gu, ld_gu};
      return gemv(l.gate_up, 1, src, dst, s);
    });
    if (rc) return rc;
    rc = with_np_bucket((int)l.gate_up.ntiles, [&](auto B) -> int {
      SwigluSrc<decltype(B)::value> src{x->p_gu, (int)l.gate_up.ntiles, ld_gu, F, x->ss[1], th, H, c.rms_eps};
      PartialDst dst{x->p_down, ld_h};
      return gemv(l.down, 1, src, dst, s);
    });
    if (rc) return rc;
  }
  FinalArgs fa{x->h[1], x->p_down, (int)m->L[c.n_layers - 1].down.ntiles, ld_h, x->h_fin, x->ss_fin, H};
  rc = with_np_bucket(fa.np, [&](auto B) -> int {
    hipLaunchKernelGGL(final_reduce_kernel<decltype(B)::value>, dim3((unsigned)th), dim3(512), 0, s, fa);
    DZ_HIP_CHECK(hipGetLastError());
    return DZ_OK;
  });
  if (rc) return rc;
  NormedSrc src{x->h_fin, m->output_norm, x->ss_fin, th, H, c.rms_eps};
  LogitsDst dst{x->logits, c.vocab, x->am_val, x->am_idx};
  if ((rc = gemv(m->lm_head, (int)m->lm_head.ntiles, src, dst, s))) return rc;
  return DZ_OK;
}

template <class Src, class Dst>
static int set_gemv_attr() {
  DZ_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(gemv_lut_kernel<kGemvWaves, kGemvM, Src, Dst>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, kGemvShmemMax));
  return DZ_OK;
}

}  // namespace dz

// Dynamic-LDS limits of every GEMV instantiation, set once before any launch or graph capture.
int dz::prepare_gemv_kernels() {
  static bool done = false;
  if (done) return DZ_OK;
  int rc;
  for (int np : {2, 4, 8, 12, 16, 24, 36, 48}) {
    rc = with_np_bucket(np, [&](auto B) -> int {
      constexpr int NB = decltype(B)::value;
      int r;
      if ((r = set_gemv_attr<ResidSrc<NB>, PartialDst>())) return r;
      return set_gemv_attr<SwigluSrc<NB>, PartialDst>();
    });
    if (rc) return rc;
  }
  if ((rc = set_gemv_attr<GatedYSrc, PartialDst>())) return rc;
  if ((rc = set_gemv_attr<NormedSrc, LogitsDst>())) return rc;
  if ((rc = set_gemv_attr<PlainSrc, PartialDst>())) return rc;
  done = true;
  return DZ_OK;
}

namespace dz {

static int ctx_build_graph(dz_ctx* x) {
  if (x->gexec) return DZ_OK;
  DZ_HIP_CHECK(hipStreamBeginCapture(x->s, hipStreamCaptureModeThreadLocal));
  int rc = enqueue_token(x, x->s);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(x->s, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return set_error(DZ_ERR_DEVICE, "graph capture: %s", hipGetErrorString(e));
  e = hipGraphInstantiate(&x->gexec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return set_error(DZ_ERR_DEVICE, "graph instantiate: %s", hipGetErrorString(e));
  }
  x->graph = g;
  return DZ_OK;
}

}  // namespace dz

// ---------------------------------------------------------------- context C ABI

namespace dz {

static void bt_release(dz_ctx* x);

static void ctx_release(dz_ctx* x) {
  if (!x) return;
  if (x->gexec) (void)hipGraphExecDestroy(x->gexec);
  if (x->graph) (void)hipGraphDestroy(x->graph);
  if (x->s) (void)hipStreamSynchronize(x->s);
  bt_release(x);
  for (void* p : x->allocs) (void)hipFree(p);
  if (x->s) (void)hipStreamDestroy(x->s);
  delete x;
}

static int ctx_zero_state(dz_ctx* x) {
  const dz_config& c = x->m->cfg;
  const int64_t hd = c.ssm_state, qkvd = (2 * (int64_t)c.ssm_k_heads + c.ssm_v_heads) * hd;
  const size_t kvsz = (size_t)c.n_head_kv * c.max_ctx * c.head_dim;
  if (x->m->n_ssm) {
    DZ_HIP_CHECK(hipMemsetAsync(x->ssm_state, 0, (size_t)x->m->n_ssm * c.ssm_v_heads * hd * hd * 4, x->s));
    DZ_HIP_CHECK(hipMemsetAsync(x->conv, 0, (size_t)x->m->n_ssm * 4 * qkvd * 4, x->s));
    DZ_HIP_CHECK(hipMemsetAsync(x->ring_base_dev, 0, (size_t)x->m->n_ssm * 4, x->s));
  }
  if (x->m->n_attn) DZ_HIP_CHECK(hipMemsetAsync(x->kv, 0, (size_t)x->m->n_attn * 2 * kvsz * 4, x->s));
  std::fill(x->ring_base.begin(), x->ring_base.end(), 0);
  TokState st;
  memset(&st, 0, sizeof st);
  DZ_HIP_CHECK(hipMemcpyAsync(x->st, &st, sizeof st, hipMemcpyHostToDevice, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  x->pos_host = 0;
  x->poisoned = false;
  return DZ_OK;
}

// Host-fed token ids consumed by the next forwards (TokState::feed_len / feed_idx).
static int ctx_feed(dz_ctx* x, const uint32_t* ids, int n) {
  if (n > x->feed_cap) return set_error(DZ_ERR_TENSOR, "feed of %d ids exceeds capacity %d", n, x->feed_cap);
  for (int i = 0; i < n; ++i)
    if (ids[i] >= (uint32_t)x->m->cfg.vocab) return set_error(DZ_ERR_TENSOR, "token id %u >= vocab %d", ids[i], x->m->cfg.vocab);
  if (n) DZ_HIP_CHECK(hipMemcpyAsync(x->feed, ids, (size_t)n * 4, hipMemcpyHostToDevice, x->s));
  int two[2] = {n, 0};
  DZ_HIP_CHECK(hipMemcpyAsync(reinterpret_cast<char*>(x->st) + offsetof(TokState, feed_len), two, sizeof two,
                              hipMemcpyHostToDevice, x->s));
  // the copies above read pageable host memory: make them complete before `ids` may change
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return DZ_OK;
}

// DAIZA_GRAPH=0 enqueues each token's kernels directly instead of replaying the captured graph
// (same kernels and arguments; for tools that do not trace graph launches).
static bool use_graph() {
  static int v = -1;
  if (v < 0) {
    const char* e = getenv("DAIZA_GRAPH");
    v = (e && e[0] == '0') ? 0 : 1;
  }
  return v == 1;
}

static int ctx_run(dz_ctx* x, int n) {
  if (x->pos_host + n > x->m->cfg.max_ctx)
    return set_error(DZ_ERR_TENSOR, "context full: pos %d + %d > max_ctx %d", x->pos_host, n, x->m->cfg.max_ctx);
  if (use_graph()) {
    int rc = ctx_build_graph(x);
    if (rc) return rc;
    for (int i = 0; i < n; ++i) DZ_HIP_CHECK(hipGraphLaunch(x->gexec, x->s));
  } else {
    for (int i = 0; i < n; ++i) {
      int rc = enqueue_token(x, x->s);
      if (rc) return rc;
    }
  }
  x->pos_host += n;
  return DZ_OK;
}

// Writes the greedy token of the current logits to toklog[pos_next] without consuming it.
static int ctx_peek_argmax(dz_ctx* x) {
  SelectArgs sa;
  memset(&sa, 0, sizeof sa);
  sa.st = x->st;
  sa.feed = x->feed;
  sa.am_val = x->am_val;
  sa.am_idx = x->am_idx;
  sa.n_am = x->n_am;
  sa.toklog = x->toklog;
  sa.H = x->m->cfg.hidden;
  sa.commit = 0;
  hipLaunchKernelGGL(select_token_kernel, dim3(1), dim3(1024), 0, x->s, sa);
  DZ_HIP_CHECK(hipGetLastError());
  return DZ_OK;
}

static int ctx_set_pos_dev(dz_ctx* x, int pos);

// Moves the position to pos while every DeltaNet layer's conv-ring head stays where it is: heads are
// stored relative to the position ((ring_base + pos) & 3), so each base is rebased by the move.
// SsmState::conv_head (cache/ssm_state.rs:10-39) is independent of the KV length, and neither
// KvCache::truncate (kv_cache.rs:119-130) nor a position change touches it.
static int ctx_move_pos(dz_ctx* x, int pos) {
  const int old = x->pos_host;
  for (size_t i = 0; i < x->ring_base.size(); ++i) x->ring_base[i] = ((x->ring_base[i] + old - pos) % 4 + 4) % 4;
  if (!x->ring_base.empty())
    DZ_HIP_CHECK(hipMemcpy(x->ring_base_dev, x->ring_base.data(), x->ring_base.size() * 4, hipMemcpyHostToDevice));
  return ctx_set_pos_dev(x, pos);
}

// Refuses work on a context whose last token-kernel launch gave up part-way.
int ctx_usable(const dz_ctx* x) {
  if (x->poisoned)
    return set_error(DZ_ERR_DEVICE, "context state is inconsistent after a failed launch: call dz_ctx_reset");
  return DZ_OK;
}

static int ctx_set_pos_dev(dz_ctx* x, int pos) {
  int v[2] = {pos, pos};  // TokState.pos_next and a consistent .pos for direct mixer launches
  DZ_HIP_CHECK(hipMemcpyAsync(reinterpret_cast<char*>(x->st) + offsetof(TokState, pos_next), &v[0], 4,
                              hipMemcpyHostToDevice, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  x->pos_host = pos;
  return DZ_OK;
}

// ---------------------------------------------------------------- persistent token kernel (host)

static const void* ptk_pick(const PtkShape& s) {
  if (ptk_fits(s, kPtkShape27b)) return reinterpret_cast<const void*>(ptk_kernel<10, 6, 2, 1, 4, 2, 3, 12, 3, 2, 32>);
  if (ptk_fits(s, kPtkShapeSmall)) return reinterpret_cast<const void*>(ptk_kernel<1, 2, 1, 1, 1, 1, 3, 4, 1, 1, 8>);
  return nullptr;
}

// DAIZA_PTK=0 selects the graph path for new contexts.
static bool ptk_wanted() {
  const char* e = getenv("DAIZA_PTK");
  return !(e && e[0] == '0');
}

// Builds the plan of a context; leaves ptk.on false when the shape or the device does not fit.
static int ptk_prepare(dz_ctx* x) {
  dz_model* m = x->m;
  const dz_config& c = m->cfg;
  int dev = 0;
  DZ_HIP_CHECK(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  DZ_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
  const int G = prop.multiProcessorCount;
  int64_t ld_in, ld_h, ld_gu;
  int th, to, tf;
  ctx_dims(m, &ld_in, &ld_h, &ld_gu, &th, &to, &tf);
  const int grp = c.n_head / c.n_head_kv;
  if (c.head_dim != 256 || c.rope_dim != 64 || c.ssm_state != 128 || G < 8 || G > kPtkThreads ||
      c.n_layers > kPtkMaxLayers || th > kMaxTilesH || c.hidden < G)
    return DZ_OK;
  // workgroup roles: GEMV workgroups [0, Gp), reducers [Gp, G) (one in eight)
  const int NR = std::max(8, G / 8), Gp = G - NR;
  // shape limits of the static work split: row-block slots per compute wave of each matrix kind
  const int nrb_h = (int)(ld_h / kRowBlock), nrb_gu = (int)(ld_gu / kRowBlock), nrb_v = (int)m->lm_head.nrb;
  auto slots = [&](int T, int nrb) {
    if (T > Gp) return 1 << 20;
    int mx = 0;
    for (int t = 0; t < T; ++t) {
      const int nw = tile_first_wg(t + 1, T, Gp) - tile_first_wg(t, T, Gp);
      mx = std::max(mx, (nrb + nw - 1) / nw);
    }
    return (mx + kLW - 1) / kLW;  // layer GEMVs: every wave runs lookups
  };
  auto per = [](int n, int k) { return (n + k - 1) / k; };  // items per part of an even split
  const int nc = per(c.hidden, NR);                        // reducer residual columns per workgroup
  auto resid_q = [&](int np) {                             // terms per thread of a residual sum
    const int K = np + 1, nq = std::min(kPtkThreads / nc, K);
    return per(K, nq);
  };
  PtkShape sh{th, grp, 0, 0, slots(th, nrb_gu), slots(tf, nrb_h), per(per(nrb_v, G), kCW), 0,
              per(2 * per(c.ffn, NR), kPtkThreads), 0, per(c.n_head * c.head_dim, Gp)};
  int max_rows_in = 0;
  for (auto& l : m->L) {
    sh.u_in = std::max(sh.u_in, slots(th, (int)l.in_proj.nrb));
    sh.u_out = std::max(sh.u_out, slots((int)l.out_proj.ntiles, nrb_h));
    sh.qr = std::max(sh.qr, resid_q((int)l.out_proj.ntiles));
    max_rows_in = std::max(max_rows_in, (int)l.in_proj.rows);
  }
  sh.qr = std::max(sh.qr, resid_q(tf));
  sh.mr = per(per(max_rows_in, NR), kPtkThreads);
  if (nc > kPtkThreads || sh.mo > 64 || sh.mo > c.head_dim || 2 * per(c.ffn, NR) * 4 > kLdsScratchBytes) return DZ_OK;
  const void* kfn = ptk_pick(sh);
  if (!kfn) return DZ_OK;
  int occ = 0;
  DZ_HIP_CHECK(hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPtkLds));
  DZ_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kfn, kPtkThreads, kPtkLds));
  // one workgroup per CU, all G of them resident at once: the hand-overs need every workgroup
  // running (a short grid is caught by the bounded waits: DZ_ERR_DEVICE, never a hang)
  if (occ < 1) return DZ_OK;
  const int gmax = std::min(64, Gp / std::max(1, c.n_head_kv));
  if (4 * c.ssm_v_heads > Gp || c.n_head_kv * gmax > Gp || gmax < 1) return DZ_OK;
  PtkPlan& P = x->ptk.plan;
  memset(&P, 0, sizeof P);
  P.G = G;
  P.Gp = Gp;
  P.NR = NR;
  P.n_layers = c.n_layers;
  P.H = c.hidden;
  P.F = c.ffn;
  P.vocab = c.vocab;
  P.nT_h = th;
  P.nrb_h = nrb_h;
  P.nT_f = tf;
  P.nrb_gu = nrb_gu;
  P.nrb_v = nrb_v;
  const int hd = c.ssm_state;
  P.nkh = c.ssm_k_heads;
  P.nvh = c.ssm_v_heads;
  P.inner = c.ssm_v_heads * hd;
  P.qkvd = 2 * c.ssm_k_heads * hd + P.inner;
  P.off_z = P.qkvd;
  P.off_a = P.qkvd + P.inner;
  P.off_b = P.qkvd + P.inner + c.ssm_v_heads;
  P.nq = c.n_head;
  P.nkv = c.n_head_kv;
  P.hd = c.head_dim;
  P.rope_dim = c.rope_dim;
  P.grp = grp;
  P.gmax = gmax;
  P.max_ctx = c.max_ctx;
  P.eps = c.rms_eps;
  P.embd_f16 = c.embd_f16;
  // LL layout of one layer region (64-word aligned sub-buffers)
  auto al = [](int64_t v) { return (v + 63) / 64 * 64; };
  int64_t o = 0;
  auto take = [&](int64_t n) { const int64_t r = o; o += al(n); return r; };
  const int64_t qdim = (int64_t)c.n_head * c.head_dim;
  const int64_t attn_rows = 2 * qdim + 2 * (int64_t)c.n_head_kv * c.head_dim;
  P.off.pin = take((int64_t)th * ld_in);
  P.off.sst_in = take(th);
  P.off.po = take((int64_t)to * ld_h);
  P.off.hmid = take(ld_h);
  P.off.sst_mid = take(th);
  P.off.pgu = take((int64_t)th * ld_gu);
  P.off.sw = take((int64_t)tf * kTileCols);
  P.off.pd = take((int64_t)tf * ld_h);
  P.off.h = take(ld_h);
  P.off.y = take(P.inner);
  P.off.zs = take(P.inner);
  P.off.yss = take(16 * (int64_t)P.nvh);
  P.off.qkv = take(std::max<int64_t>(attn_rows, max_rows_in));
  P.off.rec = take((int64_t)c.n_head * gmax * (2 + c.head_dim));
  P.off.ao = take(qdim);
  P.off.words = std::max<int64_t>(o, al(ptk_samp_off(ld_h, G) + ptk_samp_words(G)));
  // phases: S, then 9 per DeltaNet layer / 10 per attention layer, then L
  std::vector<PtkLayer> Ls((size_t)c.n_layers);
  const size_t kvsz = (size_t)c.n_head_kv * c.max_ctx * c.head_dim;
  const int64_t hd2 = hd;
  const int64_t qkvd = P.qkvd;
  int ph = 1;
  for (int i = 0; i < c.n_layers; ++i) {
    LayerDev& l = m->L[i];
    PtkLayer& y = Ls[(size_t)i];
    memset(&y, 0, sizeof y);
    y.attn = l.attn ? 1 : 0;
    y.rows_in = (int)l.in_proj.rows;
    y.nrb_in = (int)l.in_proj.nrb;
    y.nt_out = (int)l.out_proj.ntiles;
    y.w_in = l.in_proj.data;
    y.w_out = l.out_proj.data;
    y.w_gu = l.gate_up.data;
    y.w_dn = l.down.data;
    y.attn_norm = l.attn_norm;
    y.post_norm = l.post_norm;
    if (!l.attn) {
      y.conv_w = l.conv_w;
      y.ssm_a = l.ssm_a;
      y.dt_bias = l.dt_bias;
      y.ssm_norm = l.ssm_norm;
      y.conv = x->conv + (size_t)l.kind_idx * 4 * qkvd;
      y.state = x->ssm_state + (size_t)l.kind_idx * c.ssm_v_heads * hd2 * hd2;
      y.ring_base = x->ring_base_dev + l.kind_idx;
    } else {
      y.q_norm = l.q_norm;
      y.k_norm = l.k_norm;
      y.kc = x->kv + (size_t)l.kind_idx * 2 * kvsz;
      y.vc = y.kc + kvsz;
    }
    y.ph0 = ph;
    ph += l.attn ? 10 : 9;
  }
  // the kernel assigns GEMV work per matrix kind: every layer of a kind has the same shapes
  P.nrb_in_k[0] = P.nrb_in_k[1] = P.nt_out_k[0] = P.nt_out_k[1] = -1;
  for (const PtkLayer& y : Ls) {
    int& nrb = P.nrb_in_k[y.attn];
    int& nto = P.nt_out_k[y.attn];
    if ((nrb >= 0 && nrb != y.nrb_in) || (nto >= 0 && nto != y.nt_out)) return DZ_OK;
    nrb = y.nrb_in;
    nto = y.nt_out;
  }
  for (int k = 0; k < 2; ++k)
    if (P.nrb_in_k[k] < 0) P.nrb_in_k[k] = P.nt_out_k[k] = 1;
  P.ph_l = ph;
  P.ppt = ph + 1;
  P.w_lm = m->lm_head.data;
  P.output_norm = m->output_norm;
  P.emb_f16 = m->emb_f16;
  P.emb_q1 = m->emb_q1.data;
  P.emb_ntiles = (int)m->emb_q1.ntiles;
  P.rope = x->rope;
  P.st = x->st;
  P.toklog = x->toklog;
  P.logits = x->logits;
  auto& A = x->allocs;
  int rc;
  const size_t ll_words = (size_t)2 * (c.n_layers + 1) * (size_t)P.off.words;
  if ((rc = alloc_t(A, &P.ll, ll_words)) || (rc = alloc_t(A, &x->ptk.layers_d, Ls.size())) ||
      (rc = alloc_t(A, &x->ptk.err, 4)) || (rc = alloc_t(A, &x->ptk.rng, 1)) ||
      (rc = alloc_t(A, &x->ptk.logits_all, (size_t)x->ptk.chunk * c.vocab)))
    return rc;
  DZ_HIP_CHECK(hipMemset(P.ll, 0, ll_words * sizeof(u64)));
  DZ_HIP_CHECK(hipMemset(x->ptk.err, 0, 16));
  DZ_HIP_CHECK(hipMemcpy(x->ptk.layers_d, Ls.data(), Ls.size() * sizeof(PtkLayer), hipMemcpyHostToDevice));
  P.L = x->ptk.layers_d;
  x->ptk.kfn = kfn;
  // the sampled instance, where it fits one workgroup per CU as the greedy one does
  const void* kfn_s = ptk_pick_samp(sh);
  int occ_s = 0;
  DZ_HIP_CHECK(hipFuncSetAttribute(kfn_s, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPtkLds));
  DZ_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ_s, kfn_s, kPtkThreads, kPtkLds));
  x->ptk.kfn_s = occ_s >= 1 ? kfn_s : nullptr;
  for (int t = 0; t < 2; ++t) {
    x->ptk.kfn_t[t] = ptk_pick_trace(sh, t == 1);
    DZ_HIP_CHECK(hipFuncSetAttribute(x->ptk.kfn_t[t], hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPtkLds));
  }
  x->ptk.gti = 0;
  x->ptk.on = true;
  return DZ_OK;
}

// One launch of the token kernel on the context's stream.  A plain launch of G workgroups, one per
// CU (the occupancy query at plan time found room for one per CU, and more than 80 KiB of LDS keeps a
// second one off each CU): every workgroup is resident once the device is otherwise idle, which the
// hand-overs need; should one not start, the others' bounded waits end the launch with an error.
// DAIZA_PTK_COOP=1 asks for a cooperative launch instead, whose residency guarantee comes from the
// runtime (profilers on this stack fault at process exit after a cooperative launch).
static int ptk_launch(dz_ctx* x, PtkRun& r) {
  void* args[] = {&r};
  const PtkPlan& P = x->ptk.plan;
  const void* kfn = r.trace ? x->ptk.kfn_t[r.samp.k > 0] : r.samp.k > 0 ? x->ptk.kfn_s : x->ptk.kfn;
  if (!kfn) return set_error(DZ_ERR_UNSUPPORTED, "token kernel: no instance for this run");
  const char* coop = getenv("DAIZA_PTK_COOP");
  if (coop && coop[0] == '1')
    DZ_HIP_CHECK(hipLaunchCooperativeKernel(kfn, dim3((unsigned)P.G), dim3(kPtkThreads), args, kPtkLds, x->s));
  else
    DZ_HIP_CHECK(hipLaunchKernel(kfn, dim3((unsigned)P.G), dim3(kPtkThreads), args, kPtkLds, x->s));
  return DZ_OK;
}

// The wait bound of a launch: DAIZA_PTK_SPIN=<n> lowers it (a wait that gives up ends the launch with
// DZ_ERR_DEVICE); for tests of the failure path, which must stay on the host's side.
static int ptk_spin_limit() {
  if (const char* sl = getenv("DAIZA_PTK_SPIN")) {
    const long v = strtol(sl, nullptr, 10);
    if (v > 0 && v < (1 << 21)) return (int)v;
  }
  return 1 << 21;
}

// Runs n tokens at positions pos_host.. in one launch: tokens [0, n_feed) take the fed
// ids (already in x->feed), the rest the greedy pick.  toklog[pos + i] receives token i and
// toklog[pos + n] the greedy pick after the last one; logits of the last token land in x->logits,
// and with per_pos every token's logits in ptk.logits_all[i] (n <= ptk.chunk).
// With eos >= 0 a greedy pick equal to eos ends the launch before that token is forwarded; *n_done
// (if given) receives the number of tokens forwarded and the position advances by that many.
// With smp.k > 0 the tokens past the fed ones (and the pick after the last) are drawn on the device
// from the previous logits' smp.k best instead of the greedy pick.
static int ptk_run(dz_ctx* x, int n, int n_feed, bool per_pos, int feed_off = 0, int eos = -1, int* n_done = nullptr,
                   const PtkSamp& smp = PtkSamp{}) {
  const PtkPlan& P = x->ptk.plan;
  if (x->pos_host + n > x->m->cfg.max_ctx)
    return set_error(DZ_ERR_TENSOR, "context full: pos %d + %d > max_ctx %d", x->pos_host, n, x->m->cfg.max_ctx);
  if (per_pos && n > x->ptk.chunk) return set_error(DZ_ERR_TENSOR, "per-position logits: %d tokens per launch", n);
  // tags stay below 2^31: restart them (and clear every LL word) before they would pass it
  if ((x->ptk.gti + (uint64_t)n + 2) * (uint64_t)P.ppt + 1 >= (1ull << 31)) {
    const size_t ll_words = (size_t)2 * (P.n_layers + 1) * (size_t)P.off.words;
    DZ_HIP_CHECK(hipMemsetAsync(P.ll, 0, ll_words * sizeof(u64), x->s));
    x->ptk.gti = 0;
  }
  PtkRun r;
  r.plan = x->ptk.plan;
  r.plan.logits_all = per_pos ? x->ptk.logits_all : nullptr;
  r.feed = x->feed + feed_off;
  r.n_feed = n_feed;
  r.n_tok = n;
  r.pos0 = x->pos_host;
  r.tag0 = (unsigned)(1 + x->ptk.gti * (uint64_t)P.ppt);
  r.want_logits = 1;
  r.eos = eos;
  r.samp = smp;
  r.err.flag = x->ptk.err;
  r.err.spin_limit = ptk_spin_limit();
  // DAIZA_PTK_TRACE=<file>: append per-phase times of every workgroup to <file> (binary: int32
  // n_tok, ppt, G, slots, then n_tok*ppt*G*slots uint64 s_memrealtime ticks of 10 ns)
  const char* trace_path = getenv("DAIZA_PTK_TRACE");
  u64* trace = nullptr;
  r.trace = nullptr;
  const size_t trace_n = (size_t)n * P.ppt * P.G * kPtkTraceSlots;
  if (trace_path && trace_path[0]) {
    DZ_HIP_CHECK(hipMalloc(&trace, trace_n * sizeof(u64)));
    DZ_HIP_CHECK(hipMemset(trace, 0, trace_n * sizeof(u64)));
    r.trace = trace;
  }
  if (int rc = ptk_launch(x, r)) return rc;
  int err[4];
  DZ_HIP_CHECK(hipMemcpyAsync(err, x->ptk.err, 16, hipMemcpyDeviceToHost, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  x->ptk.gti += (uint64_t)n;
  if (trace) {
    std::vector<u64> h(trace_n);
    DZ_HIP_CHECK(hipMemcpy(h.data(), trace, trace_n * sizeof(u64), hipMemcpyDeviceToHost));
    DZ_HIP_CHECK(hipFree(trace));
    FILE* f = fopen(trace_path, "ab");
    if (f) {
      const int32_t hdr[4] = {n, P.ppt, P.G, kPtkTraceSlots};
      fwrite(hdr, sizeof hdr, 1, f);
      fwrite(h.data(), sizeof(u64), h.size(), f);
      fclose(f);
    }
  }
  if (err[0]) {
    DZ_HIP_CHECK(hipMemset(x->ptk.err, 0, 16));
    x->poisoned = true;
    return set_error(DZ_ERR_DEVICE, "token kernel: wait timed out (code %d, phase tag %u, workgroup %d)", err[0],
                     (unsigned)err[1], err[2]);
  }
  if (err[3] < 0 || err[3] > n) {
    x->poisoned = true;
    return set_error(DZ_ERR_DEVICE, "token kernel: %d of %d tokens reported", err[3], n);
  }
  n = err[3];
  if (n_done) *n_done = n;
  x->pos_host += n;
  // keep TokState consistent for the graph-path kernels (mixer steps)
  int pp[2] = {x->pos_host - 1, x->pos_host};
  DZ_HIP_CHECK(hipMemcpy(reinterpret_cast<char*>(x->st) + offsetof(TokState, pos), &pp[0], 4, hipMemcpyHostToDevice));
  DZ_HIP_CHECK(hipMemcpy(reinterpret_cast<char*>(x->st) + offsetof(TokState, pos_next), &pp[1], 4, hipMemcpyHostToDevice));
  return DZ_OK;
}

// Copies ids into the device feed array (synchronously: `ids` may be reused after the call).
static int ptk_feed(dz_ctx* x, const uint32_t* ids, int n) {
  if (n > x->feed_cap) return set_error(DZ_ERR_TENSOR, "feed of %d ids exceeds capacity %d", n, x->feed_cap);
  for (int i = 0; i < n; ++i)
    if (ids[i] >= (uint32_t)x->m->cfg.vocab) return set_error(DZ_ERR_TENSOR, "token id %u >= vocab %d", ids[i], x->m->cfg.vocab);
  DZ_HIP_CHECK(hipMemcpyAsync(x->feed, ids, (size_t)n * 4, hipMemcpyHostToDevice, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return DZ_OK;
}

// ---- sampled decode on the token kernel (dz_decode_sample, spec.hip): forward i takes feed[i]
// and leaves its logits in x->logits; the caller's kernels after each launch write feed[i + 1].
// The launches are enqueued without a host wait; ctx_sample_end synchronises and checks them.

int ctx_sample_begin(dz_ctx* x, uint32_t first, int n, uint32_t** feed, const float** logits, hipStream_t* s,
                     Scratch** scratch) {
  if (!x) return set_error(DZ_ERR_MODEL, "null context");
  if (int rc0 = ctx_usable(x)) return rc0;
  if (!x->ptk.on) return DZ_ERR_UNSUPPORTED;  // the caller samples on the host instead
  if (n < 1 || x->pos_host + n > x->m->cfg.max_ctx || n + 1 > x->feed_cap)
    return set_error(DZ_ERR_TENSOR, "sampled decode: %d tokens from position %d (max_ctx %d)", n, x->pos_host,
                     x->m->cfg.max_ctx);
  x->bt.pending = 0;
  if (int rc = ptk_feed(x, &first, 1)) return rc;
  const PtkPlan& P = x->ptk.plan;
  if ((x->ptk.gti + (uint64_t)n + 2) * (uint64_t)P.ppt + 1 >= (1ull << 31)) {
    const size_t ll_words = (size_t)2 * (P.n_layers + 1) * (size_t)P.off.words;
    DZ_HIP_CHECK(hipMemsetAsync(P.ll, 0, ll_words * sizeof(u64), x->s));
    x->ptk.gti = 0;
  }
  *feed = reinterpret_cast<uint32_t*>(x->feed);
  *logits = x->logits;
  *s = x->s;
  *scratch = &x->bt.spec;
  return DZ_OK;
}

int ctx_sample_launch(dz_ctx* x, int i) {
  const PtkPlan& P = x->ptk.plan;
  PtkRun r;
  r.plan = P;
  r.plan.logits_all = nullptr;
  r.feed = x->feed + i;
  r.n_feed = 1;
  r.n_tok = 1;
  r.pos0 = x->pos_host + i;
  r.tag0 = (unsigned)(1 + x->ptk.gti * (uint64_t)P.ppt);
  r.want_logits = 1;
  r.eos = -1;
  r.samp = PtkSamp{};
  r.err.flag = x->ptk.err;
  r.err.spin_limit = ptk_spin_limit();
  r.trace = nullptr;
  if (int rc = ptk_launch(x, r)) return rc;
  x->ptk.gti += 1;
  return DZ_OK;
}

int ctx_sample_decode(dz_ctx* x, uint32_t first, int n, int k, float inv_t, float top_p, uint64_t* rng,
                      uint32_t* out) {
  if (!x) return set_error(DZ_ERR_MODEL, "null context");
  if (int rc0 = ctx_usable(x)) return rc0;
  if (!x->ptk.on || !x->ptk.kfn_s || x->ptk.plan.G > kPtkFan * kPtkFan || k < 1 || k > kPtkSampMax)
    return DZ_ERR_UNSUPPORTED;
  x->bt.pending = 0;
  const int p0 = x->pos_host;
  int rc = ptk_feed(x, &first, 1);
  if (rc) return rc;
  DZ_HIP_CHECK(hipMemcpyAsync(x->ptk.rng, rng, 8, hipMemcpyHostToDevice, x->s));
  PtkSamp smp;
  smp.k = k;
  smp.inv_t = inv_t;
  smp.top_p = top_p;
  smp.rng = x->ptk.rng;
  if ((rc = ptk_run(x, n, 1, false, 0, -1, nullptr, smp))) return rc;
  DZ_HIP_CHECK(hipMemcpy(out, x->toklog + p0 + 1, (size_t)n * 4, hipMemcpyDeviceToHost));
  DZ_HIP_CHECK(hipMemcpy(rng, x->ptk.rng, 8, hipMemcpyDeviceToHost));
  return DZ_OK;
}

int ctx_sample_end(dz_ctx* x, int n) {
  int err[4];
  DZ_HIP_CHECK(hipMemcpyAsync(err, x->ptk.err, 16, hipMemcpyDeviceToHost, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  if (err[0] || err[3] != 1) {
    DZ_HIP_CHECK(hipMemset(x->ptk.err, 0, 16));
    x->poisoned = true;
    return set_error(DZ_ERR_DEVICE, "token kernel: wait timed out (code %d, phase tag %u, workgroup %d)", err[0],
                     (unsigned)err[1], err[2]);
  }
  x->pos_host += n;
  int pp[2] = {x->pos_host - 1, x->pos_host};
  DZ_HIP_CHECK(hipMemcpy(reinterpret_cast<char*>(x->st) + offsetof(TokState, pos), &pp[0], 4, hipMemcpyHostToDevice));
  DZ_HIP_CHECK(hipMemcpy(reinterpret_cast<char*>(x->st) + offsetof(TokState, pos_next), &pp[1], 4, hipMemcpyHostToDevice));
  return DZ_OK;
}

// ---------------------------------------------------------------- n-token forward (host)

static void bt_release(dz_ctx* x) {
  for (void* p : x->bt.allocs) (void)hipFree(p);
  x->bt.allocs.clear();
  x->bt.cap = 0;
  x->bt.kv_cap = 0;
  x->bt.logits_rows = 0;
  x->bt.rx.clear();
  x->bt.rec.clear();
  if (x->bt.pack.ptr) (void)hipFree(x->bt.pack.ptr);
  if (x->bt.split.ptr) (void)hipFree(x->bt.split.ptr);
  if (x->bt.arec.ptr) (void)hipFree(x->bt.arec.ptr);
  if (x->bt.spec.ptr) (void)hipFree(x->bt.spec.ptr);
  x->bt.pack = Scratch{};
  x->bt.split = Scratch{};
  x->bt.arec = Scratch{};
  x->bt.spec = Scratch{};
}

// Activation buffers for chunks of up to cap tokens.
static int bt_reserve(dz_ctx* x, int cap) {
  if (cap <= x->bt.cap) return DZ_OK;
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  const dz_model* m = x->m;
  const dz_config& c = m->cfg;
  for (void* p : x->bt.allocs) (void)hipFree(p);
  x->bt.allocs.clear();
  x->bt.cap = 0;
  x->bt.kv_cap = 0;
  x->bt.logits_rows = 0;
  x->bt.rx.clear();
  x->bt.rec.clear();
  const int64_t hd = c.ssm_state, kdim = (int64_t)c.ssm_k_heads * hd, inner = (int64_t)c.ssm_v_heads * hd;
  const int64_t qkvd = 2 * kdim + inner, qd = (int64_t)c.n_head * c.head_dim;
  int64_t rows_in = 1;
  for (const LayerDev& l : m->L) rows_in = std::max(rows_in, l.in_proj.rows);
  const size_t n = (size_t)cap;
  auto& A = x->bt.allocs;
  int rc;
  if ((rc = alloc_t(A, &x->bt.ids, n)) || (rc = alloc_t(A, &x->bt.h, n * c.hidden)) ||
      (rc = alloc_t(A, &x->bt.yin, n * rows_in)) || (rc = alloc_t(A, &x->bt.cout, n * qkvd)) ||
      (rc = alloc_t(A, &x->bt.qk, n * 2 * kdim)) || (rc = alloc_t(A, &x->bt.ys, n * inner)) ||
      (rc = alloc_t(A, &x->bt.gy, n * std::max(inner, qd))) || (rc = alloc_t(A, &x->bt.ygu, n * 2 * c.ffn)) ||
      (rc = alloc_t(A, &x->bt.sw, n * c.ffn)) || (rc = alloc_t(A, &x->bt.qb, n * qd)) ||
      (rc = alloc_t(A, &x->bt.gate, n * qd)))
    return rc;
  x->bt.cap = cap;
  return DZ_OK;
}

static int bt_reserve_logits(dz_ctx* x, int rows) {
  if (rows <= x->bt.logits_rows) return DZ_OK;
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  int rc = alloc_t(x->bt.allocs, &x->bt.logits, (size_t)rows * x->m->cfg.vocab);
  if (rc) return rc;
  x->bt.logits_rows = rows;
  return DZ_OK;
}

// Rollback records of a verify chunk of up to k tokens, per DeltaNet layer.
static int bt_reserve_verify(dz_ctx* x, int k) {
  if (k <= x->bt.kv_cap) return DZ_OK;
  const dz_config& c = x->m->cfg;
  const int64_t hd = c.ssm_state, kdim = (int64_t)c.ssm_k_heads * hd, inner = (int64_t)c.ssm_v_heads * hd;
  const int64_t qkvd = 2 * kdim + inner;
  x->bt.rx.assign((size_t)x->m->n_ssm, nullptr);
  x->bt.rec.assign((size_t)x->m->n_ssm, DnRecord{nullptr, nullptr, nullptr});
  auto& A = x->bt.allocs;
  int rc;
  for (int i = 0; i < x->m->n_ssm; ++i) {
    DnRecord& r = x->bt.rec[(size_t)i];
    if ((rc = alloc_t(A, &x->bt.rx[(size_t)i], (size_t)k * qkvd)) || (rc = alloc_t(A, &r.decay, (size_t)k * c.ssm_v_heads)) ||
        (rc = alloc_t(A, &r.d, (size_t)k * inner)) || (rc = alloc_t(A, &r.k, (size_t)k * kdim)))
      return rc;
  }
  x->bt.kv_cap = k;
  return DZ_OK;
}

template <class K, class... Args>
static hipError_t launch(K kfn, dim3 g, dim3 b, hipStream_t s, Args... args) {
  hipLaunchKernelGGL(kfn, g, b, 0, s, args...);
  return hipGetLastError();
}

// Grid (token groups, nkv, nch); with at least 8 (kv-head, chunk) pairs, a 1-D grid that keeps each
// pair's token groups on one XCD (bt_attn_kernel).  A few tokens (speculative verify) go two to a
// workgroup, so that each cache row is read half as often; a long prefill keeps one token per
// workgroup (more workgroups, fewer registers each).
static hipError_t launch_bt_attn(int grp, int n, int nkv, int nch, hipStream_t s, const float* qb, const float* gate,
                                 const float* kc, const float* vc, int max_ctx, int nq, int pos0, float* ao, int csz,
                                 float* rec) {
  const int tpw = n <= 16 ? 2 : 1;
  const int ng = (n + tpw - 1) / tpw;
  const int pairs = nkv * nch;
  const bool xcd = nch > 1 && pairs >= 8;
  const dim3 g = xcd ? dim3((unsigned)(8 * ((pairs + 7) / 8) * ng)) : dim3((unsigned)ng, (unsigned)nkv, (unsigned)nch);
  const int nx = xcd ? ng : 0;
#define DZ_ATTN(G_, T_) \
  launch(bt_attn_kernel<G_, T_>, g, dim3(256), s, qb, gate, kc, vc, max_ctx, nq, pos0, n, ao, csz, rec, nx, nkv, nch)
#define DZ_ATTN_G(G_) return tpw == 2 ? DZ_ATTN(G_, 2) : DZ_ATTN(G_, 1)
  switch (grp) {
    case 1: DZ_ATTN_G(1);
    case 2: DZ_ATTN_G(2);
    case 3: DZ_ATTN_G(3);
    case 4: DZ_ATTN_G(4);
    case 6: DZ_ATTN_G(6);
    case 8: DZ_ATTN_G(8);
    default: return hipErrorInvalidValue;
  }
#undef DZ_ATTN_G
#undef DZ_ATTN
}

// The few-token attention on the matrix cores (every token of a kv-head in one workgroup), grid
// (nch, nkv), with about one workgroup per CU (one wave per SIMD: the kernel holds its block's
// keys and values a block ahead in registers).
static hipError_t launch_bt_attn_mfma(int grp, int nkv, int nch, hipStream_t s, const float* qb, const float* kc,
                                      const float* vc, int max_ctx, int nq, int pos0, int n, int csz, float* rec) {
  const dim3 g((unsigned)nch, (unsigned)nkv);
#define DZ_ATTN_M(G_) return launch(bt_attn_mfma_kernel<G_>, g, dim3(256), s, qb, kc, vc, max_ctx, nq, pos0, n, csz, nch, rec)
  switch (grp) {
    case 1: DZ_ATTN_M(1);
    case 2: DZ_ATTN_M(2);
    case 3: DZ_ATTN_M(3);
    case 4: DZ_ATTN_M(4);
    case 6: DZ_ATTN_M(6);
    case 8: DZ_ATTN_M(8);
    default: return hipErrorInvalidValue;
  }
#undef DZ_ATTN_M
}

static int bt_attn_mfma_chunks(int nkv, int ctx_max, int* csz) {
  int nch = std::max(1, std::min(256, (256 + nkv - 1) / nkv));
  *csz = ((ctx_max + nch - 1) / nch + 15) / 16 * 16;  // whole blocks of 16 positions
  return (ctx_max + *csz - 1) / *csz;
}

// Position chunks of the chunk's attention: enough workgroups to fill the device when the chunk
// has few tokens (speculative verify at long context), one chunk for a long prefill.
// A chunk of several positions is a whole number of 256-position rounds (the kernel's 4 waves take
// 64 each) where that keeps about the wanted number of chunks.
static int bt_attn_chunks(int n, int nkv, int ctx_max, int* csz) {
  int nch = (1024 + n * nkv - 1) / (n * nkv);
  nch = std::max(1, std::min({nch, std::max(1, ctx_max / 64), 256}));  // the merge takes up to 256
  *csz = (ctx_max + nch - 1) / nch;
  if (nch > 1 && *csz > 256) *csz = (*csz + 128) / 256 * 256;
  return (ctx_max + *csz - 1) / *csz;
}

// y[n][W.rows] (=|+=) W · (optionally RMS-normalised) x[n][W.cols].
static int bt_gemm(dz_ctx* x, const Q1Dev& W, const float* xin, int64_t ldx, int n, const float* norm_w, float* y,
                   int64_t ldy, int accumulate, GemmDefer* defer = nullptr) {
  if (n <= 16) {
    // few tokens (verify): the product packs its tiles itself (folding in the RMSNorm, whose 1/rms is
    // applied to the sums), which saves the packing launch; with many tokens every row-block group
    // would repeat the packing of the same tiles
    DZ_HIP_CHECK(launch_q1_gemm_raw(W, xin, ldx, n, y, ldy, accumulate, x->s, &x->bt.split, norm_w,
                                    x->m->cfg.rms_eps, defer));
    return DZ_OK;
  }
  PackedX p;
  int rc = packed_x_reserve(x->bt.pack, n, W.cols, &p);
  if (rc) return rc;
  DZ_HIP_CHECK(launch_x_pack(xin, ldx, W.cols, n, norm_w, x->m->cfg.rms_eps, p, x->s));
  DZ_HIP_CHECK(launch_q1_gemm(W, p, n, y, ldy, accumulate, x->s, &x->bt.split, defer));
  return DZ_OK;
}

// The forward of tokens ids[0..n) (host) at positions pos_host .. pos_host+n-1 (forward_batch,
// forward.rs:394-1407, with the per-token block order of forward.rs:204-375).  Writes the logits
// of the last out_rows tokens to bt.logits.  With verify set, the DeltaNet states and conv rings
// are left as they were and the rollback records are filled instead; the KV cache gets the chunk's
// entries either way.  Does not move the position.
static int bt_forward(dz_ctx* x, const uint32_t* ids, int n, int out_rows, bool verify) {
  dz_model* m = x->m;
  const dz_config& c = m->cfg;
  hipStream_t s = x->s;
  int rc;
  if ((rc = bt_reserve(x, n)) || (rc = bt_reserve_logits(x, out_rows))) return rc;
  if (verify && (rc = bt_reserve_verify(x, n))) return rc;
  for (int i = 0; i < n; ++i)
    if (ids[i] >= (uint32_t)c.vocab) return set_error(DZ_ERR_TENSOR, "token id %u >= vocab %d", ids[i], c.vocab);
  DZ_HIP_CHECK(hipMemcpyAsync(x->bt.ids, ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
  const int p0 = x->pos_host;
  const int64_t H = c.hidden, hd = c.ssm_state, F = c.ffn;
  const int64_t kdim = (int64_t)c.ssm_k_heads * hd, inner = (int64_t)c.ssm_v_heads * hd, qkvd = 2 * kdim + inner;
  const int64_t qd = (int64_t)c.n_head * c.head_dim;
  const size_t kvsz = (size_t)c.n_head_kv * c.max_ctx * c.head_dim;
  const unsigned nb = (unsigned)n;
  DZ_HIP_CHECK(launch(bt_embed_kernel, dim3(nb), dim3(256), s, (const int*)x->bt.ids, H, (const uint16_t*)m->emb_f16,
                      (const uint8_t*)m->emb_q1.data, (int)m->emb_q1.ntiles, x->bt.h));
  for (size_t li = 0; li < m->L.size(); ++li) {
    const LayerDev& l = m->L[li];
    const int64_t ld_in = l.in_proj.rows;
    if ((rc = bt_gemm(x, l.in_proj, x->bt.h, H, n, l.attn_norm, x->bt.yin, ld_in, 0))) return rc;
    if (!l.attn) {
      const int si = l.kind_idx;
      float* ring = x->conv + (size_t)si * 4 * qkvd;
      const int head0 = (x->ring_base[(size_t)si] + p0) & 3;
      const unsigned gch = (unsigned)((qkvd + 255) / 256);
      // verify keeps the chunk's conv inputs (bt.rx) for the commit; a kept forward updates the ring now
      // (conv, SiLU and the q/k L2 norms in one launch)
      DZ_HIP_CHECK(launch(bt_conv_kernel, dim3(gch, nb), dim3(256), s, (const float*)x->bt.yin, ld_in, n,
                          (const float*)ring, head0, (const float*)l.conv_w, qkvd, x->bt.cout,
                          verify ? x->bt.rx[(size_t)si] : nullptr, (int)c.ssm_k_heads, x->bt.qk));
      DnRecord rec{nullptr, nullptr, nullptr};
      if (verify) {
        rec = x->bt.rec[(size_t)si];
      } else {
        DZ_HIP_CHECK(launch(bt_ring_kernel, dim3(gch), dim3(256), s, (const float*)x->bt.yin, ld_in, std::max(0, n - 4),
                            n, ring, head0, qkvd));
      }
      float* state = x->ssm_state + (size_t)si * c.ssm_v_heads * hd * hd;
      DZ_HIP_CHECK(launch(bt_scan_kernel, dim3((unsigned)(4 * c.ssm_v_heads)), dim3(256), s, (const float*)x->bt.yin,
                          ld_in, (const float*)x->bt.cout, qkvd, (const float*)x->bt.qk, n, (int)c.ssm_k_heads,
                          (int)c.ssm_v_heads, qkvd + inner, qkvd + inner + c.ssm_v_heads, (const float*)l.ssm_a,
                          (const float*)l.dt_bias, state, x->bt.ys, rec));
      DZ_HIP_CHECK(launch(bt_gate_y_kernel, dim3(nb, (unsigned)c.ssm_v_heads), dim3(128), s, (const float*)x->bt.ys,
                          (const float*)x->bt.yin, ld_in, qkvd, (const float*)l.ssm_norm, c.rms_eps,
                          (int)c.ssm_v_heads, x->bt.gy));
      if ((rc = bt_gemm(x, l.out_proj, x->bt.gy, inner, n, nullptr, x->bt.h, H, 1))) return rc;
    } else {
      float* kc = x->kv + (size_t)l.kind_idx * 2 * kvsz;
      float* vc = kc + kvsz;
      DZ_HIP_CHECK(launch(bt_attn_prep_kernel, dim3(nb, (unsigned)(c.n_head + c.n_head_kv)), dim3(256), s,
                          (const float*)x->bt.yin, ld_in, (int)c.n_head, (int)c.n_head_kv, (const float*)l.q_norm,
                          (const float*)l.k_norm, c.rms_eps, (const float*)x->rope, (int)c.rope_dim, p0, x->bt.qb,
                          x->bt.gate, kc, vc, (int)c.max_ctx));
      // few tokens (verify): all of a kv-head's query rows in one matrix-core workgroup, chunk records
      // always merged; otherwise token groups per workgroup
      const int grp = (int)(c.n_head / c.n_head_kv);
      const bool mf = n * grp <= 64;
      int csz;
      const int nch = mf ? bt_attn_mfma_chunks((int)c.n_head_kv, p0 + n, &csz)
                         : bt_attn_chunks(n, (int)c.n_head_kv, p0 + n, &csz);
      float* rec = nullptr;
      if (nch > 1 || mf) {
        if ((rc = x->bt.arec.reserve((size_t)n * c.n_head * nch * (2 + c.head_dim) * sizeof(float)))) return rc;
        rec = static_cast<float*>(x->bt.arec.ptr);
      }
      if (mf)
        DZ_HIP_CHECK(launch_bt_attn_mfma(grp, (int)c.n_head_kv, nch, s, x->bt.qb, kc, vc, (int)c.max_ctx, (int)c.n_head,
                                         p0, n, csz, rec));
      else
        DZ_HIP_CHECK(launch_bt_attn(grp, n, (int)c.n_head_kv, nch, s, x->bt.qb, x->bt.gate, kc, vc, (int)c.max_ctx,
                                    (int)c.n_head, p0, x->bt.gy, csz, rec));
      if (nch > 1 || mf)
        DZ_HIP_CHECK(launch(bt_attn_merge_kernel, dim3(nb, (unsigned)c.n_head), dim3(256), s, (const float*)rec, nch,
                            (const float*)x->bt.gate, (int)c.n_head, x->bt.gy));
      if ((rc = bt_gemm(x, l.out_proj, x->bt.gy, qd, n, nullptr, x->bt.h, H, 1))) return rc;
    }
    // MLP (mlp.rs:28-47): h += W_down (silu(W_gate n) * W_up n), n = rmsnorm(h, post_attention_norm)
    // a split gate/up product (few tokens) goes from its partials straight to the SwiGLU
    GemmDefer gd;
    if ((rc = bt_gemm(x, l.gate_up, x->bt.h, H, n, l.post_norm, x->bt.ygu, 2 * F, 0, &gd))) return rc;
    if (gd.splits > 1)
      DZ_HIP_CHECK(launch(bt_split_swiglu_kernel, dim3((unsigned)((F + 255) / 256), nb), dim3(256), s, gd.part,
                          gd.splits, gd.zstride, F, n, x->bt.sw, gd.ssq, gd.ssq_ld, gd.K, gd.eps));
    else
      DZ_HIP_CHECK(launch(bt_swiglu_kernel, dim3((unsigned)((F + 255) / 256), nb), dim3(256), s,
                          (const float*)x->bt.ygu, F, n, x->bt.sw));
    if ((rc = bt_gemm(x, l.down, x->bt.sw, F, n, nullptr, x->bt.h, H, 1))) return rc;
  }
  // output norm + lm_head for the last out_rows tokens
  const float* hl = x->bt.h + (size_t)(n - out_rows) * H;
  if ((rc = bt_gemm(x, m->lm_head, hl, H, out_rows, m->output_norm, x->bt.logits, c.vocab, 0))) return rc;
  return DZ_OK;
}

// After a forward of n tokens ids at p0 that is kept: the token log, TokState and the context's
// logits (the last token's row of bt.logits, row `last_row`) as forward_single_token leaves them.
static int bt_finish(dz_ctx* x, const uint32_t* ids, int n, int p0, int last_row) {
  const dz_config& c = x->m->cfg;
  DZ_HIP_CHECK(hipMemcpyAsync(x->toklog + p0, ids, (size_t)n * 4, hipMemcpyHostToDevice, x->s));
  TokState st;
  memset(&st, 0, sizeof st);
  st.pos = p0 + n - 1;
  st.token = (int)ids[n - 1];
  st.pos_next = p0 + n;
  DZ_HIP_CHECK(hipMemcpyAsync(x->st, &st, sizeof st, hipMemcpyHostToDevice, x->s));
  DZ_HIP_CHECK(hipMemcpyAsync(x->logits, x->bt.logits + (size_t)last_row * c.vocab, (size_t)c.vocab * 4,
                              hipMemcpyDeviceToDevice, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));  // the host copies above read caller memory
  x->pos_host = p0 + n;
  return DZ_OK;
}

// Speculative verify, first half: the forward of draft[0..k) at positions pos .. pos+k-1 with
// every position's logits (bt.logits rows), the DeltaNet states and conv rings untouched and their
// rollback records kept.  The position does not move until bt_verify_commit.
static int bt_verify_forward(dz_ctx* x, const uint32_t* draft, int k) {
  if (x->pos_host + k > x->m->cfg.max_ctx) return set_error(DZ_ERR_TENSOR, "verify: context full");
  x->bt.pending = 0;
  int rc = bt_forward(x, draft, k, k, true);
  if (rc) return rc;
  x->bt.pending_ids.assign(draft, draft + k);
  x->bt.pending = k;
  return DZ_OK;
}

// Second half: keeps the first a drafts (0 <= a <= k) as if they alone had been forwarded: each
// DeltaNet layer replays a recorded updates onto its state and takes their conv inputs into its
// ring; the KV entries beyond pos + a are dropped by the position; the context's logits become
// those after draft a-1 (unchanged for a = 0).
static int bt_verify_commit(dz_ctx* x, int a) {
  const int k = x->bt.pending;
  if (a < 0 || a > k) return set_error(DZ_ERR_TENSOR, "verify commit: %d of %d drafts", a, k);
  x->bt.pending = 0;
  if (a == 0) return DZ_OK;
  const dz_model* m = x->m;
  const dz_config& c = m->cfg;
  const int64_t hd = c.ssm_state, kdim = (int64_t)c.ssm_k_heads * hd, inner = (int64_t)c.ssm_v_heads * hd;
  const int64_t qkvd = 2 * kdim + inner;
  const int p0 = x->pos_host;
  for (const LayerDev& l : m->L) {
    if (l.attn) continue;
    const int si = l.kind_idx;
    DZ_HIP_CHECK(launch(bt_commit_state_kernel, dim3((unsigned)(4 * c.ssm_v_heads)), dim3(256), x->s,
                        x->ssm_state + (size_t)si * c.ssm_v_heads * hd * hd, x->bt.rec[(size_t)si], a,
                        (int)c.ssm_k_heads, (int)c.ssm_v_heads));
    DZ_HIP_CHECK(launch(bt_ring_kernel, dim3((unsigned)((qkvd + 255) / 256)), dim3(256), x->s,
                        (const float*)x->bt.rx[(size_t)si], qkvd, std::max(0, a - 4), a,
                        x->conv + (size_t)si * 4 * qkvd, (x->ring_base[(size_t)si] + p0) & 3, qkvd));
  }
  return bt_finish(x, x->bt.pending_ids.data(), a, p0, a - 1);
}

// Device logits of a pending verify for the sampler (spec.hip): row 0 = the context's logits (they
// predict draft 0), rows = the verify forward's per-position rows; its stream and scratch memory.
// Largest chunk of one n-token forward (activations ~0.3 MB per token at the 27B shape).
constexpr int kBatchChunk = 1024;

int ctx_verify_enqueue(dz_ctx* x, const uint32_t* draft, int k) {
  if (!x || !draft) return set_error(DZ_ERR_MODEL, "null argument");
  if (k < 1) return set_error(DZ_ERR_TENSOR, "verify: %d drafts", k);
  if (k > kBatchChunk) return set_error(DZ_ERR_TENSOR, "verify: %d drafts (at most %d)", k, kBatchChunk);
  if (int rc0 = ctx_usable(x)) return rc0;
  return bt_verify_forward(x, draft, k);
}

int ctx_verify_view(dz_ctx* x, const float** row0, const float** rows, hipStream_t* s, Scratch** scratch) {
  if (x->bt.pending == 0) return set_error(DZ_ERR_TENSOR, "no pending verify forward");
  *row0 = x->logits;
  *rows = x->bt.logits;
  *s = x->s;
  *scratch = &x->bt.spec;
  return DZ_OK;
}

// DAIZA_BATCH=0 runs forward_batch token by token through the decode path instead.
static bool batch_wanted() {
  const char* e = getenv("DAIZA_BATCH");
  return !(e && e[0] == '0');
}


static int bt_prefill(dz_ctx* x, const uint32_t* ids, int n, float* last_logits, float* per_pos) {
  const size_t V = (size_t)x->m->cfg.vocab;
  const int chunk = per_pos ? 128 : kBatchChunk;
  x->bt.pending = 0;
  for (int i0 = 0; i0 < n; i0 += chunk) {
    const int k = std::min(chunk, n - i0);
    const int rows = per_pos ? k : 1;
    int rc = bt_forward(x, ids + i0, k, rows, false);
    if (rc || (rc = bt_finish(x, ids + i0, k, x->pos_host, rows - 1))) return rc;
    if (per_pos)
      DZ_HIP_CHECK(hipMemcpyAsync(per_pos + (size_t)i0 * V, x->bt.logits, (size_t)k * V * 4, hipMemcpyDeviceToHost, x->s));
  }
  if (last_logits) DZ_HIP_CHECK(hipMemcpyAsync(last_logits, x->logits, V * 4, hipMemcpyDeviceToHost, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return DZ_OK;
}

}  // namespace dz

extern "C" {

int dz_ctx_create(dz_model* m, dz_ctx** out) {
  if (!m || !out) return set_error(DZ_ERR_MODEL, "null argument");
  int rc = ensure_device();
  if (rc) return rc;
  if ((rc = prepare_gemv_kernels())) return rc;
  dz_ctx* x = new dz_ctx();
  x->m = m;
  const dz_config& c = m->cfg;
  auto fail = [&](int code) { ctx_release(x); return code; };
  hipError_t e = hipStreamCreateWithFlags(&x->s, hipStreamNonBlocking);
  if (e != hipSuccess) return fail(set_error(DZ_ERR_DEVICE, "stream: %s", hipGetErrorString(e)));
  int64_t ld_in, ld_h, ld_gu;
  int th, to, tf;
  ctx_dims(m, &ld_in, &ld_h, &ld_gu, &th, &to, &tf);
  const int64_t hd = c.ssm_state, inner = (int64_t)c.ssm_v_heads * hd;
  const int64_t qkvd = 2 * (int64_t)c.ssm_k_heads * hd + inner;
  const size_t kvsz = (size_t)c.n_head_kv * c.max_ctx * c.head_dim;
  auto& A = x->allocs;
  x->feed_cap = c.max_ctx + 1;  // a sampled run writes the draw after its last token too
  x->n_am = (int)m->lm_head.nrb;
  if ((rc = alloc_t(A, &x->st, 1)) || (rc = alloc_t(A, &x->feed, (size_t)x->feed_cap)) ||
      (rc = alloc_t(A, &x->toklog, (size_t)c.max_ctx + 1)) || (rc = alloc_t(A, &x->emb_row, (size_t)c.hidden)) ||
      (rc = alloc_t(A, &x->h[0], (size_t)ld_h)) || (rc = alloc_t(A, &x->h[1], (size_t)ld_h)) ||
      (rc = alloc_t(A, &x->ss[0], (size_t)th)) || (rc = alloc_t(A, &x->ss[1], (size_t)th)) ||
      (rc = alloc_t(A, &x->p_in, (size_t)th * ld_in)) || (rc = alloc_t(A, &x->p_o, (size_t)to * ld_h)) ||
      (rc = alloc_t(A, &x->p_gu, (size_t)th * ld_gu)) || (rc = alloc_t(A, &x->p_down, (size_t)tf * ld_h)) ||
      (rc = alloc_t(A, &x->y, (size_t)inner)) || (rc = alloc_t(A, &x->zs, (size_t)inner)) ||
      (rc = alloc_t(A, &x->apart, (size_t)c.n_head * x->gmax * (2 + c.head_dim))) ||
      (rc = alloc_t(A, &x->attn_u, (size_t)c.n_head * c.head_dim)) ||
      (rc = alloc_t(A, &x->h_fin, (size_t)ld_h)) || (rc = alloc_t(A, &x->ss_fin, (size_t)th)) ||
      (rc = alloc_t(A, &x->logits, (size_t)m->lm_head.nrb * kRowBlock)) ||
      (rc = alloc_t(A, &x->am_val, (size_t)x->n_am)) || (rc = alloc_t(A, &x->am_idx, (size_t)x->n_am)) ||
      (rc = alloc_t(A, &x->ssm_state, (size_t)std::max(1, m->n_ssm) * c.ssm_v_heads * hd * hd)) ||
      (rc = alloc_t(A, &x->conv, (size_t)std::max(1, m->n_ssm) * 4 * qkvd)) ||
      (rc = alloc_t(A, &x->ring_base_dev, (size_t)std::max(1, m->n_ssm))) ||
      (rc = alloc_t(A, &x->kv, (size_t)std::max(1, m->n_attn) * 2 * kvsz)))
    return fail(rc);
  x->ring_base.assign((size_t)m->n_ssm, 0);
  std::vector<float> rope;
  rope_table(c, rope);
  if ((rc = upload_f32(A, &x->rope, rope.data(), rope.size()))) return fail(rc);
  // argmax partials of "no logits yet": value -inf everywhere, selects token 0 if ever read
  if ((rc = ctx_zero_state(x))) return fail(rc);
  if (ptk_wanted() && (rc = ptk_prepare(x))) return fail(rc);
  *out = x;
  return DZ_OK;
}

int dz_ctx_free(dz_ctx* x) {
  ctx_release(x);
  return DZ_OK;
}

int dz_ctx_reset(dz_ctx* x) {
  if (!x) return set_error(DZ_ERR_MODEL, "null context");
  x->bt.pending = 0;
  return ctx_zero_state(x);
}

int dz_ctx_pos(const dz_ctx* x) { return x ? x->pos_host : -1; }

}  // extern "C"

const dz_config* dz::ctx_config(const dz_ctx* x) { return &x->m->cfg; }

extern "C" {

void* dz_ctx_stream(dz_ctx* x) { return x ? (void*)x->s : nullptr; }

int dz_ctx_token_kernel(const dz_ctx* x) { return x && x->ptk.on ? 1 : 0; }

int dz_forward_token(dz_ctx* x, uint32_t token, float* logits, uint32_t* argmax) {
  if (!x) return set_error(DZ_ERR_MODEL, "null context");
  if (int rc0 = ctx_usable(x)) return rc0;
  x->bt.pending = 0;
  if (x->ptk.on) {
    int rc = ptk_feed(x, &token, 1);
    if (rc || (rc = ptk_run(x, 1, 1, false))) return rc;
    if (argmax) {
      int t;
      DZ_HIP_CHECK(hipMemcpy(&t, x->toklog + x->pos_host, 4, hipMemcpyDeviceToHost));
      *argmax = (uint32_t)t;
    }
    if (logits) DZ_HIP_CHECK(hipMemcpy(logits, x->logits, (size_t)x->m->cfg.vocab * 4, hipMemcpyDeviceToHost));
    return DZ_OK;
  }
  int rc = ctx_feed(x, &token, 1);
  if (rc) return rc;
  if ((rc = ctx_run(x, 1))) return rc;
  if (argmax) {
    if ((rc = ctx_peek_argmax(x))) return rc;
    int t;
    DZ_HIP_CHECK(hipMemcpyAsync(&t, x->toklog + x->pos_host, 4, hipMemcpyDeviceToHost, x->s));
    DZ_HIP_CHECK(hipStreamSynchronize(x->s));
    *argmax = (uint32_t)t;
  }
  if (logits) DZ_HIP_CHECK(hipMemcpyAsync(logits, x->logits, (size_t)x->m->cfg.vocab * 4, hipMemcpyDeviceToHost, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return DZ_OK;
}

int dz_forward_batch(dz_ctx* x, const uint32_t* ids, int n, int start_pos, float* last_logits, float* per_pos) {
  if (!x || (!ids && n)) return set_error(DZ_ERR_MODEL, "null argument");
  if (n < 1) return set_error(DZ_ERR_TENSOR, "forward_batch: empty batch");
  if (int rc0 = ctx_usable(x)) return rc0;
  if (start_pos != x->pos_host)
    return set_error(DZ_ERR_TENSOR, "forward_batch: start_pos %d != context position %d", start_pos, x->pos_host);
  if (x->pos_host + n > x->m->cfg.max_ctx) return set_error(DZ_ERR_TENSOR, "forward_batch: context full");
  x->bt.pending = 0;
  const size_t V = (size_t)x->m->cfg.vocab;
  if (batch_wanted()) return bt_prefill(x, ids, n, last_logits, per_pos);
  if (x->ptk.on) {
    int rc = ptk_feed(x, ids, n);
    if (rc) return rc;
    if (per_pos) {
      for (int i0 = 0; i0 < n; i0 += x->ptk.chunk) {
        const int k = std::min(x->ptk.chunk, n - i0);
        if ((rc = ptk_run(x, k, k, true, i0))) return rc;
        DZ_HIP_CHECK(hipMemcpy(per_pos + (size_t)i0 * V, x->ptk.logits_all, (size_t)k * V * 4, hipMemcpyDeviceToHost));
      }
    } else if ((rc = ptk_run(x, n, n, false))) {
      return rc;
    }
    if (last_logits) DZ_HIP_CHECK(hipMemcpy(last_logits, x->logits, V * 4, hipMemcpyDeviceToHost));
    return DZ_OK;
  }
  int rc = ctx_feed(x, ids, n);
  if (rc) return rc;
  for (int i = 0; i < n; ++i) {
    if ((rc = ctx_run(x, 1))) return rc;
    if (per_pos) DZ_HIP_CHECK(hipMemcpyAsync(per_pos + (size_t)i * V, x->logits, V * 4, hipMemcpyDeviceToHost, x->s));
  }
  if (last_logits) DZ_HIP_CHECK(hipMemcpyAsync(last_logits, x->logits, V * 4, hipMemcpyDeviceToHost, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return DZ_OK;
}

int dz_decode_greedy(dz_ctx* x, uint32_t first_token, int n, uint32_t* out_tokens) {
  if (!x || !out_tokens) return set_error(DZ_ERR_MODEL, "null argument");
  if (int rc0 = ctx_usable(x)) return rc0;
  if (n < 1) return DZ_OK;
  x->bt.pending = 0;
  const int p0 = x->pos_host;
  if (x->ptk.on) {
    int rc = ptk_feed(x, &first_token, 1);
    if (rc || (rc = ptk_run(x, n, 1, false))) return rc;
    DZ_HIP_CHECK(hipMemcpy(out_tokens, x->toklog + p0 + 1, (size_t)n * 4, hipMemcpyDeviceToHost));
    return DZ_OK;
  }
  int rc = ctx_feed(x, &first_token, 1);
  if (rc) return rc;
  if ((rc = ctx_run(x, n))) return rc;
  if ((rc = ctx_peek_argmax(x))) return rc;
  DZ_HIP_CHECK(hipMemcpyAsync(out_tokens, x->toklog + p0 + 1, (size_t)n * 4, hipMemcpyDeviceToHost, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return DZ_OK;
}

int dz_decode_greedy_eos(dz_ctx* x, uint32_t first_token, int n, int32_t eos_id, uint32_t* out_tokens,
                         int* n_forwarded) {
  if (!x || !out_tokens || !n_forwarded) return set_error(DZ_ERR_MODEL, "null argument");
  *n_forwarded = 0;
  if (int rc0 = ctx_usable(x)) return rc0;
  if (n < 1 || (eos_id >= 0 && first_token == (uint32_t)eos_id)) return DZ_OK;
  x->bt.pending = 0;
  const int p0 = x->pos_host;
  if (x->ptk.on) {
    int done = 0;
    int rc = ptk_feed(x, &first_token, 1);
    if (rc || (rc = ptk_run(x, n, 1, false, 0, eos_id < 0 ? -1 : eos_id, &done))) return rc;
    if (done) DZ_HIP_CHECK(hipMemcpy(out_tokens, x->toklog + p0 + 1, (size_t)done * 4, hipMemcpyDeviceToHost));
    *n_forwarded = done;
    return DZ_OK;
  }
  // graph path: one token per replay, the pick read back and checked on the host
  int rc = ctx_feed(x, &first_token, 1);
  if (rc) return rc;
  for (int i = 0; i < n; ++i) {
    if ((rc = ctx_run(x, 1)) || (rc = ctx_peek_argmax(x))) return rc;
    int t;
    DZ_HIP_CHECK(hipMemcpyAsync(&t, x->toklog + x->pos_host, 4, hipMemcpyDeviceToHost, x->s));
    DZ_HIP_CHECK(hipStreamSynchronize(x->s));
    out_tokens[i] = (uint32_t)t;
    *n_forwarded = i + 1;
    if (eos_id >= 0 && t == eos_id) break;
  }
  return DZ_OK;
}

int dz_verify_forward(dz_ctx* x, const uint32_t* draft, int k, float* per_pos_logits) {
  int rc = dz::ctx_verify_enqueue(x, draft, k);
  if (rc) return rc;
  // the context's stream is non-blocking: copy on it, then wait
  if (per_pos_logits)
    DZ_HIP_CHECK(hipMemcpyAsync(per_pos_logits, x->bt.logits, (size_t)k * x->m->cfg.vocab * 4, hipMemcpyDeviceToHost,
                                x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return DZ_OK;
}

int dz_verify_commit(dz_ctx* x, int n_accept) {
  if (!x) return set_error(DZ_ERR_MODEL, "null context");
  if (int rc0 = ctx_usable(x)) return rc0;
  if (x->bt.pending == 0 && n_accept == 0) return DZ_OK;
  if (x->bt.pending == 0) return set_error(DZ_ERR_TENSOR, "verify commit without a verify forward");
  return bt_verify_commit(x, n_accept);
}

int dz_ctx_vocab(const dz_ctx* x, int* vocab) {
  if (!x || !vocab) return set_error(DZ_ERR_MODEL, "null argument");
  *vocab = x->m->cfg.vocab;
  return DZ_OK;
}

int dz_ctx_logits(dz_ctx* x, float* logits) {
  if (!x || !logits) return set_error(DZ_ERR_MODEL, "null argument");
  DZ_HIP_CHECK(hipMemcpyAsync(logits, x->logits, (size_t)x->m->cfg.vocab * 4, hipMemcpyDeviceToHost, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return DZ_OK;
}

static int layer_of(dz_ctx* x, int layer, bool want_attn, LayerDev** out) {
  if (!x) return set_error(DZ_ERR_MODEL, "null context");
  if (layer < 0 || layer >= x->m->cfg.n_layers) return set_error(DZ_ERR_TENSOR, "layer %d out of range", layer);
  LayerDev& l = x->m->L[layer];
  if (l.attn != want_attn) return set_error(DZ_ERR_TENSOR, "layer %d is not a%s layer", layer, want_attn ? "n attention" : " DeltaNet");
  *out = &l;
  return DZ_OK;
}

int dz_ctx_set_ssm_state(dz_ctx* x, int layer, const float* state, const float* conv_hist, int conv_head) {
  LayerDev* l;
  int rc = layer_of(x, layer, false, &l);
  if (rc) return rc;
  const dz_config& c = x->m->cfg;
  const int64_t hd = c.ssm_state, nvh = c.ssm_v_heads, qkvd = (2 * (int64_t)c.ssm_k_heads + nvh) * hd;
  if (conv_head < 0 || conv_head > 3) return set_error(DZ_ERR_TENSOR, "conv_head %d", conv_head);
  DZ_HIP_CHECK(hipMemcpy(x->ssm_state + (size_t)l->kind_idx * nvh * hd * hd, state, (size_t)(nvh * hd * hd) * 4,
                         hipMemcpyHostToDevice));
  DZ_HIP_CHECK(hipMemcpy(x->conv + (size_t)l->kind_idx * 4 * qkvd, conv_hist, (size_t)(4 * qkvd) * 4, hipMemcpyHostToDevice));
  const int base = ((conv_head - x->pos_host) % 4 + 4) % 4;
  x->ring_base[l->kind_idx] = base;
  DZ_HIP_CHECK(hipMemcpy(x->ring_base_dev + l->kind_idx, &base, 4, hipMemcpyHostToDevice));
  return DZ_OK;
}

int dz_ctx_get_ssm_state(dz_ctx* x, int layer, float* state, float* conv_hist, int* conv_head) {
  LayerDev* l;
  int rc = layer_of(x, layer, false, &l);
  if (rc) return rc;
  const dz_config& c = x->m->cfg;
  const int64_t hd = c.ssm_state, nvh = c.ssm_v_heads, qkvd = (2 * (int64_t)c.ssm_k_heads + nvh) * hd;
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  if (state)
    DZ_HIP_CHECK(hipMemcpy(state, x->ssm_state + (size_t)l->kind_idx * nvh * hd * hd, (size_t)(nvh * hd * hd) * 4,
                           hipMemcpyDeviceToHost));
  if (conv_hist)
    DZ_HIP_CHECK(hipMemcpy(conv_hist, x->conv + (size_t)l->kind_idx * 4 * qkvd, (size_t)(4 * qkvd) * 4, hipMemcpyDeviceToHost));
  if (conv_head) *conv_head = (x->ring_base[l->kind_idx] + x->pos_host) & 3;
  return DZ_OK;
}

int dz_ctx_set_kv(dz_ctx* x, int layer, const float* k, const float* v, int len) {
  LayerDev* l;
  int rc = layer_of(x, layer, true, &l);
  if (rc) return rc;
  const dz_config& c = x->m->cfg;
  if (len < 0 || len > c.max_ctx) return set_error(DZ_ERR_TENSOR, "kv len %d", len);
  const size_t kvsz = (size_t)c.n_head_kv * c.max_ctx * c.head_dim, hd = (size_t)c.head_dim;
  float* kb = x->kv + (size_t)l->kind_idx * 2 * kvsz;
  for (int h = 0; h < c.n_head_kv; ++h) {
    DZ_HIP_CHECK(hipMemcpy(kb + (size_t)h * c.max_ctx * hd, k + (size_t)h * len * hd, (size_t)len * hd * 4, hipMemcpyHostToDevice));
    DZ_HIP_CHECK(hipMemcpy(kb + kvsz + (size_t)h * c.max_ctx * hd, v + (size_t)h * len * hd, (size_t)len * hd * 4,
                           hipMemcpyHostToDevice));
  }
  return DZ_OK;
}

int dz_ctx_get_kv(dz_ctx* x, int layer, float* k, float* v, int len) {
  LayerDev* l;
  int rc = layer_of(x, layer, true, &l);
  if (rc) return rc;
  const dz_config& c = x->m->cfg;
  if (len < 0 || len > c.max_ctx) return set_error(DZ_ERR_TENSOR, "kv len %d", len);
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  const size_t kvsz = (size_t)c.n_head_kv * c.max_ctx * c.head_dim, hd = (size_t)c.head_dim;
  const float* kb = x->kv + (size_t)l->kind_idx * 2 * kvsz;
  for (int h = 0; h < c.n_head_kv; ++h) {
    DZ_HIP_CHECK(hipMemcpy(k + (size_t)h * len * hd, kb + (size_t)h * c.max_ctx * hd, (size_t)len * hd * 4, hipMemcpyDeviceToHost));
    DZ_HIP_CHECK(hipMemcpy(v + (size_t)h * len * hd, kb + kvsz + (size_t)h * c.max_ctx * hd, (size_t)len * hd * 4,
                           hipMemcpyDeviceToHost));
  }
  return DZ_OK;
}

// In this build every attention layer holds exactly `pos` cached positions.
int dz_ctx_kv_len(dz_ctx* x, int layer) {
  LayerDev* l;
  if (layer_of(x, layer, true, &l)) return -1;
  return x->pos_host;
}

int dz_kv_truncate(dz_ctx* x, int len) {
  if (!x) return set_error(DZ_ERR_MODEL, "null context");
  x->bt.pending = 0;
  if (len >= x->pos_host) return DZ_OK;  // KvCache::truncate keeps longer requests as no-ops
  if (len < 0) return set_error(DZ_ERR_TENSOR, "truncate to %d", len);
  return ctx_move_pos(x, len);
}

int dz_ctx_set_pos(dz_ctx* x, int pos) {
  if (!x) return set_error(DZ_ERR_MODEL, "null context");
  x->bt.pending = 0;
  // max_ctx itself is a full context: forwards are refused there, but the state is valid
  if (pos < 0 || pos > x->m->cfg.max_ctx) return set_error(DZ_ERR_TENSOR, "pos %d out of [0, max_ctx]", pos);
  return ctx_move_pos(x, pos);
}

// ModelState::clone (forward.rs:31-77, derive(Clone); session_persist.rs:159 clones it for the
// background save) onto another context: dst takes src's position, DeltaNet states, conv rings and
// ring heads, the cached K/V rows [0, pos), the token log, and the last forward's logits and argmax
// candidates.  The two contexts may belong to different models of the same shape (max_ctx may
// differ if src's position fits dst's).
int dz_ctx_copy_state(dz_ctx* dst, const dz_ctx* src) {
  if (!dst || !src) return set_error(DZ_ERR_MODEL, "null context");
  if (dst == src) return DZ_OK;
  const dz_config &a = dst->m->cfg, &b = src->m->cfg;
  const bool same = a.n_layers == b.n_layers && a.hidden == b.hidden && a.ffn == b.ffn && a.vocab == b.vocab &&
                    a.n_head == b.n_head && a.n_head_kv == b.n_head_kv && a.head_dim == b.head_dim &&
                    a.rope_dim == b.rope_dim && a.rope_base == b.rope_base && a.rms_eps == b.rms_eps &&
                    a.full_attn_interval == b.full_attn_interval && a.ssm_conv_kernel == b.ssm_conv_kernel &&
                    a.ssm_state == b.ssm_state && a.ssm_k_heads == b.ssm_k_heads && a.ssm_v_heads == b.ssm_v_heads;
  if (!same) return set_error(DZ_ERR_MODEL, "copy_state: the contexts' model shapes differ");
  const int pos = src->pos_host;
  if (pos > a.max_ctx) return set_error(DZ_ERR_TENSOR, "copy_state: position %d exceeds max_ctx %d", pos, a.max_ctx);
  DZ_HIP_CHECK(hipStreamSynchronize(src->s));
  DZ_HIP_CHECK(hipStreamSynchronize(dst->s));
  dst->bt.pending = 0;
  const int64_t hd = a.ssm_state, qkvd = (2 * (int64_t)a.ssm_k_heads + a.ssm_v_heads) * hd;
  hipStream_t s = dst->s;
  const int n_ssm = dst->m->n_ssm, n_attn = dst->m->n_attn;
  if (n_ssm) {
    DZ_HIP_CHECK(hipMemcpyAsync(dst->ssm_state, src->ssm_state, (size_t)n_ssm * a.ssm_v_heads * hd * hd * 4,
                                hipMemcpyDeviceToDevice, s));
    DZ_HIP_CHECK(hipMemcpyAsync(dst->conv, src->conv, (size_t)n_ssm * 4 * qkvd * 4, hipMemcpyDeviceToDevice, s));
    DZ_HIP_CHECK(hipMemcpyAsync(dst->ring_base_dev, src->ring_base_dev, (size_t)n_ssm * 4, hipMemcpyDeviceToDevice, s));
  }
  if (n_attn && pos) {
    // rows [0, pos) of every (layer, K|V, kv head) block; each context strides by its own max_ctx
    const size_t row = (size_t)a.head_dim * 4;
    DZ_HIP_CHECK(hipMemcpy2DAsync(dst->kv, (size_t)a.max_ctx * row, src->kv, (size_t)b.max_ctx * row, (size_t)pos * row,
                                  (size_t)n_attn * 2 * a.n_head_kv, hipMemcpyDeviceToDevice, s));
  }
  DZ_HIP_CHECK(hipMemcpyAsync(dst->toklog, src->toklog, (size_t)(pos + 1) * 4, hipMemcpyDeviceToDevice, s));
  DZ_HIP_CHECK(hipMemcpyAsync(dst->logits, src->logits, (size_t)a.vocab * 4, hipMemcpyDeviceToDevice, s));
  DZ_HIP_CHECK(hipMemcpyAsync(dst->am_val, src->am_val, (size_t)dst->n_am * 4, hipMemcpyDeviceToDevice, s));
  DZ_HIP_CHECK(hipMemcpyAsync(dst->am_idx, src->am_idx, (size_t)dst->n_am * 4, hipMemcpyDeviceToDevice, s));
  TokState st;
  DZ_HIP_CHECK(hipMemcpy(&st, src->st, sizeof st, hipMemcpyDeviceToHost));
  st.feed_len = 0;  // host-fed ids belong to a call in progress, not to the state
  st.feed_idx = 0;
  DZ_HIP_CHECK(hipMemcpyAsync(dst->st, &st, sizeof st, hipMemcpyHostToDevice, s));
  DZ_HIP_CHECK(hipStreamSynchronize(s));
  dst->ring_base = src->ring_base;
  dst->pos_host = pos;
  dst->poisoned = src->poisoned;
  return DZ_OK;
}


int dz_ctx_mixer_step_dev(dz_ctx* x, int layer, const float* h_dev, float* h_out_dev) {
  if (!x || !h_dev || !h_out_dev) return set_error(DZ_ERR_MODEL, "null argument");
  if (int rc0 = ctx_usable(x)) return rc0;
  if (layer < 0 || layer >= x->m->cfg.n_layers) return set_error(DZ_ERR_TENSOR, "layer %d out of range", layer);
  if (x->pos_host >= x->m->cfg.max_ctx) return set_error(DZ_ERR_TENSOR, "context full");
  const dz_config& c = x->m->cfg;
  int64_t ld_in, ld_h, ld_gu;
  int th, to, tf;
  ctx_dims(x->m, &ld_in, &ld_h, &ld_gu, &th, &to, &tf);
  const int P = x->pos_host;
  x->bt.pending = 0;
  // the kernels take the position as an argument and read the caller's h directly; the residual
  // kernel writes the caller's output (which may be h itself: every read of h is in the first kernel)
  // and leaves TokState at this token (pos P, pos_next P + 1)
  int rc = enqueue_mixer(x, layer, h_dev, nullptr, 0, ld_h, x->h[0], x->ss[0], x->s, P);
  if (rc) return rc;
  FinalArgs fa{x->h[0], x->p_o, (int)x->m->L[layer].out_proj.ntiles, ld_h, h_out_dev, x->ss_fin, c.hidden, x->st, P};
  rc = with_np_bucket(fa.np, [&](auto B) -> int {
    hipLaunchKernelGGL(final_reduce_kernel<decltype(B)::value>, dim3((unsigned)th), dim3(512), 0, x->s, fa);
    DZ_HIP_CHECK(hipGetLastError());
    return DZ_OK;
  });
  if (rc) return rc;
  x->pos_host = P + 1;
  return DZ_OK;
}

int dz_ctx_mixer_step(dz_ctx* x, int layer, float* h) {
  if (!x || !h) return set_error(DZ_ERR_MODEL, "null argument");
  if (int rc0 = ctx_usable(x)) return rc0;
  if (layer < 0 || layer >= x->m->cfg.n_layers) return set_error(DZ_ERR_TENSOR, "layer %d out of range", layer);
  if (x->pos_host >= x->m->cfg.max_ctx) return set_error(DZ_ERR_TENSOR, "context full");
  const dz_config& c = x->m->cfg;
  int64_t ld_in, ld_h, ld_gu;
  int th, to, tf;
  ctx_dims(x->m, &ld_in, &ld_h, &ld_gu, &th, &to, &tf);
  const int P = x->pos_host;
  DZ_HIP_CHECK(hipMemcpyAsync(x->h[1], h, (size_t)c.hidden * 4, hipMemcpyHostToDevice, x->s));
  int rc = enqueue_mixer(x, layer, x->h[1], nullptr, 0, ld_h, x->h[0], x->ss[0], x->s, P);
  if (rc) return rc;
  // the residual kernel leaves TokState at this token (pos P, pos_next P + 1)
  FinalArgs fa{x->h[0], x->p_o, (int)x->m->L[layer].out_proj.ntiles, ld_h, x->h_fin, x->ss_fin, c.hidden, x->st, P};
  rc = with_np_bucket(fa.np, [&](auto B) -> int {
    hipLaunchKernelGGL(final_reduce_kernel<decltype(B)::value>, dim3((unsigned)th), dim3(512), 0, x->s, fa);
    DZ_HIP_CHECK(hipGetLastError());
    return DZ_OK;
  });
  if (rc) return rc;
  DZ_HIP_CHECK(hipMemcpyAsync(h, x->h_fin, (size_t)c.hidden * 4, hipMemcpyDeviceToHost, x->s));
  DZ_HIP_CHECK(hipStreamSynchronize(x->s));
  return ctx_set_pos_dev(x, P + 1);
}

}  // extern "C"
