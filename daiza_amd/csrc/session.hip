// session.hip — DZSS session snapshots of a context: Session::save_to_disk / load_from_disk
// (Daiza-runtime/src/session_persist.rs:47-312), file format v1, on the device state.
//
//   header, 128 bytes: "DZSS", u32 version 1, u64 cfg_hash, u64 pos, u64 n_history, u32 n_blocks,
//                      u8 think_enabled, u8 has_system_prompt, zeros
//   u32 history[n_history]
//   per block, in layer order: u8 kind; kind 0 (attention): u64 per_token (= n_kv_heads * head_dim),
//     u64 len, f32 k[len][n_kv_heads][head_dim], f32 v[...]; kind 1 (DeltaNet): u64 state_len,
//     f32 state[state_len] (S[v head][i][j]), u64 conv_len, f32 conv[4][qkv_dim] (ring rows), u64 conv_head
//   if has_system_prompt: u64 length, bytes
//
// cfg_hash is the reference's cfg_hash: Rust's DefaultHasher (SipHash-1-3, keys 0 and 0) over ten
// usize fields written as 8-byte little-endian words: block_count, hidden, head_count, head_count_kv,
// head_dim, full_attention_interval, ssm_state_size, ssm_time_step_rank, ssm_conv_kernel,
// context_length.  Host code: the state moves through the context's state accessors.
#include "runtime.h"

#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include <sys/stat.h>

namespace dz {

static inline uint64_t rotl64(uint64_t x, int b) { return (x << b) | (x >> (64 - b)); }

// SipHash with c compression and d finalisation rounds (Aumasson and Bernstein, 2012), 128-bit key
// (k0, k1), 64-bit output.
uint64_t siphash(int c, int d, uint64_t k0, uint64_t k1, const uint8_t* m, size_t n) {
  uint64_t v0 = k0 ^ 0x736f6d6570736575ull, v1 = k1 ^ 0x646f72616e646f6dull;
  uint64_t v2 = k0 ^ 0x6c7967656e657261ull, v3 = k1 ^ 0x7465646279746573ull;
  auto round = [&]() {
    v0 += v1; v1 = rotl64(v1, 13); v1 ^= v0; v0 = rotl64(v0, 32);
    v2 += v3; v3 = rotl64(v3, 16); v3 ^= v2;
    v0 += v3; v3 = rotl64(v3, 21); v3 ^= v0;
    v2 += v1; v1 = rotl64(v1, 17); v1 ^= v2; v2 = rotl64(v2, 32);
  };
  const size_t full = n / 8;
  for (size_t i = 0; i < full; ++i) {
    uint64_t w;
    memcpy(&w, m + 8 * i, 8);
    v3 ^= w;
    for (int r = 0; r < c; ++r) round();
    v0 ^= w;
  }
  uint64_t last = (uint64_t)(n & 0xFF) << 56;
  for (size_t i = 0; i < (n & 7); ++i) last |= (uint64_t)m[8 * full + i] << (8 * i);
  v3 ^= last;
  for (int r = 0; r < c; ++r) round();
  v0 ^= last;
  v2 ^= 0xFF;
  for (int r = 0; r < d; ++r) round();
  return v0 ^ v1 ^ v2 ^ v3;
}

}  // namespace dz

using namespace dz;

namespace {

constexpr size_t kDzssHeader = 128;

bool is_attn(const dz_config& c, int i) {
  return c.full_attn_interval == 0 || i % c.full_attn_interval == c.full_attn_interval - 1;
}

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) fclose(f);
  }
};

bool wr(FILE* f, const void* p, size_t n) { return fwrite(p, 1, n, f) == n; }
bool rd(FILE* f, void* p, size_t n) { return fread(p, 1, n, f) == n; }
bool wr64(FILE* f, uint64_t v) { return wr(f, &v, 8); }
bool rd64(FILE* f, uint64_t* v) { return rd(f, v, 8); }

}  // namespace

extern "C" {

uint64_t dz_session_cfg_hash(const dz_config* c, uint64_t context_length) {
  if (!c) return 0;
  const uint64_t w[10] = {(uint64_t)c->n_layers,  (uint64_t)c->hidden,    (uint64_t)c->n_head,
                          (uint64_t)c->n_head_kv, (uint64_t)c->head_dim,  (uint64_t)c->full_attn_interval,
                          (uint64_t)c->ssm_state, (uint64_t)c->ssm_v_heads, (uint64_t)c->ssm_conv_kernel,
                          context_length};
  uint8_t m[80];
  for (int i = 0; i < 10; ++i) memcpy(m + 8 * i, &w[i], 8);  // little-endian host
  return siphash(1, 3, 0, 0, m, sizeof m);
}

static int ctx_save(dz_ctx* x, const char* path, uint64_t context_length, const uint32_t* history, uint64_t n_history,
                    int32_t think_enabled, const char* system_prompt) {
  if (!x || !path || (!history && n_history)) return set_error(DZ_ERR_MODEL, "null argument");
  // a context left inconsistent by a failed launch is not a session state
  if (int rc0 = ctx_usable(x)) return rc0;
  const dz_config* c = ctx_config(x);
  const int pos = dz_ctx_pos(x);
  File fh;
  fh.f = fopen(path, "wb");
  if (!fh.f) return set_error(DZ_ERR_MODEL, "create %s", path);
  FILE* f = fh.f;
  uint8_t hdr[kDzssHeader] = {};
  memcpy(hdr, "DZSS", 4);
  const uint32_t ver = 1, nb = (uint32_t)c->n_layers;
  const uint64_t h = dz_session_cfg_hash(c, context_length), p = (uint64_t)pos;
  memcpy(hdr + 4, &ver, 4);
  memcpy(hdr + 8, &h, 8);
  memcpy(hdr + 16, &p, 8);
  memcpy(hdr + 24, &n_history, 8);
  memcpy(hdr + 32, &nb, 4);
  hdr[36] = think_enabled ? 1 : 0;
  hdr[37] = system_prompt ? 1 : 0;
  bool ok = wr(f, hdr, sizeof hdr) && wr(f, history, (size_t)n_history * 4);
  const int64_t hd = c->ssm_state, qkvd = (2 * (int64_t)c->ssm_k_heads + c->ssm_v_heads) * hd;
  const size_t st_n = (size_t)c->ssm_v_heads * hd * hd, cv_n = (size_t)c->ssm_conv_kernel * qkvd;
  const size_t per_tok = (size_t)c->n_head_kv * c->head_dim, hdim = (size_t)c->head_dim;
  std::vector<float> a, b, fa, fb;
  for (int l = 0; ok && l < c->n_layers; ++l) {
    int rc;
    if (is_attn(*c, l)) {
      // KvCache per kv head [kvh][seq][dim] -> the file's [seq][kvh][dim]
      a.resize(per_tok * (size_t)pos);
      b.resize(per_tok * (size_t)pos);
      fa.resize(a.size());
      fb.resize(b.size());
      if (pos && (rc = dz_ctx_get_kv(x, l, a.data(), b.data(), pos))) return rc;
      for (int s = 0; s < pos; ++s)
        for (int h2 = 0; h2 < c->n_head_kv; ++h2) {
          memcpy(&fa[((size_t)s * c->n_head_kv + h2) * hdim], &a[((size_t)h2 * pos + s) * hdim], hdim * 4);
          memcpy(&fb[((size_t)s * c->n_head_kv + h2) * hdim], &b[((size_t)h2 * pos + s) * hdim], hdim * 4);
        }
      const uint8_t kind = 0;
      ok = wr(f, &kind, 1) && wr64(f, per_tok) && wr64(f, (uint64_t)pos) && wr(f, fa.data(), fa.size() * 4) &&
           wr(f, fb.data(), fb.size() * 4);
    } else {
      a.resize(st_n);
      b.resize(cv_n);
      int head = 0;
      if ((rc = dz_ctx_get_ssm_state(x, l, a.data(), b.data(), &head))) return rc;
      // a state that has seen no token has an empty conv history in the reference (SsmState::new,
      // ssm_state.rs:24-31; the ring is sized on the first token), written as conv_len 0
      const size_t cn = pos ? cv_n : 0;
      const uint8_t kind = 1;
      ok = wr(f, &kind, 1) && wr64(f, st_n) && wr(f, a.data(), st_n * 4) && wr64(f, cn) && wr(f, b.data(), cn * 4) &&
           wr64(f, (uint64_t)head);
    }
  }
  if (ok && system_prompt) {
    const uint64_t n = strlen(system_prompt);
    ok = wr64(f, n) && wr(f, system_prompt, (size_t)n);
  }
  if (!ok || fflush(f) != 0) return set_error(DZ_ERR_MODEL, "write %s", path);
  return DZ_OK;
}

static int ctx_load(dz_ctx* x, const char* path, uint64_t context_length, uint32_t* history, uint64_t history_cap,
                    uint64_t* n_history, int32_t* think_enabled, char* system_prompt, uint64_t prompt_cap,
                    uint64_t* prompt_len) {
  if (!x || !path) return set_error(DZ_ERR_MODEL, "null argument");
  const dz_config* c = ctx_config(x);
  File fh;
  fh.f = fopen(path, "rb");
  if (!fh.f) return set_error(DZ_ERR_MODEL, "open %s", path);
  FILE* f = fh.f;
  uint8_t hdr[kDzssHeader];
  if (!rd(f, hdr, sizeof hdr)) return set_error(DZ_ERR_MODEL, "%s: short header", path);
  if (memcmp(hdr, "DZSS", 4) != 0) return set_error(DZ_ERR_MODEL, "invalid magic (not a Daiza session file)");
  uint32_t ver, nb;
  uint64_t h, pos, nh;
  memcpy(&ver, hdr + 4, 4);
  memcpy(&h, hdr + 8, 8);
  memcpy(&pos, hdr + 16, 8);
  memcpy(&nh, hdr + 24, 8);
  memcpy(&nb, hdr + 32, 4);
  if (ver != 1) return set_error(DZ_ERR_MODEL, "unsupported version %u, expected 1", ver);
  const uint64_t want = dz_session_cfg_hash(c, context_length);
  if (h != want)
    return set_error(DZ_ERR_MODEL, "cfg hash mismatch: file=%016llx expected=%016llx (model mismatch?)",
                     (unsigned long long)h, (unsigned long long)want);
  if (nb != (uint32_t)c->n_layers) return set_error(DZ_ERR_MODEL, "block_count mismatch: file=%u expected=%d", nb, c->n_layers);
  if (pos > (uint64_t)c->max_ctx) return set_error(DZ_ERR_TENSOR, "session position %llu exceeds max_ctx %d",
                                                   (unsigned long long)pos, c->max_ctx);
  // the history is bounded before anything is allocated for it: at most 2^32 tokens, and no more
  // than the bytes left after the header
  struct stat sb;
  if (fstat(fileno(f), &sb) != 0) return set_error(DZ_ERR_MODEL, "stat %s", path);
  const uint64_t left = (uint64_t)sb.st_size > kDzssHeader ? (uint64_t)sb.st_size - kDzssHeader : 0;
  if (nh > (1ull << 32) || nh > left / 4)
    return set_error(DZ_ERR_MODEL, "%s: history of %llu tokens exceeds the file", path, (unsigned long long)nh);
  std::vector<uint32_t> hist((size_t)nh);
  if (!rd(f, hist.data(), (size_t)nh * 4)) return set_error(DZ_ERR_MODEL, "%s: short history", path);
  // read every block before touching the context, so that a bad file leaves it as it was
  const int64_t hd = c->ssm_state, qkvd = (2 * (int64_t)c->ssm_k_heads + c->ssm_v_heads) * hd;
  const size_t st_n = (size_t)c->ssm_v_heads * hd * hd, cv_n = (size_t)c->ssm_conv_kernel * qkvd;
  const size_t per_tok = (size_t)c->n_head_kv * c->head_dim, hdim = (size_t)c->head_dim;
  struct Blk {
    std::vector<float> a, b;
    uint64_t head = 0;
  };
  std::vector<Blk> blk((size_t)c->n_layers);
  for (int l = 0; l < c->n_layers; ++l) {
    uint8_t kind = 0xFF;
    if (!rd(f, &kind, 1)) return set_error(DZ_ERR_MODEL, "%s: short file at block %d", path, l);
    Blk& B = blk[(size_t)l];
    if (is_attn(*c, l)) {
      uint64_t pt, len;
      if (kind != 0) return set_error(DZ_ERR_MODEL, "block %d: expected KV (kind=0), got kind=%u", l, kind);
      if (!rd64(f, &pt) || !rd64(f, &len)) return set_error(DZ_ERR_MODEL, "%s: short file at block %d", path, l);
      if (pt != per_tok || len != pos)
        return set_error(DZ_ERR_TENSOR, "block %d: KV of %llu x %llu, expected %zu x %llu", l, (unsigned long long)len,
                         (unsigned long long)pt, per_tok, (unsigned long long)pos);
      std::vector<float> fa(per_tok * (size_t)len), fb(fa.size());
      if (!rd(f, fa.data(), fa.size() * 4) || !rd(f, fb.data(), fb.size() * 4))
        return set_error(DZ_ERR_MODEL, "%s: short KV at block %d", path, l);
      // the file's [seq][kvh][dim] -> KvCache per kv head [kvh][seq][dim]
      B.a.resize(fa.size());
      B.b.resize(fb.size());
      for (uint64_t s = 0; s < len; ++s)
        for (int h2 = 0; h2 < c->n_head_kv; ++h2) {
          memcpy(&B.a[((size_t)h2 * len + s) * hdim], &fa[((size_t)s * c->n_head_kv + h2) * hdim], hdim * 4);
          memcpy(&B.b[((size_t)h2 * len + s) * hdim], &fb[((size_t)s * c->n_head_kv + h2) * hdim], hdim * 4);
        }
    } else {
      uint64_t sn, cn;
      if (kind != 1) return set_error(DZ_ERR_MODEL, "block %d: expected SSM (kind=1), got kind=%u", l, kind);
      if (!rd64(f, &sn) || sn != st_n) return set_error(DZ_ERR_TENSOR, "block %d: SSM state of %llu floats", l, (unsigned long long)sn);
      B.a.resize(st_n);
      if (!rd(f, B.a.data(), st_n * 4)) return set_error(DZ_ERR_MODEL, "%s: short SSM state at block %d", path, l);
      // conv_len 0: the empty history of a state that has seen no token, i.e. a zero ring
      if (!rd64(f, &cn) || (cn != cv_n && cn != 0))
        return set_error(DZ_ERR_TENSOR, "block %d: conv history of %llu floats", l, (unsigned long long)cn);
      B.b.assign(cv_n, 0.0f);
      if (!rd(f, B.b.data(), (size_t)cn * 4) || !rd64(f, &B.head))
        return set_error(DZ_ERR_MODEL, "%s: short conv history at block %d", path, l);
      if (B.head >= (uint64_t)c->ssm_conv_kernel) return set_error(DZ_ERR_TENSOR, "block %d: conv_head %llu", l, (unsigned long long)B.head);
    }
  }
  std::string sys;
  const bool has_sys = hdr[37] != 0;
  if (has_sys) {
    uint64_t n;
    if (!rd64(f, &n) || n > (1ull << 30)) return set_error(DZ_ERR_MODEL, "%s: bad system prompt", path);
    sys.resize((size_t)n);
    if (n && !rd(f, &sys[0], (size_t)n)) return set_error(DZ_ERR_MODEL, "%s: short system prompt", path);
  }
  if (history && nh > history_cap) return set_error(DZ_ERR_TENSOR, "history of %llu tokens, buffer of %llu",
                                                    (unsigned long long)nh, (unsigned long long)history_cap);
  if (system_prompt && has_sys && sys.size() + 1 > prompt_cap)
    return set_error(DZ_ERR_TENSOR, "system prompt of %zu bytes, buffer of %llu", sys.size(), (unsigned long long)prompt_cap);
  // the context: a fresh state at the file's position, then every block (ModelState rebuilt, pos set)
  int rc = dz_ctx_reset(x);
  if (rc || (pos && (rc = dz_ctx_set_pos(x, (int)pos)))) return rc;
  for (int l = 0; l < c->n_layers; ++l) {
    Blk& B = blk[(size_t)l];
    if (is_attn(*c, l))
      rc = pos ? dz_ctx_set_kv(x, l, B.a.data(), B.b.data(), (int)pos) : DZ_OK;
    else
      rc = dz_ctx_set_ssm_state(x, l, B.a.data(), B.b.data(), (int)B.head);
    if (rc) return rc;
  }
  if (n_history) *n_history = nh;
  if (history && nh) memcpy(history, hist.data(), (size_t)nh * 4);
  if (think_enabled) *think_enabled = hdr[36] != 0;
  if (prompt_len) *prompt_len = has_sys ? sys.size() : 0;
  if (system_prompt && prompt_cap) {
    const size_t n = has_sys ? sys.size() : 0;
    memcpy(system_prompt, sys.data(), n);
    system_prompt[n] = 0;
  }
  return DZ_OK;
}

// The C entry points: no C++ exception (an allocation that fails, for one) leaves the library.
int dz_ctx_save(dz_ctx* x, const char* path, uint64_t context_length, const uint32_t* history, uint64_t n_history,
                int32_t think_enabled, const char* system_prompt) {
  try {
    return ctx_save(x, path, context_length, history, n_history, think_enabled, system_prompt);
  } catch (const std::exception& ex) {
    return set_error(DZ_ERR_MODEL, "session save: %s", ex.what());
  } catch (...) {
    return set_error(DZ_ERR_MODEL, "session save: unexpected exception");
  }
}

int dz_ctx_load(dz_ctx* x, const char* path, uint64_t context_length, uint32_t* history, uint64_t history_cap,
                uint64_t* n_history, int32_t* think_enabled, char* system_prompt, uint64_t prompt_cap,
                uint64_t* prompt_len) {
  try {
    return ctx_load(x, path, context_length, history, history_cap, n_history, think_enabled, system_prompt,
                    prompt_cap, prompt_len);
  } catch (const std::exception& ex) {
    return set_error(DZ_ERR_MODEL, "session load: %s", ex.what());
  } catch (...) {
    return set_error(DZ_ERR_MODEL, "session load: unexpected exception");
  }
}

}  // extern "C"
