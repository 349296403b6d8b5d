// gguf.hip — GGUF v3 files to device weights: the header parser of GgufFile::open
// (Daiza-engine/src/gguf/parser.rs:40-119, metadata.rs, tensor_info.rs:41-201), the model config
// of Config::from_metadata (model/config.rs:76-160) and LoadedWeights::load_all
// (model/weights.rs:1308-1379) through dz_model_create.  Host code only: the file is memory-mapped
// read-only and the tensors are handed to dz_model_create as slices of the mapping (no copy on the
// host; the device upload repacks them).
#include "runtime.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <map>
#include <string>
#include <vector>

namespace dz {

// GGUF metadata value types (gguf_metadata_value_type).
enum GgufVt { kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64 };

struct GgufValue {
  int type = -1;
  uint64_t u = 0;  // integer and bool values (sign-extended for the signed types)
  double f = 0.0;  // float values
  std::string s;
  int elem_type = -1;               // arrays
  std::vector<GgufValue> elems;
};

struct GgufTensor {
  std::string name;
  std::vector<uint64_t> dims;  // GGUF order: dims[0] = columns (innermost)
  uint32_t type = 0;
  uint64_t offset = 0;         // from the data section's start
  uint64_t n_bytes = 0;        // 0 for a type this build does not size
};

// Bounds-checked little-endian reader over the mapping.
struct GgufReader {
  const uint8_t* p;
  size_t n, pos = 0;
  bool fail = false;
  bool need(size_t k) {
    if (fail || pos + k > n || pos + k < pos) {
      fail = true;
      return false;
    }
    return true;
  }
  template <class T>
  T get() {
    T v{};
    if (need(sizeof(T))) {
      memcpy(&v, p + pos, sizeof(T));
      pos += sizeof(T);
    }
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    if (len > (1u << 30) || !need((size_t)len)) {
      fail = true;
      return std::string();
    }
    std::string s(reinterpret_cast<const char*>(p + pos), (size_t)len);
    pos += (size_t)len;
    return s;
  }
};

static bool read_scalar(GgufReader& r, int t, GgufValue& v) {
  v.type = t;
  switch (t) {
    case kU8: v.u = r.get<uint8_t>(); break;
    case kI8: v.u = (uint64_t)(int64_t)r.get<int8_t>(); break;
    case kU16: v.u = r.get<uint16_t>(); break;
    case kI16: v.u = (uint64_t)(int64_t)r.get<int16_t>(); break;
    case kU32: v.u = r.get<uint32_t>(); break;
    case kI32: v.u = (uint64_t)(int64_t)r.get<int32_t>(); break;
    case kF32: v.f = r.get<float>(); break;
    case kBool: v.u = r.get<uint8_t>() != 0; break;
    case kStr: v.s = r.str(); break;
    case kU64: v.u = r.get<uint64_t>(); break;
    case kI64: v.u = (uint64_t)r.get<int64_t>(); break;
    case kF64: v.f = r.get<double>(); break;
    default: return false;
  }
  return !r.fail;
}

static bool read_value(GgufReader& r, int t, GgufValue& v) {
  if (t != kArr) return read_scalar(r, t, v);
  v.type = kArr;
  v.elem_type = (int)r.get<uint32_t>();
  const uint64_t len = r.get<uint64_t>();
  if (r.fail || len > (r.n - r.pos)) return false;  // every element takes at least one byte
  v.elems.resize((size_t)len);
  for (auto& e : v.elems)
    if (!read_scalar(r, v.elem_type, e)) return false;
  return true;
}

// Bytes of n elements of a ggml type, as byte_size (tensor/dtype.rs) for the types of this path.
// Bytes of n elements of a loadable type (0 for other types).  *overflow is set when the size does
// not fit 64 bits.
static uint64_t type_bytes(uint32_t type, uint64_t n, bool* overflow) {
  uint64_t r = 0;
  switch (type) {
    case 0: *overflow |= __builtin_mul_overflow(n, (uint64_t)4, &r); return r;   // F32
    case 1:                                                                       // F16
    case 30: *overflow |= __builtin_mul_overflow(n, (uint64_t)2, &r); return r;  // BF16
    case 41:  // Q1_0: 18 bytes per 128 weights
      if (n % kGroup) return 0;
      *overflow |= __builtin_mul_overflow(n / kGroup, (uint64_t)kBlockBytes, &r);
      return r;
    default: return 0;
  }
}

}  // namespace dz

struct dz_gguf {
  int fd = -1;
  const uint8_t* map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t alignment = 32;
  uint64_t data_offset = 0;
  std::map<std::string, dz::GgufValue> kv;
  std::vector<dz::GgufTensor> tensors;
  std::map<std::string, size_t> index;
};

using namespace dz;

static void gguf_release(dz_gguf* g) {
  if (!g) return;
  if (g->map) munmap(const_cast<uint8_t*>(g->map), g->size);
  if (g->fd >= 0) close(g->fd);
  delete g;
}

extern "C" {

int dz_gguf_open(const char* path, dz_gguf** out) {
  if (!path || !out) return set_error(DZ_ERR_MODEL, "null argument");
  dz_gguf* g = new dz_gguf();
  auto fail = [&](int code) {
    gguf_release(g);
    return code;
  };
  g->fd = open(path, O_RDONLY);
  if (g->fd < 0) return fail(set_error(DZ_ERR_MODEL, "open %s: %s", path, strerror(errno)));
  struct stat st;
  if (fstat(g->fd, &st) != 0 || st.st_size < 24) return fail(set_error(DZ_ERR_MODEL, "%s: too short for GGUF", path));
  g->size = (size_t)st.st_size;
  void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
  if (m == MAP_FAILED) return fail(set_error(DZ_ERR_MODEL, "mmap %s: %s", path, strerror(errno)));
  g->map = static_cast<const uint8_t*>(m);
  GgufReader r{g->map, g->size};
  const uint32_t magic = r.get<uint32_t>();
  if (magic != 0x46554747u) return fail(set_error(DZ_ERR_MODEL, "bad GGUF magic 0x%08X", magic));
  g->version = r.get<uint32_t>();
  if (g->version != 3) return fail(set_error(DZ_ERR_MODEL, "unsupported GGUF version %u (only 3)", g->version));
  const uint64_t n_tensors = r.get<uint64_t>();
  const uint64_t n_kv = r.get<uint64_t>();
  if (r.fail || n_tensors > (1u << 24) || n_kv > (1u << 24)) return fail(set_error(DZ_ERR_MODEL, "bad GGUF counts"));
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key = r.str();
    const int t = (int)r.get<uint32_t>();
    GgufValue v;
    if (r.fail || !read_value(r, t, v))
      return fail(set_error(DZ_ERR_MODEL, "GGUF metadata entry %llu (%s): bad value of type %d", (unsigned long long)i,
                            key.c_str(), t));
    g->kv[key] = std::move(v);
  }
  // general.alignment as Metadata::get_u64 reads it (parser.rs:74, metadata.rs): only a u64 or i64
  // value counts; any other type (the spec writes u32) leaves the default 32, as in the reference
  auto al = g->kv.find("general.alignment");
  if (al != g->kv.end() && (al->second.type == kU64 || al->second.type == kI64)) g->alignment = al->second.u;
  if (g->alignment == 0) return fail(set_error(DZ_ERR_MODEL, "general.alignment must be > 0"));
  g->tensors.resize((size_t)n_tensors);
  for (auto& t : g->tensors) {
    t.name = r.str();
    const uint32_t nd = r.get<uint32_t>();
    if (r.fail || nd > 4) return fail(set_error(DZ_ERR_MODEL, "tensor %s: %u dims (at most 4)", t.name.c_str(), nd));
    uint64_t ne = 1;
    bool ovf = false;
    for (uint32_t d = 0; d < nd; ++d) {
      t.dims.push_back(r.get<uint64_t>());
      ovf |= __builtin_mul_overflow(ne, t.dims.back(), &ne);
    }
    t.type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    t.n_bytes = type_bytes(t.type, ne, &ovf);
    if (r.fail) return fail(set_error(DZ_ERR_MODEL, "truncated GGUF tensor table"));
    if (ovf) return fail(set_error(DZ_ERR_MODEL, "tensor %s: size overflows 64 bits", t.name.c_str()));
  }
  // the data section starts at the next multiple of the alignment
  g->data_offset = ((uint64_t)r.pos + g->alignment - 1) / g->alignment * g->alignment;
  for (size_t i = 0; i < g->tensors.size(); ++i) {
    const GgufTensor& t = g->tensors[i];
    // compared without sums that could wrap: offset and size each within what follows the data start
    const uint64_t room = g->size > g->data_offset ? g->size - g->data_offset : 0;
    if (t.n_bytes && (t.offset > room || t.n_bytes > room - t.offset))
      return fail(set_error(DZ_ERR_MODEL, "tensor %s data out of range", t.name.c_str()));
    g->index[t.name] = i;
  }
  *out = g;
  return DZ_OK;
}

int dz_gguf_close(dz_gguf* g) {
  gguf_release(g);
  return DZ_OK;
}

int dz_gguf_n_tensors(const dz_gguf* g) { return g ? (int)g->tensors.size() : -1; }

int dz_gguf_tensor_info(const dz_gguf* g, int i, const char** name, int32_t* type, int32_t* n_dims, uint64_t* dims,
                        uint64_t* offset, uint64_t* n_bytes) {
  if (!g || i < 0 || i >= (int)g->tensors.size()) return set_error(DZ_ERR_TENSOR, "tensor index %d", i);
  const GgufTensor& t = g->tensors[(size_t)i];
  if (name) *name = t.name.c_str();
  if (type) *type = (int32_t)t.type;
  if (n_dims) *n_dims = (int32_t)t.dims.size();
  if (dims)
    for (size_t d = 0; d < 4; ++d) dims[d] = d < t.dims.size() ? t.dims[d] : 1;
  if (offset) *offset = g->data_offset + t.offset;
  if (n_bytes) *n_bytes = t.n_bytes;
  return DZ_OK;
}

const void* dz_gguf_tensor_data(const dz_gguf* g, int i) {
  if (!g || i < 0 || i >= (int)g->tensors.size() || !g->tensors[(size_t)i].n_bytes) return nullptr;
  return g->map + g->data_offset + g->tensors[(size_t)i].offset;
}

// Config::from_metadata (config.rs:76-160): Config::default with every qwen35.* key present; the
// vocabulary is the length of tokenizer.ggml.tokens when that reads as an integer array (a string
// array, as in real files, keeps the default 248320, as the reference does).
int dz_gguf_config(const dz_gguf* g, int32_t max_ctx, dz_config* cfg, int32_t* eos_token_id) {
  if (!g || !cfg) return set_error(DZ_ERR_MODEL, "null argument");
  auto it = g->kv.find("general.architecture");
  if (it == g->kv.end() || it->second.type != kStr) return set_error(DZ_ERR_MODEL, "missing general.architecture");
  if (it->second.s != "qwen35")
    return set_error(DZ_ERR_MODEL, "expected architecture 'qwen35', got '%s'", it->second.s.c_str());
  dz_config_bonsai27b(cfg, max_ctx);
  int32_t eos = 248046;
  auto u32 = [&](const char* key, int32_t* dst) {
    auto f = g->kv.find(key);
    if (f != g->kv.end() && (f->second.type == kU32 || f->second.type == kI32)) *dst = (int32_t)f->second.u;
  };
  auto f32 = [&](const char* key, float* dst) {
    auto f = g->kv.find(key);
    if (f != g->kv.end() && f->second.type == kF32) *dst = (float)f->second.f;
  };
  u32("qwen35.block_count", &cfg->n_layers);
  u32("qwen35.embedding_length", &cfg->hidden);
  u32("qwen35.feed_forward_length", &cfg->ffn);
  u32("qwen35.attention.head_count", &cfg->n_head);
  u32("qwen35.attention.head_count_kv", &cfg->n_head_kv);
  u32("qwen35.attention.key_length", &cfg->head_dim);
  f32("qwen35.attention.layer_norm_rms_epsilon", &cfg->rms_eps);
  u32("qwen35.rope.dimension_count", &cfg->rope_dim);
  f32("qwen35.rope.freq_base", &cfg->rope_base);
  u32("qwen35.full_attention_interval", &cfg->full_attn_interval);
  u32("qwen35.ssm.conv_kernel", &cfg->ssm_conv_kernel);
  u32("qwen35.ssm.state_size", &cfg->ssm_state);
  u32("qwen35.ssm.group_count", &cfg->ssm_k_heads);
  u32("qwen35.ssm.time_step_rank", &cfg->ssm_v_heads);
  u32("tokenizer.ggml.eos_token_id", &eos);
  auto tk = g->kv.find("tokenizer.ggml.tokens");
  if (tk != g->kv.end() && tk->second.type == kArr && (tk->second.elem_type == kI32 || tk->second.elem_type == kU32))
    cfg->vocab = (int32_t)tk->second.elems.size();
  // the token embedding's storage type decides the embedding format (Q1_0 in the reference's files)
  auto te = g->index.find("token_embd.weight");
  if (te != g->index.end()) cfg->embd_f16 = g->tensors[te->second].type == 1 ? 1 : 0;
  if (eos_token_id) *eos_token_id = eos;
  return DZ_OK;
}

// Config::context_length (config.rs:52, 92-93): qwen35.context_length read with Metadata::get_u64,
// so only a u64 or i64 value replaces the default 262144.  It sizes nothing on this path; DZSS
// session files hash it.
int dz_gguf_context_length(const dz_gguf* g, uint64_t* out) {
  if (!g || !out) return set_error(DZ_ERR_MODEL, "null argument");
  *out = 262144;
  auto f = g->kv.find("qwen35.context_length");
  if (f != g->kv.end() && (f->second.type == kU64 || f->second.type == kI64)) *out = f->second.u;
  return DZ_OK;
}

// LoadedWeights::load_all (weights.rs:1308-1379): every tensor of the file, by name, to
// dz_model_create, which checks the names, types and sizes the model needs.
int dz_model_create_gguf(const dz_gguf* g, const dz_config* cfg, dz_model** out) {
  if (!g || !cfg || !out) return set_error(DZ_ERR_MODEL, "null argument");
  std::vector<dz_tensor> t;
  t.reserve(g->tensors.size());
  for (const GgufTensor& x : g->tensors) {
    if (!x.n_bytes) continue;  // a type this path does not use
    dz_tensor d;
    d.name = x.name.c_str();
    d.type = (int32_t)x.type;
    d.data = g->map + g->data_offset + x.offset;
    d.n_bytes = (size_t)x.n_bytes;
    t.push_back(d);
  }
  return dz_model_create(cfg, t.data(), (int)t.size(), out);
}

}  // extern "C"
