// GGUF model files: header and metadata parsing, configuration, and a plan
// built straight from a read-only mapping of the file.
//
// Format (the layout the reference parses, tensor/GGUF.java:43-92,217-311):
// little-endian header {magic 'GGUF', version 2|3, tensor_count u64, kv_count
// u64}; kv_count metadata pairs {key string, value type u32, value}; tensor
// infos {name string, n_dims u32, dims u64[n_dims] (ne0 first), type u32,
// offset u64}; padding to general.alignment (default 32); tensor data, each
// tensor at its offset from the start of the data.  A string is {u64 length,
// bytes}; an array is {element type u32, count u64, elements}.
//
// Reference paths are relative to src/main/java/org/beehive/gpullama3/.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/gl3.h"
#include "gl3_host.h"

namespace {

using gl3::host_fail;

enum : uint32_t { GGUF_MAGIC = 0x46554747u, DEFAULT_ALIGNMENT = 32 };
// gguf metadata value types
enum : uint32_t {
  V_U8, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STRING, V_ARRAY, V_U64, V_I64, V_F64
};

struct Value {
  uint32_t type = 0;
  double num = 0.0;          // numeric scalars and bools
  std::string str;           // strings
  uint32_t elem_type = 0;    // arrays: element type and count (elements are skipped)
  uint64_t count = 0;
};

struct TensorInfo {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0;
};

struct Gguf {
  uint32_t version = 0;
  std::map<std::string, Value> meta;
  std::vector<TensorInfo> tensors;
  uint64_t data_offset = 0;  // file offset of the tensor data
  uint64_t file_size = 0;
};

// Bounds-checked little-endian reader over the mapped file.
struct Reader {
  const uint8_t *p;
  uint64_t size, pos = 0;
  bool ok = true;
  bool take(void *dst, uint64_t n) {
    if (!ok || n > size - pos) return ok = false;
    memcpy(dst, p + pos, n);
    pos += n;
    return true;
  }
  bool skip(uint64_t n) {
    if (!ok || n > size - pos) return ok = false;
    pos += n;
    return true;
  }
  template <class T>
  T get() {
    T v{};
    take(&v, sizeof v);
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (!ok || n > size - pos) {
      ok = false;
      return {};
    }
    std::string s((const char *)p + pos, (size_t)n);
    pos += n;
    return s;
  }
};

uint64_t scalar_size(uint32_t t) {
  switch (t) {
    case V_U8: case V_I8: case V_BOOL: return 1;
    case V_U16: case V_I16: return 2;
    case V_U32: case V_I32: case V_F32: return 4;
    case V_U64: case V_I64: case V_F64: return 8;
    default: return 0;
  }
}

double scalar(Reader &r, uint32_t t) {
  switch (t) {
    case V_U8: return r.get<uint8_t>();
    case V_I8: return r.get<int8_t>();
    case V_BOOL: return r.get<uint8_t>() != 0;
    case V_U16: return r.get<uint16_t>();
    case V_I16: return r.get<int16_t>();
    case V_U32: return r.get<uint32_t>();
    case V_I32: return r.get<int32_t>();
    case V_F32: return r.get<float>();
    case V_U64: return (double)r.get<uint64_t>();
    case V_I64: return (double)r.get<int64_t>();
    case V_F64: return r.get<double>();
    default: r.ok = false; return 0.0;
  }
}

bool read_value(Reader &r, uint32_t t, Value &v) {
  v.type = t;
  if (t == V_STRING) {
    v.str = r.str();
  } else if (t == V_ARRAY) {
    v.elem_type = r.get<uint32_t>();
    v.count = r.get<uint64_t>();
    if (v.elem_type == V_STRING) {
      for (uint64_t i = 0; i < v.count && r.ok; ++i) r.skip(r.get<uint64_t>());
    } else {
      const uint64_t es = scalar_size(v.elem_type);
      if (es == 0 || v.count > (r.size - r.pos) / es) return r.ok = false;
      r.skip(es * v.count);
    }
  } else if (scalar_size(t) != 0) {
    v.num = scalar(r, t);
  } else {
    return r.ok = false;
  }
  return r.ok;
}

// Bytes of a tensor of n elements (F32, F16, Q8_0 only: the types of this path).
bool tensor_bytes(uint32_t type, uint64_t n, uint64_t *out) {
  if (type == GL3_TYPE_F32) *out = 4 * n;
  else if (type == GL3_TYPE_F16) *out = 2 * n;
  else if (type == GL3_TYPE_Q8_0 && n % 32 == 0) *out = n / 32 * 34;
  else return false;
  return true;
}

// Header, metadata and tensor infos (GGUF.loadGGUFMetadata, tensor/GGUF.java:43-92).
int parse(const uint8_t *base, uint64_t size, Gguf &g) {
  Reader r{base, size};
  const uint32_t magic = r.get<uint32_t>();
  if (!r.ok || magic != GGUF_MAGIC) return host_fail(GL3_ERR_INVALID_ARGUMENT, "unsupported header.magic %#x", magic);
  g.version = r.get<uint32_t>();
  if (g.version != 2 && g.version != 3)
    return host_fail(GL3_ERR_UNSUPPORTED, "unsupported header.version %u", g.version);
  const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
  for (uint64_t i = 0; i < n_kv && r.ok; ++i) {
    std::string key = r.str();
    const uint32_t t = r.get<uint32_t>();
    Value v;
    if (!r.ok || !read_value(r, t, v)) break;
    g.meta[key] = std::move(v);
  }
  for (uint64_t i = 0; i < n_tensors && r.ok; ++i) {
    TensorInfo ti;
    ti.name = r.str();
    const uint32_t nd = r.get<uint32_t>();
    if (!r.ok || nd == 0 || nd > 4) return host_fail(GL3_ERR_INVALID_ARGUMENT, "tensor %s: %u dimensions", ti.name.c_str(), nd);
    for (uint32_t d = 0; d < nd; ++d) ti.dims.push_back(r.get<uint64_t>());
    ti.type = r.get<uint32_t>();
    ti.offset = r.get<uint64_t>();
    g.tensors.push_back(std::move(ti));
  }
  if (!r.ok) return host_fail(GL3_ERR_INVALID_ARGUMENT, "truncated GGUF header or metadata");
  uint64_t align = DEFAULT_ALIGNMENT;
  auto a = g.meta.find("general.alignment");
  if (a != g.meta.end() && a->second.type != V_STRING && a->second.type != V_ARRAY) align = (uint64_t)a->second.num;
  if (align == 0 || (align & (align - 1))) return host_fail(GL3_ERR_INVALID_ARGUMENT, "general.alignment %llu is not a power of two", (unsigned long long)align);
  g.data_offset = (r.pos + align - 1) / align * align;
  g.file_size = size;
  for (const TensorInfo &ti : g.tensors) {
    uint64_t n = 1, bytes = 0;
    for (uint64_t d : ti.dims) {
      if (d != 0 && n > (UINT64_MAX / 64) / d)
        return host_fail(GL3_ERR_INVALID_ARGUMENT, "tensor %s: too many elements", ti.name.c_str());
      n *= d;
    }
    if (ti.offset % align) return host_fail(GL3_ERR_INVALID_ARGUMENT, "tensor %s: offset not aligned", ti.name.c_str());
    if (!tensor_bytes(ti.type, n, &bytes)) continue;  // other types are checked where a tensor is used
    if (g.data_offset + ti.offset > size || bytes > size - g.data_offset - ti.offset)
      return host_fail(GL3_ERR_INVALID_ARGUMENT, "tensor %s: data past the end of the file", ti.name.c_str());
  }
  return GL3_OK;
}

bool num(const Gguf &g, const std::string &k, double *out) {
  auto it = g.meta.find(k);
  if (it == g.meta.end() || it->second.type == V_STRING || it->second.type == V_ARRAY) return false;
  *out = it->second.num;
  return true;
}

int need_int(const Gguf &g, const std::string &k, int32_t *out) {
  double v;
  if (!num(g, k, &v)) return host_fail(GL3_ERR_INVALID_ARGUMENT, "missing metadata %s", k.c_str());
  *out = (int32_t)v;
  return GL3_OK;
}

// ModelLoader.detectModelType (model/loader/ModelLoader.java:45-67): first match on the lower-cased general.name.
int detect_model_type(const Gguf &g, int32_t *type) {
  auto it = g.meta.find("general.name");
  if (it == g.meta.end() || it->second.type != V_STRING)
    return host_fail(GL3_ERR_UNSUPPORTED, "general.name is missing: unknown model type");
  std::string n = it->second.str;
  std::transform(n.begin(), n.end(), n.begin(), [](unsigned char c) { return (char)std::tolower(c); });
  if (n.find("mistral") != std::string::npos) *type = GL3_MODEL_MISTRAL;
  else if (n.find("llama") != std::string::npos) *type = GL3_MODEL_LLAMA_3;
  else if (n.find("qwen2") != std::string::npos) *type = GL3_MODEL_QWEN_2;
  else if (n.find("qwen3") != std::string::npos) *type = GL3_MODEL_QWEN_3;
  else if (n.find("deepseek r1 distill") != std::string::npos) *type = GL3_MODEL_DEEPSEEK_R1_DISTILL_QWEN;
  else if (n.find("phi3") != std::string::npos || n.find("phi-3") != std::string::npos) *type = GL3_MODEL_PHI_3;
  else return host_fail(GL3_ERR_UNSUPPORTED, "unknown model type for general.name \"%s\"", it->second.str.c_str());
  return GL3_OK;
}

const TensorInfo *find_tensor(const Gguf &g, const char *name) {
  for (const TensorInfo &t : g.tensors)
    if (t.name == name) return &t;
  return nullptr;
}

// The Configuration of the reference's loaders (LlamaModelLoader.java:47-62,
// MistralModelLoader.java:44-66, Qwen3ModelLoader.java:48-73, Phi3ModelLoader.java:45-60).
int make_config(const Gguf &g, int32_t context_length, uint32_t flags, gl3_config *c) {
  memset(c, 0, sizeof *c);
  c->abi_version = GL3_ABI_VERSION;
  c->flags = flags;
  int rc = detect_model_type(g, &c->model_type);
  if (rc) return rc;
  if (c->model_type == GL3_MODEL_QWEN_2 || c->model_type == GL3_MODEL_DEEPSEEK_R1_DISTILL_QWEN)
    return host_fail(GL3_ERR_UNSUPPORTED, "Qwen2 / DeepSeek-R1-Distill models (QKV bias) are not supported");
  const std::string a = c->model_type == GL3_MODEL_QWEN_3 ? "qwen3." : c->model_type == GL3_MODEL_PHI_3 ? "phi3." : "llama.";
  if ((rc = need_int(g, a + "embedding_length", &c->dim)) || (rc = need_int(g, a + "feed_forward_length", &c->hidden_dim)) ||
      (rc = need_int(g, a + "block_count", &c->n_layers)) || (rc = need_int(g, a + "attention.head_count", &c->n_heads)))
    return rc;
  double v;
  c->n_kv_heads = num(g, a + "attention.head_count_kv", &v) ? (int32_t)v : c->n_heads;
  if (c->n_heads <= 0) return host_fail(GL3_ERR_INVALID_ARGUMENT, "%sattention.head_count is %d", a.c_str(), c->n_heads);
  // head size: Qwen3 reads attention.key_length; the others use dim / heads
  if (c->model_type == GL3_MODEL_QWEN_3) {
    if ((rc = need_int(g, a + "attention.key_length", &c->head_dim))) return rc;
  } else {
    c->head_dim = c->dim / c->n_heads;
  }
  // vocabulary: llama.vocab_size when present (Llama, Mistral), else the token list
  auto tok = g.meta.find("tokenizer.ggml.tokens");
  const bool have_tokens = tok != g.meta.end() && tok->second.type == V_ARRAY;
  if (c->model_type != GL3_MODEL_QWEN_3 && c->model_type != GL3_MODEL_PHI_3 && num(g, "llama.vocab_size", &v))
    c->vocab_size = (int32_t)v;
  else if (have_tokens)
    c->vocab_size = (int32_t)tok->second.count;
  else
    return host_fail(GL3_ERR_INVALID_ARGUMENT, "no vocabulary size (llama.vocab_size or tokenizer.ggml.tokens)");
  // context length: Llama takes the requested one when given; Mistral and Qwen3 the
  // smaller of requested and the model's; Phi-3 uses the requested one as is
  if (c->model_type == GL3_MODEL_PHI_3) {
    if (context_length <= 0)
      return host_fail(GL3_ERR_INVALID_ARGUMENT, "Phi-3 needs a context length (its loader uses the requested one)");
    c->context_length = context_length;
  } else {
    int32_t model_ctx = 0;
    if ((rc = need_int(g, a + "context_length", &model_ctx))) return rc;
    if (c->model_type == GL3_MODEL_LLAMA_3)
      c->context_length = context_length < 0 ? model_ctx : context_length;
    else
      c->context_length = (context_length < 0 || model_ctx < context_length) ? model_ctx : context_length;
  }
  // eps and theta: Qwen3 requires them; the others default to 1e-5 and 10000
  if (c->model_type == GL3_MODEL_QWEN_3) {
    if (!num(g, a + "attention.layer_norm_rms_epsilon", &v)) return host_fail(GL3_ERR_INVALID_ARGUMENT, "missing metadata qwen3.attention.layer_norm_rms_epsilon");
    c->rms_norm_eps = (float)v;
    if (!num(g, a + "rope.freq_base", &v)) return host_fail(GL3_ERR_INVALID_ARGUMENT, "missing metadata qwen3.rope.freq_base");
    c->rope_theta = (float)v;
  } else {
    c->rms_norm_eps = num(g, a + "attention.layer_norm_rms_epsilon", &v) ? (float)v : 1e-5f;
    c->rope_theta = num(g, a + "rope.freq_base", &v) ? (float)v : 10000.0f;
  }
  // the planner key: the type of output.weight, or of token_embd when tied (AbstractModelLoader.java:146-150)
  const TensorInfo *out = find_tensor(g, "output.weight");
  if (!out) out = find_tensor(g, "token_embd.weight");
  if (!out) return host_fail(GL3_ERR_INVALID_ARGUMENT, "neither output.weight nor token_embd.weight is present");
  c->weight_type = (int32_t)out->type;
  return GL3_OK;
}

// GGUF tensor name -> (kind, layer); false for tensors this path does not read.
bool kind_of(const std::string &name, int *kind, int *layer) {
  static const std::map<std::string, int> kinds = {
      {"token_embd.weight", GL3_TOKEN_EMBD},   {"output_norm.weight", GL3_OUTPUT_NORM}, {"output.weight", GL3_OUTPUT},
      {"attn_norm.weight", GL3_ATTN_NORM},     {"attn_q.weight", GL3_ATTN_Q},           {"attn_k.weight", GL3_ATTN_K},
      {"attn_v.weight", GL3_ATTN_V},           {"attn_qkv.weight", GL3_ATTN_QKV},       {"attn_output.weight", GL3_ATTN_OUTPUT},
      {"attn_q_norm.weight", GL3_ATTN_Q_NORM}, {"attn_k_norm.weight", GL3_ATTN_K_NORM}, {"ffn_norm.weight", GL3_FFN_NORM},
      {"ffn_gate.weight", GL3_FFN_GATE},       {"ffn_up.weight", GL3_FFN_UP},           {"ffn_down.weight", GL3_FFN_DOWN}};
  std::string rest = name;
  *layer = 0;
  if (name.compare(0, 4, "blk.") == 0) {
    const size_t dot = name.find('.', 4);
    if (dot == std::string::npos || dot == 4) return false;
    for (size_t i = 4; i < dot; ++i)
      if (!isdigit((unsigned char)name[i])) return false;
    *layer = atoi(name.c_str() + 4);
    rest = name.substr(dot + 1);
  }
  auto it = kinds.find(rest);
  if (it == kinds.end()) return false;
  *kind = it->second;
  return true;
}

// A read-only mapping of a whole file.
struct Mapping {
  const uint8_t *p = nullptr;
  uint64_t size = 0;
  int open(const char *path) {
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) return host_fail(GL3_ERR_INVALID_ARGUMENT, "cannot open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
      ::close(fd);
      return host_fail(GL3_ERR_INVALID_ARGUMENT, "cannot read %s", path);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return host_fail(GL3_ERR_INVALID_ARGUMENT, "cannot map %s: %s", path, strerror(errno));
    p = (const uint8_t *)m;
    size = (uint64_t)st.st_size;
    return GL3_OK;
  }
  ~Mapping() {
    if (p) munmap((void *)p, (size_t)size);
  }
};

}  // namespace

extern "C" int gl3_gguf_config(const char *path, int32_t context_length, uint32_t flags, gl3_config *cfg_out) {
  if (!path || !cfg_out) return host_fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  Mapping m;
  int rc = m.open(path);
  if (rc) return rc;
  Gguf g;
  if ((rc = parse(m.p, m.size, g))) return rc;
  return make_config(g, context_length, flags, cfg_out);
}

extern "C" int gl3_create_from_gguf(const char *path, int32_t context_length, uint32_t flags, gl3_plan **out) {
  if (!path || !out) return host_fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  Mapping m;
  int rc = m.open(path);
  if (rc) return rc;
  Gguf g;
  gl3_config cfg;
  if ((rc = parse(m.p, m.size, g)) || (rc = make_config(g, context_length, flags, &cfg))) return rc;
  gl3_plan *p = nullptr;
  if ((rc = gl3_create(&cfg, &p))) return rc;
  for (const TensorInfo &t : g.tensors) {
    int kind = 0, layer = 0;
    // rope_freqs.weight and any tensor this path does not read are skipped (GGUF.java:120-123)
    if (!kind_of(t.name, &kind, &layer)) continue;
    uint64_t n = 1, bytes = 0;
    for (uint64_t d : t.dims) n *= d;
    if (!tensor_bytes(t.type, n, &bytes)) {
      gl3_destroy(p);
      return host_fail(GL3_ERR_UNSUPPORTED, "tensor %s: GGML type %u is not supported", t.name.c_str(), t.type);
    }
    if ((rc = gl3_upload(p, kind, layer, m.p + g.data_offset + t.offset, (size_t)bytes, (int)t.type))) {
      gl3_destroy(p);
      return rc;
    }
  }
  if ((rc = gl3_prepare(p))) {
    gl3_destroy(p);
    return rc;
  }
  *out = p;
  return GL3_OK;
}
