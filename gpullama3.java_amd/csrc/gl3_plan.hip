// Host side of libgpullama3_hip.so: the C ABI declared in include/gl3.h.
//
// A gl3_plan owns the device copy of the model (weights in the GEMV layout,
// fp16 KV cache, activations), one HIP stream, and the per-token schedule:
// either the persistent per-token kernel (one cooperative launch per token) or
// the per-phase kernels captured once in a hipGraph.
//
// Reference paths are relative to src/main/java/org/beehive/gpullama3/.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/gl3.h"
#include "gl3_host.h"
#include "gl3_internal.h"

using namespace gl3;

// ------------------------------------------------------------ errors

static thread_local std::string g_last_error;

static int vfail(int code, const char *fmt, va_list ap) {
  char buf[512];
  vsnprintf(buf, sizeof buf, fmt, ap);
  g_last_error = buf;
  return code;
}
static int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int r = vfail(code, fmt, ap);
  va_end(ap);
  return r;
}
int gl3::host_fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  const int r = vfail(code, fmt, ap);
  va_end(ap);
  return r;
}

#define HIP_TRY(expr)                                                                                     \
  do {                                                                                                    \
    hipError_t e_ = (expr);                                                                               \
    if (e_ != hipSuccess) {                                                                               \
      if (e_ == hipErrorOutOfMemory || e_ == hipErrorMemoryAllocation)                                    \
        return fail(GL3_ERR_OUT_OF_MEMORY, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
      return fail(GL3_ERR_DEVICE, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__);   \
    }                                                                                                     \
  } while (0)

extern "C" const char *gl3_last_error(void) { return g_last_error.c_str(); }

// ------------------------------------------------------------ the plan

struct DevMat {
  uint8_t *q = nullptr;
  uint16_t *s = nullptr;
  int rows = 0, cols = 0;
  Mat view() const { return Mat{q, s, rows, cols}; }
};

struct gl3_plan {
  gl3_config cfg{};
  int family = 0, fmt = 0, embd_fmt = -1, cls_fmt = -1;
  int q_dim = 0, kv_dim = 0, G = 0;
  int device = 0, n_cu = 0;
  hipStream_t stream = nullptr;
  std::vector<void *> allocs;

  // device model
  std::vector<DevMat> qkv, wo, gu, down;
  std::vector<DevMat> down_sl;  // fused FFN: Wdown in 32-column slices
  uint2 *tdp = nullptr;         // fused FFN: down partials [grid][dim]
  int hidden = 0;
  std::vector<float *> attn_norm, ffn_norm, q_norm, k_norm;
  DevMat embd, cls;
  bool cls_tied = true;
  float *out_norm = nullptr;
  LayerDev *layers_d = nullptr;
  ModelDev m{};

  // upload bookkeeping: bit per (kind, layer)
  std::vector<uint32_t> uploaded;  // per layer: bitmask of kinds
  uint32_t uploaded_global = 0;
  bool rope_set = false;

  // schedule
  bool prepared = false;
  bool use_step_kernel = false;
  StepKernel sk;
  int step_grid = 0;
  int logits_grid = 0;
  int nbest = 0;
  GridBarrier gb{};
  unsigned epoch = 0;     // grid barriers completed since the counters were last zeroed
  unsigned tag = 1;       // next tag of the persistent kernel's tagged vectors (0 = never written)
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;

  // staging
  uint8_t *staging = nullptr;
  size_t staging_bytes = 0;
  // batched prefill workspace, allocated on first use: residual rows, q/k/v
  // rows, and two pairs of hi / lo fp16 activation planes (a: normed rows and
  // attention output, b: SwiGLU output)
  float *pf_x = nullptr, *pf_qkv = nullptr, *pf_part = nullptr;
  _Float16 *pf_ah = nullptr, *pf_al = nullptr, *pf_bh = nullptr, *pf_bl = nullptr;
  float *probs = nullptr;             // sampler scratch [2 vocab]: probabilities, then candidate indices
  float *coins = nullptr;             // sampler draws of the current generate call [context length]
  DecodeState *h_state = nullptr;     // pinned
  unsigned long long *h_best = nullptr;  // pinned [nbest]
  unsigned *h_err = nullptr;          // pinned

  // timing
  std::vector<hipEvent_t> ev;
  int ev_used = 0;
  hipEvent_t ev_begin = nullptr, ev_end = nullptr;
  double last_elapsed_ms = 0, last_kernel_ms = 0;
  int last_launches = 0;
};

// Tagged vectors of the persistent kernel back to "never written" (tag 0).
static hipError_t zero_tagged(gl3_plan *p) {
  const ModelDev &m = p->m;
  const size_t n[7] = {(size_t)m.dim, (size_t)m.dim, (size_t)(m.q_dim + 2 * m.kv_dim), (size_t)m.q_dim,
                       (size_t)m.hidden, (size_t)m.n_heads * m.max_split * (m.hd + 4),
                       (size_t)p->step_grid * m.dim};
  uint2 *b[7] = {m.txa, m.txb, m.tqkv, m.tatt, m.thb, m.tpart, m.tdp};
  for (int i = 0; i < 7; ++i) {
    if (!b[i]) continue;
    hipError_t e = hipMemsetAsync(b[i], 0, n[i] * sizeof(uint2), p->stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <class T>
static int dev_alloc(gl3_plan *p, T **out, size_t count) {
  void *ptr = nullptr;
  size_t bytes = count * sizeof(T);
  if (bytes == 0) bytes = 16;
  hipError_t e = hipMalloc(&ptr, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(e == hipErrorOutOfMemory ? GL3_ERR_OUT_OF_MEMORY : GL3_ERR_DEVICE, "hipMalloc(%zu bytes): %s", bytes,
                hipGetErrorString(e));
  }
  p->allocs.push_back(ptr);
  *out = (T *)ptr;
  return GL3_OK;
}

static int alloc_mat(gl3_plan *p, DevMat &dm, int fmt, int rows, int cols) {
  dm.rows = rows;
  dm.cols = cols;
  size_t n = (size_t)rows * cols;
  int rc;
  if (fmt == FMT_Q8) {
    if ((rc = dev_alloc(p, &dm.q, n))) return rc;
    if ((rc = dev_alloc(p, &dm.s, n / 32))) return rc;
  } else if (fmt == FMT_F16) {
    if ((rc = dev_alloc(p, &dm.q, n * 2))) return rc;
  } else {
    if ((rc = dev_alloc(p, &dm.q, n * 4))) return rc;
  }
  return GL3_OK;
}

static int ggml_to_fmt(int t) {
  switch (t) {
    case GL3_TYPE_Q8_0: return FMT_Q8;
    case GL3_TYPE_F16: return FMT_F16;
    case GL3_TYPE_F32: return FMT_F32;
    default: return -1;
  }
}
static size_t fmt_bytes(int fmt, size_t n) { return fmt == FMT_Q8 ? n / 32 * 34 : fmt == FMT_F16 ? n * 2 : n * 4; }

// Host-side RoPE tables: RoPE.precomputeFreqsCis without scaling
// (inference/operation/RoPE.java:6-37; scaling is never enabled, LlamaModelLoader.java:67).
static void rope_tables(int ctx, int hs, double theta, std::vector<float> &cr, std::vector<float> &ci) {
  cr.resize((size_t)ctx * (hs / 2));
  ci.resize(cr.size());
  size_t n = 0;
  for (int pos = 0; pos < ctx; ++pos)
    for (int i = 0; i < hs; i += 2) {
      float freq = (float)(1.0 / std::pow(theta, i / (double)hs));
      float val = (float)pos * freq;
      cr[n] = (float)std::cos((double)val);
      ci[n] = (float)std::sin((double)val);
      ++n;
    }
}

static void destroy_plan(gl3_plan *p) {
  if (!p) return;
  if (p->stream) (void)hipStreamSynchronize(p->stream);
  if (p->graph_exec) (void)hipGraphExecDestroy(p->graph_exec);
  if (p->graph) (void)hipGraphDestroy(p->graph);
  for (hipEvent_t e : p->ev) (void)hipEventDestroy(e);
  if (p->ev_begin) (void)hipEventDestroy(p->ev_begin);
  if (p->ev_end) (void)hipEventDestroy(p->ev_end);
  for (void *a : p->allocs) (void)hipFree(a);
  if (p->staging) (void)hipFree(p->staging);
  if (p->h_state) (void)hipHostFree(p->h_state);
  if (p->h_best) (void)hipHostFree(p->h_best);
  if (p->h_err) (void)hipHostFree(p->h_err);
  if (p->stream) (void)hipStreamDestroy(p->stream);
  delete p;
}

extern "C" void gl3_destroy(gl3_plan *p) { destroy_plan(p); }

extern "C" int gl3_device_name(char *buf, size_t len) {
  if (!buf || len == 0) return fail(GL3_ERR_INVALID_ARGUMENT, "buffer is null");
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, dev));
  snprintf(buf, len, "%s %s", prop.name, prop.gcnArchName);
  return GL3_OK;
}

// QuantizationPlannerFactory.create (layerplanner/base/QuantizationPlannerFactory.java:41-73)
// routes (weight type, model type) to a planner; the same pairs are accepted here.
static int validate_config(const gl3_config *c, int *family) {
  if (!c) return fail(GL3_ERR_INVALID_ARGUMENT, "config is null");
  if (c->abi_version != GL3_ABI_VERSION)
    return fail(GL3_ERR_INVALID_ARGUMENT, "abi_version %d, library implements %d", c->abi_version, GL3_ABI_VERSION);
  switch (c->model_type) {
    case GL3_MODEL_LLAMA_3:
    case GL3_MODEL_MISTRAL: *family = FAM_LLAMA; break;
    case GL3_MODEL_QWEN_3: *family = FAM_QWEN3; break;
    case GL3_MODEL_PHI_3: *family = FAM_PHI3; break;
    case GL3_MODEL_QWEN_2:
    case GL3_MODEL_DEEPSEEK_R1_DISTILL_QWEN:
      return fail(GL3_ERR_UNSUPPORTED, "model type %d (Qwen2-style QKV bias) is not supported", c->model_type);
    default: return fail(GL3_ERR_INVALID_ARGUMENT, "unknown model type %d", c->model_type);
  }
  if (c->weight_type != GL3_TYPE_F16 && c->weight_type != GL3_TYPE_Q8_0)
    return fail(GL3_ERR_UNSUPPORTED, "weight type %d: only F16 and Q8_0 are supported", c->weight_type);
  if (c->dim <= 0 || c->hidden_dim <= 0 || c->n_layers <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 ||
      c->head_dim <= 0 || c->vocab_size <= 0 || c->context_length <= 0)
    return fail(GL3_ERR_INVALID_ARGUMENT, "non-positive shape parameter");
  if (c->n_heads % c->n_kv_heads) return fail(GL3_ERR_INVALID_ARGUMENT, "n_heads %% n_kv_heads != 0");
  if (*family != FAM_QWEN3 && c->head_dim * c->n_heads != c->dim)
    return fail(GL3_ERR_INVALID_ARGUMENT, "head_dim * n_heads must equal dim for this model type");
  const int G = c->n_heads / c->n_kv_heads;
  if (!attention_supported(c->head_dim, G))
    return fail(GL3_ERR_UNSUPPORTED, "head_dim %d (64, 96 or 128) / GQA group %d (1, 2, 3, 4 or 8) not supported",
                c->head_dim, G);
  if (!(c->rms_norm_eps > 0.0f) || !(c->rope_theta > 0.0f)) return fail(GL3_ERR_INVALID_ARGUMENT, "eps/theta");
  const int fmt = ggml_to_fmt(c->weight_type);
  const int q_dim = c->n_heads * c->head_dim;
  if (!gemv_supported(fmt, c->dim) || !gemv_supported(fmt, q_dim) || !gemv_supported(fmt, c->hidden_dim))
    return fail(GL3_ERR_UNSUPPORTED, "dim %d / q_dim %d / hidden %d not supported by the GEMV kernels for this type",
                c->dim, q_dim, c->hidden_dim);
  return GL3_OK;
}

extern "C" int gl3_create(const gl3_config *cfg, gl3_plan **out) {
  if (!out) return fail(GL3_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  int family = 0;
  int rc = validate_config(cfg, &family);
  if (rc) return rc;
  gl3_plan *p = new gl3_plan();
  p->cfg = *cfg;
  p->family = family;
  p->fmt = ggml_to_fmt(cfg->weight_type);
  p->q_dim = cfg->n_heads * cfg->head_dim;
  p->kv_dim = cfg->n_kv_heads * cfg->head_dim;
  p->G = cfg->n_heads / cfg->n_kv_heads;
  const int L = cfg->n_layers, dim = cfg->dim, H = cfg->hidden_dim, hd = cfg->head_dim;
  hipError_t he;
  if ((he = hipGetDevice(&p->device)) != hipSuccess) {
    destroy_plan(p);
    return fail(GL3_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(he));
  }
  hipDeviceProp_t prop;
  if ((he = hipGetDeviceProperties(&prop, p->device)) != hipSuccess || (he = hipStreamCreate(&p->stream)) != hipSuccess) {
    destroy_plan(p);
    return fail(GL3_ERR_DEVICE, "device setup: %s", hipGetErrorString(he));
  }
  p->n_cu = prop.multiProcessorCount;
#define TRY(x)            \
  do {                    \
    int r_ = (x);         \
    if (r_) {             \
      destroy_plan(p);    \
      return r_;          \
    }                     \
  } while (0)
  p->qkv.resize(L);
  p->wo.resize(L);
  p->gu.resize(L);
  p->down.resize(L);
  p->down_sl.resize(L);
  p->hidden = H;
  p->attn_norm.assign(L, nullptr);
  p->ffn_norm.assign(L, nullptr);
  p->q_norm.assign(L, nullptr);
  p->k_norm.assign(L, nullptr);
  p->uploaded.assign(L, 0u);
  for (int l = 0; l < L; ++l) {
    TRY(alloc_mat(p, p->qkv[l], p->fmt, p->q_dim + 2 * p->kv_dim, dim));
    TRY(alloc_mat(p, p->wo[l], p->fmt, dim, p->q_dim));
    TRY(alloc_mat(p, p->gu[l], p->fmt, 2 * H, dim));
    TRY(alloc_mat(p, p->down[l], p->fmt, dim, H));
    TRY(dev_alloc(p, &p->attn_norm[l], dim));
    TRY(dev_alloc(p, &p->ffn_norm[l], dim));
    if (family == FAM_QWEN3) {
      TRY(dev_alloc(p, &p->q_norm[l], hd));
      TRY(dev_alloc(p, &p->k_norm[l], hd));
    }
  }
  TRY(dev_alloc(p, &p->out_norm, dim));
  TRY(dev_alloc(p, &p->layers_d, L));

  ModelDev &m = p->m;
  m.family = family;
  m.fmt = p->fmt;
  m.dim = dim;
  m.hidden = H;
  m.n_layers = L;
  m.n_heads = cfg->n_heads;
  m.n_kv = cfg->n_kv_heads;
  m.hd = hd;
  m.q_dim = p->q_dim;
  m.kv_dim = p->kv_dim;
  m.vocab = cfg->vocab_size;
  m.ctx = cfg->context_length;
  m.ctxp = (cfg->context_length + 15) / 16 * 16;
  m.eps = cfg->rms_norm_eps;
  m.sqrt_hd = (float)std::sqrt((double)hd);  // (float) Math.sqrt(headSize), InferenceCore.java:64
  // about one attention work item (kv head, split) per CU
  int ms = p->n_cu / cfg->n_kv_heads;
  m.max_split = ms < 1 ? 1 : (ms > 256 ? 256 : ms);
  m.out_norm = p->out_norm;
  m.layers = p->layers_d;
  size_t kv_elems = (size_t)L * cfg->n_kv_heads * m.ctxp * hd;
  TRY(dev_alloc(p, &m.kc, kv_elems));
  TRY(dev_alloc(p, &m.vc, kv_elems));
  float *rc_ = nullptr, *rs_ = nullptr;
  TRY(dev_alloc(p, &rc_, (size_t)cfg->context_length * (hd / 2)));
  TRY(dev_alloc(p, &rs_, (size_t)cfg->context_length * (hd / 2)));
  m.rope_cos = rc_;
  m.rope_sin = rs_;
  TRY(dev_alloc(p, &m.x, dim));
  TRY(dev_alloc(p, &m.qkv, p->q_dim + 2 * p->kv_dim));
  TRY(dev_alloc(p, &m.att, p->q_dim));
  TRY(dev_alloc(p, &m.hb, H));
  TRY(dev_alloc(p, &m.txa, dim));
  TRY(dev_alloc(p, &m.txb, dim));
  TRY(dev_alloc(p, &m.tqkv, p->q_dim + 2 * p->kv_dim));
  TRY(dev_alloc(p, &m.tatt, p->q_dim));
  TRY(dev_alloc(p, &m.thb, H));
  TRY(dev_alloc(p, &m.logits, cfg->vocab_size));
  TRY(dev_alloc(p, &m.part, (size_t)cfg->n_heads * m.max_split * (hd + 4)));
  TRY(dev_alloc(p, &m.tpart, (size_t)cfg->n_heads * m.max_split * (hd + 4)));
  TRY(dev_alloc(p, &m.att_ctr, (size_t)L * cfg->n_kv_heads));
  p->nbest = 2048;
  if (p->n_cu > p->nbest) p->nbest = (p->n_cu + 3) & ~3;  // whole 16-byte key pairs per parity half
  TRY(dev_alloc(p, &m.best, 2 * (size_t)p->nbest));
  TRY(dev_alloc(p, &m.st, 1));
  TRY(dev_alloc(p, &m.tokens_out, (size_t)cfg->context_length));
  TRY(dev_alloc(p, &p->probs, 2 * (size_t)cfg->vocab_size));
  TRY(dev_alloc(p, &p->coins, (size_t)cfg->context_length));
  {
    int *pr = nullptr;
    TRY(dev_alloc(p, &pr, (size_t)cfg->context_length));
    m.prompt = pr;
  }
  if (cfg->flags & GL3_FLAG_PHASE_TRACE) TRY(dev_alloc(p, &m.tstamp, (size_t)(4 + 10 * L) * p->n_cu));
  unsigned *bar = nullptr;
  TRY(dev_alloc(p, &bar, GL3_BAR_GROUPS * GL3_BAR_STRIDE + 64));
  p->gb.ctr = bar;
  p->gb.err = bar + GL3_BAR_GROUPS * GL3_BAR_STRIDE;
  p->gb.spin_limit = 1u << 20;
  if (hipHostMalloc((void **)&p->h_state, sizeof(DecodeState)) != hipSuccess ||
      hipHostMalloc((void **)&p->h_best, sizeof(unsigned long long) * p->nbest) != hipSuccess ||
      hipHostMalloc((void **)&p->h_err, 64) != hipSuccess) {
    destroy_plan(p);
    return fail(GL3_ERR_OUT_OF_MEMORY, "pinned host allocation failed");
  }
  // zero-initialised state (fresh State: zero KV, LlamaState.java:61-64)
  if ((he = hipMemsetAsync(m.kc, 0, kv_elems * 2, p->stream)) != hipSuccess ||
      (he = hipMemsetAsync(m.vc, 0, kv_elems * 2, p->stream)) != hipSuccess ||
      (he = hipMemsetAsync(m.att_ctr, 0, (size_t)L * cfg->n_kv_heads * 4, p->stream)) != hipSuccess ||
      (he = hipMemsetAsync(bar, 0, (GL3_BAR_GROUPS * GL3_BAR_STRIDE + 64) * 4, p->stream)) != hipSuccess ||
      (he = hipMemsetAsync(m.best, 0, 2 * (size_t)p->nbest * 8, p->stream)) != hipSuccess ||
      (he = hipMemsetAsync(m.x, 0, (size_t)dim * 4, p->stream)) != hipSuccess ||
      (he = zero_tagged(p)) != hipSuccess) {
    destroy_plan(p);
    return fail(GL3_ERR_DEVICE, "hipMemsetAsync: %s", hipGetErrorString(he));
  }
  // RoPE tables computed here unless the host provides its own
  {
    std::vector<float> cr, ci;
    rope_tables(cfg->context_length, hd, (double)cfg->rope_theta, cr, ci);
    if ((he = hipMemcpy(rc_, cr.data(), cr.size() * 4, hipMemcpyHostToDevice)) != hipSuccess ||
        (he = hipMemcpy(rs_, ci.data(), ci.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) {
      destroy_plan(p);
      return fail(GL3_ERR_DEVICE, "rope upload: %s", hipGetErrorString(he));
    }
  }
  if ((he = hipEventCreate(&p->ev_begin)) != hipSuccess || (he = hipEventCreate(&p->ev_end)) != hipSuccess) {
    destroy_plan(p);
    return fail(GL3_ERR_DEVICE, "hipEventCreate: %s", hipGetErrorString(he));
  }
#undef TRY
  *out = p;
  return GL3_OK;
}

// --------------------------------------------------------------- upload

static int ensure_staging(gl3_plan *p, size_t bytes) {
  if (p->staging_bytes >= bytes) return GL3_OK;
  if (p->staging) {
    (void)hipStreamSynchronize(p->stream);
    (void)hipFree(p->staging);
    p->staging = nullptr;
    p->staging_bytes = 0;
  }
  hipError_t e = hipMalloc((void **)&p->staging, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(GL3_ERR_OUT_OF_MEMORY, "staging buffer of %zu bytes: %s", bytes, hipGetErrorString(e));
  }
  p->staging_bytes = bytes;
  return GL3_OK;
}

// Copy a [rows][cols] matrix in GGUF encoding into rows [row0, row0+rows) of dm.
static int upload_matrix(gl3_plan *p, DevMat &dm, int row0, int rows, int cols, int fmt, const void *host) {
  const size_t n = (size_t)rows * cols;
  const size_t off = (size_t)row0 * cols;
  if (fmt == FMT_Q8) {
    int rc = ensure_staging(p, n / 32 * 34);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(p->staging, host, n / 32 * 34, hipMemcpyHostToDevice, p->stream));
    HIP_TRY(launch_repack_q8(p->staging, n / 32, dm.q + off, dm.s + off / 32, p->stream));
  } else if (fmt == FMT_F16) {
    HIP_TRY(hipMemcpyAsync(dm.q + off * 2, host, n * 2, hipMemcpyHostToDevice, p->stream));
  } else {
    HIP_TRY(hipMemcpyAsync(dm.q + off * 4, host, n * 4, hipMemcpyHostToDevice, p->stream));
  }
  HIP_TRY(hipStreamSynchronize(p->stream));  // host memory is borrowed for the call only
  return GL3_OK;
}

static int upload_f32(gl3_plan *p, float *dst, const void *host, size_t n) {
  HIP_TRY(hipMemcpyAsync(dst, host, n * 4, hipMemcpyHostToDevice, p->stream));
  HIP_TRY(hipStreamSynchronize(p->stream));
  return GL3_OK;
}

static bool is_layer_kind(int kind) { return kind >= GL3_ATTN_NORM && kind <= GL3_FFN_DOWN; }

extern "C" int gl3_upload(gl3_plan *p, int kind, int layer, const void *host, size_t bytes, int ggml_type) {
  if (!p || !host) return fail(GL3_ERR_INVALID_ARGUMENT, "null plan or host pointer");
  const gl3_config &c = p->cfg;
  const int dim = c.dim, H = c.hidden_dim, hd = c.head_dim;
  if (kind < 0 || kind > GL3_FFN_DOWN) return fail(GL3_ERR_INVALID_ARGUMENT, "unknown tensor kind %d", kind);
  if (is_layer_kind(kind) && (layer < 0 || layer >= c.n_layers))
    return fail(GL3_ERR_INVALID_ARGUMENT, "layer %d out of range [0,%d)", layer, c.n_layers);
  const int fmt = ggml_to_fmt(ggml_type);
  if (fmt < 0) return fail(GL3_ERR_UNSUPPORTED, "ggml type %d is not supported", ggml_type);

  auto expect = [&](int want_fmt, size_t n) -> int {
    if (fmt != want_fmt)
      return fail(GL3_ERR_INVALID_ARGUMENT, "tensor kind %d: ggml type %d does not match the plan's weight type", kind,
                  ggml_type);
    if (bytes != fmt_bytes(fmt, n))
      return fail(GL3_ERR_INVALID_ARGUMENT, "tensor kind %d: %zu bytes, expected %zu", kind, bytes, fmt_bytes(fmt, n));
    return GL3_OK;
  };
  int rc = GL3_OK;
  const bool phi3 = p->family == FAM_PHI3, qwen3 = p->family == FAM_QWEN3;
  switch (kind) {
    case GL3_TOKEN_EMBD: {
      const size_t n = (size_t)c.vocab_size * dim;
      if (bytes != fmt_bytes(fmt, n)) return fail(GL3_ERR_INVALID_ARGUMENT, "token_embd: %zu bytes, expected %zu", bytes, fmt_bytes(fmt, n));
      if (fmt == FMT_Q8 && dim % 32) return fail(GL3_ERR_INVALID_ARGUMENT, "Q8_0 rows must hold whole blocks");
      if (p->embd.q && p->embd_fmt != fmt) return fail(GL3_ERR_INVALID_ARGUMENT, "token_embd type changed");
      if (!p->embd.q && (rc = alloc_mat(p, p->embd, fmt, c.vocab_size, dim))) return rc;
      p->embd_fmt = fmt;
      rc = upload_matrix(p, p->embd, 0, c.vocab_size, dim, fmt, host);
      break;
    }
    case GL3_OUTPUT: {
      // the planner key: output.weight's type (LlamaModelLoader.java:108,137)
      if ((rc = expect(ggml_to_fmt(c.weight_type), (size_t)c.vocab_size * dim))) return rc;
      if (!p->cls.q || p->cls_tied) {
        p->cls = DevMat();
        if ((rc = alloc_mat(p, p->cls, fmt, c.vocab_size, dim))) return rc;
      }
      p->cls_tied = false;
      p->cls_fmt = fmt;
      rc = upload_matrix(p, p->cls, 0, c.vocab_size, dim, fmt, host);
      break;
    }
    case GL3_OUTPUT_NORM:
      if ((rc = expect(FMT_F32, dim))) return rc;
      rc = upload_f32(p, p->out_norm, host, dim);
      break;
    case GL3_ATTN_NORM:
      if ((rc = expect(FMT_F32, dim))) return rc;
      rc = upload_f32(p, p->attn_norm[layer], host, dim);
      break;
    case GL3_FFN_NORM:
      if ((rc = expect(FMT_F32, dim))) return rc;
      rc = upload_f32(p, p->ffn_norm[layer], host, dim);
      break;
    case GL3_ATTN_Q_NORM:
    case GL3_ATTN_K_NORM:
      if (!qwen3) return fail(GL3_ERR_INVALID_ARGUMENT, "per-head Q/K norms exist only for Qwen3");
      if ((rc = expect(FMT_F32, hd))) return rc;
      rc = upload_f32(p, kind == GL3_ATTN_Q_NORM ? p->q_norm[layer] : p->k_norm[layer], host, hd);
      break;
    case GL3_ATTN_Q:
    case GL3_ATTN_K:
    case GL3_ATTN_V: {
      if (phi3) return fail(GL3_ERR_INVALID_ARGUMENT, "Phi3 uses the fused attn_qkv tensor");
      const int rows = kind == GL3_ATTN_Q ? p->q_dim : p->kv_dim;
      const int row0 = kind == GL3_ATTN_Q ? 0 : kind == GL3_ATTN_K ? p->q_dim : p->q_dim + p->kv_dim;
      if ((rc = expect(p->fmt, (size_t)rows * dim))) return rc;
      rc = upload_matrix(p, p->qkv[layer], row0, rows, dim, fmt, host);
      break;
    }
    case GL3_ATTN_QKV:
      if (!phi3) return fail(GL3_ERR_INVALID_ARGUMENT, "attn_qkv exists only for Phi3");
      if ((rc = expect(p->fmt, (size_t)(p->q_dim + 2 * p->kv_dim) * dim))) return rc;
      rc = upload_matrix(p, p->qkv[layer], 0, p->q_dim + 2 * p->kv_dim, dim, fmt, host);
      break;
    case GL3_ATTN_OUTPUT:
      if ((rc = expect(p->fmt, (size_t)dim * p->q_dim))) return rc;
      rc = upload_matrix(p, p->wo[layer], 0, dim, p->q_dim, fmt, host);
      break;
    case GL3_FFN_GATE:
      if (phi3) return fail(GL3_ERR_INVALID_ARGUMENT, "Phi3 uses the fused gate-up ffn_up tensor");
      if ((rc = expect(p->fmt, (size_t)H * dim))) return rc;
      rc = upload_matrix(p, p->gu[layer], 0, H, dim, fmt, host);
      break;
    case GL3_FFN_UP:
      if (phi3) {
        if ((rc = expect(p->fmt, (size_t)2 * H * dim))) return rc;
        rc = upload_matrix(p, p->gu[layer], 0, 2 * H, dim, fmt, host);
      } else {
        if ((rc = expect(p->fmt, (size_t)H * dim))) return rc;
        rc = upload_matrix(p, p->gu[layer], H, H, dim, fmt, host);
      }
      break;
    case GL3_FFN_DOWN:
      if ((rc = expect(p->fmt, (size_t)dim * H))) return rc;
      rc = upload_matrix(p, p->down[layer], 0, dim, H, fmt, host);
      break;
  }
  if (rc) return rc;
  if (is_layer_kind(kind)) p->uploaded[layer] |= 1u << kind;
  else p->uploaded_global |= 1u << kind;
  p->prepared = false;
  return GL3_OK;
}

extern "C" int gl3_set_rope_tables(gl3_plan *p, const float *cr, const float *ci, int ctx, int half) {
  if (!p || !cr || !ci) return fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  if (half != p->cfg.head_dim / 2 || ctx < p->cfg.context_length)
    return fail(GL3_ERR_INVALID_ARGUMENT, "rope tables [%d][%d] do not cover [%d][%d]", ctx, half,
                p->cfg.context_length, p->cfg.head_dim / 2);
  size_t n = (size_t)p->cfg.context_length * half;
  HIP_TRY(hipMemcpy((void *)p->m.rope_cos, cr, n * 4, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy((void *)p->m.rope_sin, ci, n * 4, hipMemcpyHostToDevice));
  p->rope_set = true;
  return GL3_OK;
}

// ------------------------------------------------------------- schedule

static int build_graph(gl3_plan *p) {
  const ModelDev &m = p->m;
  HIP_TRY(hipStreamBeginCapture(p->stream, hipStreamCaptureModeThreadLocal));
  hipError_t e = launch_embed(m, p->stream);
  for (int l = 0; l < m.n_layers && e == hipSuccess; ++l) {
    LayerDev L;
    L.qkv = p->qkv[l].view();
    L.wo = p->wo[l].view();
    L.gu = p->gu[l].view();
    L.down = p->down[l].view();
    if ((e = launch_gemv(m.fmt, MODE_STORE, L.qkv, m.q_dim + 2 * m.kv_dim, m.x, p->attn_norm[l], m.eps, m.qkv, nullptr,
                         0, p->stream)) != hipSuccess) break;
    if ((e = launch_attention(m, l, p->stream)) != hipSuccess) break;
    if ((e = launch_gemv(m.fmt, MODE_RESIDUAL, L.wo, m.dim, m.att, nullptr, m.eps, m.x, nullptr, 0, p->stream)) !=
        hipSuccess) break;
    if ((e = launch_gemv(m.fmt, MODE_SWIGLU, L.gu, m.hidden, m.x, p->ffn_norm[l], m.eps, m.hb, nullptr, 0,
                         p->stream)) != hipSuccess) break;
    if ((e = launch_gemv(m.fmt, MODE_RESIDUAL, L.down, m.dim, m.hb, nullptr, m.eps, m.x, nullptr, 0, p->stream)) !=
        hipSuccess) break;
  }
  if (e == hipSuccess) e = launch_logits(m, p->logits_grid, p->stream);
  if (e == hipSuccess) e = launch_advance(m, p->stream);
  hipGraph_t g = nullptr;
  hipError_t e2 = hipStreamEndCapture(p->stream, &g);
  if (e != hipSuccess || e2 != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return fail(GL3_ERR_DEVICE, "graph capture: %s", hipGetErrorString(e != hipSuccess ? e : e2));
  }
  p->graph = g;
  HIP_TRY(hipGraphInstantiate(&p->graph_exec, g, nullptr, nullptr, 0));
  return GL3_OK;
}

extern "C" int gl3_prepare(gl3_plan *p) {
  if (!p) return fail(GL3_ERR_INVALID_ARGUMENT, "null plan");
  if (p->prepared) return GL3_OK;
  const gl3_config &c = p->cfg;
  // every tensor the family's forward reads must be present
  uint32_t need_layer = (1u << GL3_ATTN_NORM) | (1u << GL3_ATTN_OUTPUT) | (1u << GL3_FFN_NORM) | (1u << GL3_FFN_UP) |
                        (1u << GL3_FFN_DOWN);
  if (p->family == FAM_PHI3) need_layer |= 1u << GL3_ATTN_QKV;
  else need_layer |= (1u << GL3_ATTN_Q) | (1u << GL3_ATTN_K) | (1u << GL3_ATTN_V) | (1u << GL3_FFN_GATE);
  if (p->family == FAM_QWEN3) need_layer |= (1u << GL3_ATTN_Q_NORM) | (1u << GL3_ATTN_K_NORM);
  for (int l = 0; l < c.n_layers; ++l)
    if ((p->uploaded[l] & need_layer) != need_layer)
      return fail(GL3_ERR_STATE, "layer %d: missing tensors (have mask 0x%x, need 0x%x)", l, p->uploaded[l], need_layer);
  if (!(p->uploaded_global & (1u << GL3_TOKEN_EMBD)) || !(p->uploaded_global & (1u << GL3_OUTPUT_NORM)))
    return fail(GL3_ERR_STATE, "token_embd and output_norm must be uploaded");
  if (p->cls_tied) {
    // no output.weight: the classifier shares token_embd (AbstractModelLoader.java:149)
    if (p->embd_fmt != ggml_to_fmt(c.weight_type))
      return fail(GL3_ERR_INVALID_ARGUMENT,
                  "no output.weight and token_embd type %d differs from the plan's weight type %d", p->embd_fmt,
                  c.weight_type);
    p->cls = p->embd;
    p->cls_fmt = p->embd_fmt;
  }
  if (!gemv_supported(p->cls_fmt, c.dim)) return fail(GL3_ERR_UNSUPPORTED, "classifier shape not supported");

  std::vector<LayerDev> ld(c.n_layers);
  for (int l = 0; l < c.n_layers; ++l) {
    ld[l].qkv = p->qkv[l].view();
    ld[l].wo = p->wo[l].view();
    ld[l].gu = p->gu[l].view();
    ld[l].down = p->down[l].view();
    ld[l].attn_norm = p->attn_norm[l];
    ld[l].ffn_norm = p->ffn_norm[l];
    ld[l].q_norm = p->q_norm[l];
    ld[l].k_norm = p->k_norm[l];
  }
  HIP_TRY(hipMemcpy(p->layers_d, ld.data(), sizeof(LayerDev) * ld.size(), hipMemcpyHostToDevice));
  ModelDev &m = p->m;
  m.embd = p->embd.view();
  m.embd_fmt = p->embd_fmt;
  m.cls = p->cls.view();
  m.cls_fmt = p->cls_fmt;

  // persistent kernel when the shape has one and the device co-schedules one workgroup per CU
  p->use_step_kernel = false;
  if (!(c.flags & GL3_FLAG_PHASE_KERNELS) && find_step_kernel(m, p->n_cu, &p->sk)) {
    int dev_coop = 0, max_lds = 0;
    HIP_TRY(hipDeviceGetAttribute(&dev_coop, hipDeviceAttributeCooperativeLaunch, p->device));
    HIP_TRY(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, p->device));
    hipFuncAttributes fa;
    HIP_TRY(hipFuncGetAttributes(&fa, p->sk.fn));
    int per_cu = 0;
    if (dev_coop && fa.sharedSizeBytes + p->sk.lds_bytes <= (size_t)max_lds) {
      HIP_TRY(hipFuncSetAttribute(p->sk.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)p->sk.lds_bytes));
      HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, p->sk.fn, GL3_STEP_BLOCK, p->sk.lds_bytes));
    }
    if (per_cu >= 1 && p->sk.ffn == 0) {
      p->use_step_kernel = true;
      p->step_grid = std::min(p->n_cu, p->sk.max_grid);
    } else if (per_cu >= 1 && p->sk.req_grid > 0 && p->sk.req_grid <= p->n_cu) {
      // fused FFN: a 32-column slice copy of every Wdown and the partials
      // buffer; the copies are remade on every prepare (an upload since the
      // last one may have replaced the weights)
      p->use_step_kernel = true;
      p->step_grid = p->sk.req_grid;
      int rc;
      if (!p->tdp && (rc = dev_alloc(p, &p->tdp, (size_t)p->step_grid * c.dim))) return rc;
      m.tdp = p->tdp;
      for (int l = 0; l < c.n_layers; ++l) {
        if (!p->down_sl[l].q && (rc = alloc_mat(p, p->down_sl[l], FMT_Q8, c.dim, p->hidden))) return rc;
        HIP_TRY(launch_slice_q8(p->down[l].q, p->down[l].s, c.dim, p->hidden, p->down_sl[l].q, p->down_sl[l].s,
                                p->stream));
        ld[l].down_sl = p->down_sl[l].view();
      }
      HIP_TRY(hipMemcpyAsync(p->layers_d, ld.data(), sizeof(LayerDev) * ld.size(), hipMemcpyHostToDevice, p->stream));
      HIP_TRY(zero_tagged(p));
      HIP_TRY(hipStreamSynchronize(p->stream));
    }
  }
  p->logits_grid = p->use_step_kernel ? p->step_grid : p->nbest;
  // the captured graph holds the device pointers of this preparation (the
  // classifier of a tied plan changes when output.weight is uploaded later):
  // capture it again on every prepare
  if (p->graph_exec) {
    HIP_TRY(hipGraphExecDestroy(p->graph_exec));
    p->graph_exec = nullptr;
  }
  if (p->graph) {
    HIP_TRY(hipGraphDestroy(p->graph));
    p->graph = nullptr;
  }
  if (!p->use_step_kernel) {
    int rc = build_graph(p);
    if (rc) return rc;
  }
  // the Q8_0 upload staging buffer is not needed after the weights are in place
  // (a later upload allocates it again)
  if (p->staging) {
    HIP_TRY(hipStreamSynchronize(p->stream));
    HIP_TRY(hipFree(p->staging));
    p->staging = nullptr;
    p->staging_bytes = 0;
  }
  p->prepared = true;
  return GL3_OK;
}

// ------------------------------------------------------------- forward

static void set_state(gl3_plan *p, int token, int pos) {
  DecodeState &s = *p->h_state;
  s.pos = pos;
  s.token = token;
  s.from_best = 0;
  s.parity = 0;
  s.step = 0;
  s.nbest = p->logits_grid;
  s.n_prompt = 0;
  s.pad = 0;
}

static hipEvent_t next_event(gl3_plan *p) {
  if (p->ev_used == (int)p->ev.size()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    p->ev.push_back(e);
  }
  return p->ev[p->ev_used++];
}

#define GL3_STEPS_PER_LAUNCH 256

// Uploads the control block and starts the call's timing.
static int begin_steps(gl3_plan *p) {
  p->ev_used = 0;
  p->last_launches = 0;
  HIP_TRY(hipMemcpyAsync(p->m.st, p->h_state, sizeof(DecodeState), hipMemcpyHostToDevice, p->stream));
  HIP_TRY(hipEventRecord(p->ev_begin, p->stream));
  return GL3_OK;
}

// n_steps decode steps from the device control block as it stands.
static int launch_steps(gl3_plan *p, int n_steps) {
  const bool timing = (p->cfg.flags & GL3_FLAG_TIMING) != 0;
  // persistent kernel: up to GL3_STEPS_PER_LAUNCH steps per launch (grid
  // barriers between steps); graph schedule: one replay per step
  for (int i = 0; i < n_steps;) {
    const int n = p->use_step_kernel ? std::min(n_steps - i, GL3_STEPS_PER_LAUNCH) : 1;
    hipEvent_t e0 = timing ? next_event(p) : nullptr;
    if (e0) HIP_TRY(hipEventRecord(e0, p->stream));
    if (p->use_step_kernel) {
      const unsigned ntags = (unsigned)n * (unsigned)p->sk.tags_per_step;
      if (p->tag + ntags < p->tag) {  // the tag counter would wrap: start again from clean cells
        HIP_TRY(zero_tagged(p));
        p->tag = 1;
      }
      HIP_TRY(launch_step_kernel(p->sk, p->m, p->gb, p->epoch, p->tag, p->step_grid, n, p->stream));
      p->epoch += (unsigned)(n - 1);
      p->tag += ntags;
    } else {
      HIP_TRY(hipGraphLaunch(p->graph_exec, p->stream));
    }
    hipEvent_t e1 = timing ? next_event(p) : nullptr;
    if (e1) HIP_TRY(hipEventRecord(e1, p->stream));
    ++p->last_launches;
    i += n;
  }
  return GL3_OK;
}

static int end_steps(gl3_plan *p) {
  HIP_TRY(hipEventRecord(p->ev_end, p->stream));
  return GL3_OK;
}

static int run_steps(gl3_plan *p, int n_steps) {
  int rc = begin_steps(p);
  if (!rc) rc = launch_steps(p, n_steps);
  if (!rc) rc = end_steps(p);
  return rc;
}

static int finish_timing_and_errors(gl3_plan *p) {
  HIP_TRY(hipMemcpyAsync(p->h_err, p->gb.err, 4, hipMemcpyDeviceToHost, p->stream));
  HIP_TRY(hipStreamSynchronize(p->stream));
  float ms = 0;
  HIP_TRY(hipEventElapsedTime(&ms, p->ev_begin, p->ev_end));
  p->last_elapsed_ms = ms;
  double ksum = 0;
  for (int i = 0; i + 1 < p->ev_used; i += 2) {
    float k = 0;
    HIP_TRY(hipEventElapsedTime(&k, p->ev[i], p->ev[i + 1]));
    ksum += k;
  }
  p->last_kernel_ms = ksum;
  if (*p->h_err) {
    // a barrier timed out: reset the barrier counters so the plan stays usable
    HIP_TRY(hipMemsetAsync(p->gb.ctr, 0, (GL3_BAR_GROUPS * GL3_BAR_STRIDE + 64) * 4, p->stream));
    HIP_TRY(hipMemsetAsync(p->m.att_ctr, 0, (size_t)p->cfg.n_layers * p->cfg.n_kv_heads * 4, p->stream));
    HIP_TRY(hipStreamSynchronize(p->stream));
    p->epoch = 0;
    return fail(GL3_ERR_DEVICE, "a grid barrier or a wait for a tagged vector timed out in the per-token kernel");
  }
  return GL3_OK;
}

extern "C" int gl3_forward(gl3_plan *p, int32_t token, int32_t position, float *logits_out, int32_t *argmax_out) {
  if (!p) return fail(GL3_ERR_INVALID_ARGUMENT, "null plan");
  if (token < 0 || token >= p->cfg.vocab_size)
    return fail(GL3_ERR_INVALID_ARGUMENT, "token %d out of range [0,%d)", token, p->cfg.vocab_size);
  if (position < 0 || position >= p->cfg.context_length)
    return fail(GL3_ERR_INVALID_ARGUMENT, "position %d out of range [0,%d)", position, p->cfg.context_length);
  int rc = gl3_prepare(p);
  if (rc) return rc;
  set_state(p, token, position);
  if ((rc = run_steps(p, 1))) return rc;
  if (logits_out)
    HIP_TRY(hipMemcpyAsync(logits_out, p->m.logits, (size_t)p->cfg.vocab_size * 4, hipMemcpyDeviceToHost, p->stream));
  HIP_TRY(hipMemcpyAsync(p->h_best, p->m.best, (size_t)p->logits_grid * 8, hipMemcpyDeviceToHost, p->stream));
  if ((rc = finish_timing_and_errors(p))) return rc;
  if (argmax_out) {
    unsigned long long b = 0;
    for (int i = 0; i < p->logits_grid; ++i) b = p->h_best[i] > b ? p->h_best[i] : b;
    *argmax_out = (int32_t)(0xFFFFFFFFu - (unsigned)(b & 0xFFFFFFFFu));
  }
  return GL3_OK;
}

extern "C" int gl3_generate_greedy(gl3_plan *p, int32_t token, int32_t position, int32_t n_steps, int32_t *tokens_out) {
  if (!p || !tokens_out) return fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  if (token < 0 || token >= p->cfg.vocab_size) return fail(GL3_ERR_INVALID_ARGUMENT, "token %d out of range", token);
  if (n_steps <= 0 || position < 0 || (int64_t)position + n_steps > p->cfg.context_length)
    return fail(GL3_ERR_INVALID_ARGUMENT, "positions [%d, %d) exceed context %d", position, position + n_steps,
                p->cfg.context_length);
  int rc = gl3_prepare(p);
  if (rc) return rc;
  set_state(p, token, position);
  if ((rc = run_steps(p, n_steps))) return rc;
  HIP_TRY(launch_finish(p->m, p->stream));
  HIP_TRY(hipMemcpyAsync(tokens_out, p->m.tokens_out, (size_t)n_steps * 4, hipMemcpyDeviceToHost, p->stream));
  return finish_timing_and_errors(p);
}

// ------------------------------------------------------------- prefill

#define GL3_PREFILL_ROWS 512  // prompt rows per block of the batched prefill

static bool use_prefill(const gl3_plan *p) {
  return !(p->cfg.flags & GL3_FLAG_STEPWISE_PROMPT) && prefill_supported(p->m);
}

// Forwards the n tokens at d_tokens (device) at positions pos0 .. pos0 + n - 1
// through every layer, GL3_PREFILL_ROWS rows at a time: fills their K and V and
// nothing else (the reference's prompt loop, whose logits are unused).
static int run_prefill(gl3_plan *p, const int *d_tokens, int n, int pos0) {
  const ModelDev &m = p->m;
  const int R = GL3_PREFILL_ROWS;
  int rc;
  if (!p->pf_x) {
    const size_t wa = (size_t)R * std::max(m.dim, m.q_dim), wb = (size_t)R * m.hidden;
    if ((rc = dev_alloc(p, &p->pf_x, (size_t)R * m.dim)) || (rc = dev_alloc(p, &p->pf_qkv, (size_t)R * (m.q_dim + 2 * m.kv_dim))) ||
        (rc = dev_alloc(p, &p->pf_ah, wa)) || (rc = dev_alloc(p, &p->pf_al, wa)) ||
        (rc = dev_alloc(p, &p->pf_bh, wb)) || (rc = dev_alloc(p, &p->pf_bl, wb)) ||
        (rc = dev_alloc(p, &p->pf_part, GL3_PREFILL_PART_FLOATS)))
      return rc;
  }
  hipStream_t s = p->stream;
  _Float16 *ah = p->pf_ah, *al = p->pf_al, *bh = p->pf_bh, *bl = p->pf_bl;
  for (int r0 = 0; r0 < n; r0 += R) {
    const int T = std::min(R, n - r0), p0 = pos0 + r0;
    HIP_TRY(launch_embed_rows(m, d_tokens + r0, T, p->pf_x, s));
    for (int l = 0; l < m.n_layers; ++l) {
      HIP_TRY(launch_rmsnorm_rows(p->pf_x, p->attn_norm[l], m.eps, m.dim, T, ah, al, s));
      HIP_TRY(launch_prefill_gemm(m.fmt, MODE_STORE, p->qkv[l].view(), m.q_dim + 2 * m.kv_dim, ah, al, T, p->pf_qkv,
                                  nullptr, nullptr, p->pf_part, s));
      HIP_TRY(launch_rope_kv_rows(m, l, p->pf_qkv, p0, T, s));
      HIP_TRY(launch_attn_rows(m, l, p->pf_qkv, p0, T, ah, al, s));
      HIP_TRY(launch_prefill_gemm(m.fmt, MODE_RESIDUAL, p->wo[l].view(), m.dim, ah, al, T, p->pf_x, nullptr, nullptr,
                                  p->pf_part, s));
      HIP_TRY(launch_rmsnorm_rows(p->pf_x, p->ffn_norm[l], m.eps, m.dim, T, ah, al, s));
      HIP_TRY(launch_prefill_gemm(m.fmt, MODE_SWIGLU, p->gu[l].view(), m.hidden, ah, al, T, nullptr, bh, bl, p->pf_part,
                                  s));
      HIP_TRY(launch_prefill_gemm(m.fmt, MODE_RESIDUAL, p->down[l].view(), m.dim, bh, bl, T, p->pf_x, nullptr, nullptr,
                                  p->pf_part, s));
    }
  }
  return GL3_OK;
}

// The prompt but its last token: batched prefill where the shape allows it,
// else decode steps; then the control block stands at the last prompt token
// (step n_prompt - 1), whose forward produces the first generated token.
static int run_prompt(gl3_plan *p, const int32_t *prompt, int n_prompt, int position) {
  int rc;
  if (n_prompt > 1 && use_prefill(p)) {
    set_state(p, prompt[n_prompt - 1], position + n_prompt - 1);
    p->h_state->step = n_prompt - 1;
    p->h_state->n_prompt = n_prompt;
    if ((rc = begin_steps(p))) return rc;
    return run_prefill(p, p->m.prompt, n_prompt - 1, position);
  }
  set_state(p, prompt[0], position);
  p->h_state->n_prompt = n_prompt;
  if ((rc = begin_steps(p))) return rc;
  return n_prompt > 1 ? launch_steps(p, n_prompt - 1) : GL3_OK;
}

extern "C" int gl3_prefill(gl3_plan *p, const int32_t *tokens, int32_t n, int32_t position) {
  if (!p || !tokens) return fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  if (n <= 0 || position < 0 || (int64_t)position + n > p->cfg.context_length)
    return fail(GL3_ERR_INVALID_ARGUMENT, "positions [%d, %lld) exceed context %d", position, (long long)position + n,
                p->cfg.context_length);
  for (int i = 0; i < n; ++i)
    if (tokens[i] < 0 || tokens[i] >= p->cfg.vocab_size)
      return fail(GL3_ERR_INVALID_ARGUMENT, "token %d (index %d) out of range", tokens[i], i);
  int rc = gl3_prepare(p);
  if (rc) return rc;
  if (!prefill_supported(p->m))
    return fail(GL3_ERR_UNSUPPORTED, "batched prefill needs head_dim 64, 96 or 128 (head_dim %d)", p->cfg.head_dim);
  HIP_TRY(hipMemcpyAsync((void *)p->m.prompt, tokens, (size_t)n * 4, hipMemcpyHostToDevice, p->stream));
  p->ev_used = 0;
  p->last_launches = 0;
  HIP_TRY(hipEventRecord(p->ev_begin, p->stream));
  if ((rc = run_prefill(p, p->m.prompt, n, position))) return rc;
  if ((rc = end_steps(p))) return rc;
  return finish_timing_and_errors(p);
}

extern "C" int gl3_generate_from_prompt(gl3_plan *p, const int32_t *prompt, int32_t n_prompt, int32_t position,
                                        int32_t n_gen, int32_t *tokens_out) {
  if (!p || !prompt || !tokens_out) return fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  if (n_prompt <= 0 || n_gen <= 0) return fail(GL3_ERR_INVALID_ARGUMENT, "n_prompt %d and n_gen %d must be positive", n_prompt, n_gen);
  const int64_t steps = (int64_t)n_prompt + n_gen - 1;
  if (position < 0 || (int64_t)position + steps > p->cfg.context_length)
    return fail(GL3_ERR_INVALID_ARGUMENT, "positions [%d, %lld) exceed context %d", position,
                (long long)(position + steps), p->cfg.context_length);
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= p->cfg.vocab_size)
      return fail(GL3_ERR_INVALID_ARGUMENT, "prompt token %d (index %d) out of range", prompt[i], i);
  int rc = gl3_prepare(p);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync((void *)p->m.prompt, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, p->stream));
  if ((rc = run_prompt(p, prompt, n_prompt, position))) return rc;
  if ((rc = launch_steps(p, n_gen))) return rc;
  if ((rc = end_steps(p))) return rc;
  HIP_TRY(launch_finish(p->m, p->stream));
  // the argmax after step s is recorded at tokens_out[s]; the generated ones follow the last prompt step
  HIP_TRY(hipMemcpyAsync(tokens_out, p->m.tokens_out + (n_prompt - 1), (size_t)n_gen * 4, hipMemcpyDeviceToHost,
                         p->stream));
  return finish_timing_and_errors(p);
}

extern "C" int gl3_generate_sampled(gl3_plan *p, const int32_t *prompt, int32_t n_prompt, int32_t position,
                                    int32_t n_gen, float temperature, float topp, const float *coins,
                                    int32_t *tokens_out) {
  if (!p || !prompt || !coins || !tokens_out) return fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  if (n_prompt <= 0 || n_gen <= 0) return fail(GL3_ERR_INVALID_ARGUMENT, "n_prompt %d and n_gen %d must be positive", n_prompt, n_gen);
  if (!(temperature >= 0.0f) || std::isinf(temperature) || std::isnan(topp))
    return fail(GL3_ERR_INVALID_ARGUMENT, "temperature %g / topp %g", (double)temperature, (double)topp);
  if (p->cfg.vocab_size < 2) return fail(GL3_ERR_INVALID_ARGUMENT, "sampling needs a vocabulary of two or more");
  const int64_t steps = (int64_t)n_prompt + n_gen - 1;
  if (position < 0 || (int64_t)position + steps > p->cfg.context_length)
    return fail(GL3_ERR_INVALID_ARGUMENT, "positions [%d, %lld) exceed context %d", position,
                (long long)(position + steps), p->cfg.context_length);
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= p->cfg.vocab_size)
      return fail(GL3_ERR_INVALID_ARGUMENT, "prompt token %d (index %d) out of range", prompt[i], i);
  for (int i = 0; i < n_gen; ++i)
    if (!(coins[i] >= 0.0f && coins[i] < 1.0f))
      return fail(GL3_ERR_INVALID_ARGUMENT, "draw %d = %g is not in [0, 1)", i, (double)coins[i]);
  // temperature 0 is the argmax (Sampler.TENSOR_ARGMAX, Sampler.java:76-78): the
  // greedy loop, whose steps run up to 256 to a launch with the argmax in the kernel
  if (temperature == 0.0f) return gl3_generate_from_prompt(p, prompt, n_prompt, position, n_gen, tokens_out);
  int rc = gl3_prepare(p);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync((void *)p->m.prompt, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, p->stream));
  HIP_TRY(hipMemcpyAsync(p->coins, coins, (size_t)n_gen * 4, hipMemcpyHostToDevice, p->stream));
  // the prompt tokens but the last: their logits are not used
  if ((rc = run_prompt(p, prompt, n_prompt, position))) return rc;
  // then one step per generated token, each followed by the sampler, which
  // makes the next step forward its token (no host round trip)
  for (int k = 0; k < n_gen; ++k) {
    if ((rc = launch_steps(p, 1))) return rc;
    HIP_TRY(launch_sample(p->m.logits, p->cfg.vocab_size, temperature, topp, p->coins, k, p->probs, nullptr, p->m.st,
                          p->m.tokens_out, p->m.best, p->stream));
  }
  if ((rc = end_steps(p))) return rc;
  HIP_TRY(hipMemcpyAsync(tokens_out, p->m.tokens_out, (size_t)n_gen * 4, hipMemcpyDeviceToHost, p->stream));
  return finish_timing_and_errors(p);
}

extern "C" int gl3_reset(gl3_plan *p) {
  if (!p) return fail(GL3_ERR_INVALID_ARGUMENT, "null plan");
  size_t kv = (size_t)p->cfg.n_layers * p->cfg.n_kv_heads * p->m.ctxp * p->cfg.head_dim * 2;
  HIP_TRY(hipMemsetAsync(p->m.kc, 0, kv, p->stream));
  HIP_TRY(hipMemsetAsync(p->m.vc, 0, kv, p->stream));
  HIP_TRY(hipStreamSynchronize(p->stream));
  return GL3_OK;
}

// KV cache: device K [L][n_kv][ctxp][hd] and V [L][n_kv][ctxp/16][hd][16]; host [npos][n_kv*hd]
static int kv_copy(gl3_plan *p, int layer, int pos0, int npos, uint16_t *host_k, uint16_t *host_v, bool to_device) {
  const gl3_config &c = p->cfg;
  if (layer < 0 || layer >= c.n_layers || pos0 < 0 || npos < 0 || (int64_t)pos0 + npos > c.context_length)
    return fail(GL3_ERR_INVALID_ARGUMENT, "kv range layer %d [%d,%d) outside the cache", layer, pos0, pos0 + npos);
  if (!host_k || !host_v) return fail(GL3_ERR_INVALID_ARGUMENT, "null buffer");
  if (npos == 0) return GL3_OK;
  // one contiguous host copy of each of K and V through a device staging area in
  // the host's row order, rearranged on the device (a strided copy per head into
  // pageable host memory is orders of magnitude slower)
  const int hd = c.head_dim, nkv = c.n_kv_heads, ctxp = p->m.ctxp;
  const size_t n = (size_t)npos * p->kv_dim;
  uint16_t *stage = nullptr;  // [2][npos][kv_dim]: K rows then V rows
  hipError_t he = hipMallocAsync((void **)&stage, 2 * n * 2, p->stream);
  if (he != hipSuccess) return fail(GL3_ERR_OUT_OF_MEMORY, "kv staging: %s", hipGetErrorString(he));
  uint16_t *kl = p->m.kc + (size_t)layer * nkv * ctxp * hd, *vl = p->m.vc + (size_t)layer * nkv * ctxp * hd;
  if (to_device) {
    he = hipMemcpyAsync(stage, host_k, n * 2, hipMemcpyHostToDevice, p->stream);
    if (he == hipSuccess) he = hipMemcpyAsync(stage + n, host_v, n * 2, hipMemcpyHostToDevice, p->stream);
    if (he == hipSuccess) he = launch_kv_rows(kl, vl, stage, stage + n, nkv, hd, ctxp, pos0, npos, true, p->stream);
  } else {
    he = launch_kv_rows(kl, vl, stage, stage + n, nkv, hd, ctxp, pos0, npos, false, p->stream);
    if (he == hipSuccess) he = hipMemcpyAsync(host_k, stage, n * 2, hipMemcpyDeviceToHost, p->stream);
    if (he == hipSuccess) he = hipMemcpyAsync(host_v, stage + n, n * 2, hipMemcpyDeviceToHost, p->stream);
  }
  int rc = GL3_OK;
  if (he == hipSuccess) he = hipStreamSynchronize(p->stream);  // host memory is borrowed for the call only
  if (he != hipSuccess) rc = fail(GL3_ERR_DEVICE, "kv copy: %s", hipGetErrorString(he));
  he = hipFreeAsync(stage, p->stream);
  if (he == hipSuccess) he = hipStreamSynchronize(p->stream);
  if (he != hipSuccess && rc == GL3_OK) rc = fail(GL3_ERR_DEVICE, "kv copy: %s", hipGetErrorString(he));
  return rc;
}

extern "C" int gl3_write_kv(gl3_plan *p, int layer, int pos0, int npos, const uint16_t *k, const uint16_t *v) {
  if (!p) return fail(GL3_ERR_INVALID_ARGUMENT, "null plan");
  return kv_copy(p, layer, pos0, npos, (uint16_t *)k, (uint16_t *)v, true);
}
extern "C" int gl3_read_kv(gl3_plan *p, int layer, int pos0, int npos, uint16_t *k, uint16_t *v) {
  if (!p) return fail(GL3_ERR_INVALID_ARGUMENT, "null plan");
  return kv_copy(p, layer, pos0, npos, k, v, false);
}

extern "C" int gl3_fill_kv_normal(gl3_plan *p, uint64_t seed, int npos) {
  if (!p) return fail(GL3_ERR_INVALID_ARGUMENT, "null plan");
  const gl3_config &c = p->cfg;
  if (npos < 0 || npos > c.context_length) return fail(GL3_ERR_INVALID_ARGUMENT, "npos %d", npos);
  if (npos == 0) return GL3_OK;
  const size_t hd = c.head_dim, ctxp = p->m.ctxp;
  for (int l = 0; l < c.n_layers; ++l)
    for (int h = 0; h < c.n_kv_heads; ++h) {
      const size_t head = (size_t)l * c.n_kv_heads + h;
      unsigned long long sk = seed ^ (0x100000001B3ull * (unsigned long long)(2 * head + 1));
      HIP_TRY(launch_fill_normal_f16(p->m.kc + head * ctxp * hd, 1, (size_t)npos * hd, 0, sk, p->stream));
      HIP_TRY(launch_fill_normal_vt(p->m.vc + head * hd * ctxp, (int)hd, npos, sk ^ 0xA5A5A5A5A5A5A5A5ull, p->stream));
    }
  HIP_TRY(hipStreamSynchronize(p->stream));
  return GL3_OK;
}

static int trace_stamps(gl3_plan *p, std::vector<unsigned long long> &t, int *n_stamps, int *n_blocks) {
  if (!p->m.tstamp) return fail(GL3_ERR_STATE, "plan was created without GL3_FLAG_PHASE_TRACE");
  if (!p->use_step_kernel) return fail(GL3_ERR_STATE, "the phase trace is recorded by the persistent per-token kernel only");
  *n_stamps = 3 + 10 * p->cfg.n_layers + 1;
  *n_blocks = p->step_grid;
  t.resize((size_t)*n_stamps * *n_blocks);
  HIP_TRY(hipMemcpy(t.data(), p->m.tstamp, t.size() * 8, hipMemcpyDeviceToHost));
  return GL3_OK;
}

extern "C" int gl3_get_phase_trace(gl3_plan *p, double *us_out, int32_t max_entries, int32_t *n_out) {
  if (!p || !us_out || !n_out) return fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  std::vector<unsigned long long> t;
  int n = 0, nb = 0;
  int rc = trace_stamps(p, t, &n, &nb);
  if (rc) return rc;
  int k = 0;
  for (int i = 1; i < n && k < max_entries; ++i)
    us_out[k++] = (double)(t[(size_t)i * nb] - t[(size_t)(i - 1) * nb]) * 0.01;  // 100 MHz ticks, workgroup 0
  *n_out = k;
  return GL3_OK;
}

extern "C" int gl3_get_phase_stamps(gl3_plan *p, uint64_t *out, int64_t max_entries, int32_t *n_stamps,
                                    int32_t *n_workgroups) {
  if (!p || !out || !n_stamps || !n_workgroups) return fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  std::vector<unsigned long long> t;
  int n = 0, nb = 0;
  int rc = trace_stamps(p, t, &n, &nb);
  if (rc) return rc;
  if ((int64_t)t.size() > max_entries) return fail(GL3_ERR_INVALID_ARGUMENT, "output holds %lld entries, %zu needed",
                                                   (long long)max_entries, t.size());
  for (size_t i = 0; i < t.size(); ++i) out[i] = t[i];
  *n_stamps = n;
  *n_workgroups = nb;
  return GL3_OK;
}

extern "C" int gl3_get_timing(gl3_plan *p, double *elapsed_ms, double *kernel_ms, int32_t *launches) {
  if (!p) return fail(GL3_ERR_INVALID_ARGUMENT, "null plan");
  if (elapsed_ms) *elapsed_ms = p->last_elapsed_ms;
  if (kernel_ms) *kernel_ms = p->last_kernel_ms;
  if (launches) *launches = p->last_launches;
  return GL3_OK;
}

extern "C" int gl3_time_attention(gl3_plan *p, int layer, int32_t position, int32_t n_reps, double *avg_ms) {
  if (!p || !avg_ms) return fail(GL3_ERR_INVALID_ARGUMENT, "null argument");
  if (layer < 0 || layer >= p->cfg.n_layers) return fail(GL3_ERR_INVALID_ARGUMENT, "layer %d out of range", layer);
  if (position < 0 || position >= p->cfg.context_length)
    return fail(GL3_ERR_INVALID_ARGUMENT, "position %d out of range [0,%d)", position, p->cfg.context_length);
  if (n_reps < 1 || n_reps > 100000) return fail(GL3_ERR_INVALID_ARGUMENT, "n_reps %d", n_reps);
  int rc = gl3_prepare(p);
  if (rc) return rc;
  set_state(p, 0, position);
  HIP_TRY(hipMemcpyAsync(p->m.st, p->h_state, sizeof(DecodeState), hipMemcpyHostToDevice, p->stream));
  HIP_TRY(launch_attention(p->m, layer, p->stream));  // warm-up
  p->ev_used = 0;
  for (int i = 0; i < n_reps; ++i) {
    hipEvent_t e0 = next_event(p), e1 = next_event(p);
    if (!e0 || !e1) return fail(GL3_ERR_DEVICE, "hipEventCreate failed");
    HIP_TRY(hipEventRecord(e0, p->stream));
    HIP_TRY(launch_attention(p->m, layer, p->stream));
    HIP_TRY(hipEventRecord(e1, p->stream));
  }
  HIP_TRY(hipStreamSynchronize(p->stream));
  double sum = 0;
  for (int i = 0; i + 1 < p->ev_used; i += 2) {
    float ms = 0;
    HIP_TRY(hipEventElapsedTime(&ms, p->ev[i], p->ev[i + 1]));
    sum += ms;
  }
  *avg_ms = sum / n_reps;
  return GL3_OK;
}

// ------------------------------------------------------------ op entry points

struct DevBuf {
  void *ptr = nullptr;
  ~DevBuf() {
    if (ptr) (void)hipFree(ptr);
  }
};

#define DEV_ALLOC(buf, bytes)                                                                 \
  do {                                                                                        \
    hipError_t e_ = hipMalloc(&(buf).ptr, (bytes) ? (bytes) : 16);                            \
    if (e_ != hipSuccess) {                                                                   \
      (void)hipGetLastError();                                                                \
      return fail(GL3_ERR_OUT_OF_MEMORY, "hipMalloc(%zu): %s", (size_t)(bytes), hipGetErrorString(e_)); \
    }                                                                                         \
  } while (0)

extern "C" int gl3_op_dequant_q8_0(const void *blocks, size_t n, float *out) {
  if (!blocks || !out || n % 32) return fail(GL3_ERR_INVALID_ARGUMENT, "n must be a multiple of 32");
  DevBuf raw, q, s, o;
  DEV_ALLOC(raw, n / 32 * 34);
  DEV_ALLOC(q, n);
  DEV_ALLOC(s, n / 32 * 2);
  DEV_ALLOC(o, n * 4);
  HIP_TRY(hipMemcpy(raw.ptr, blocks, n / 32 * 34, hipMemcpyHostToDevice));
  HIP_TRY(launch_repack_q8((const uint8_t *)raw.ptr, n / 32, (uint8_t *)q.ptr, (uint16_t *)s.ptr, nullptr));
  HIP_TRY(launch_dequant_q8((const uint8_t *)q.ptr, (const uint16_t *)s.ptr, n, (float *)o.ptr, nullptr));
  HIP_TRY(hipMemcpy(out, o.ptr, n * 4, hipMemcpyDeviceToHost));
  return GL3_OK;
}

extern "C" int gl3_op_f16_to_f32(const uint16_t *in, size_t n, float *out) {
  if (!in || !out) return fail(GL3_ERR_INVALID_ARGUMENT, "null buffer");
  DevBuf i, o;
  DEV_ALLOC(i, n * 2);
  DEV_ALLOC(o, n * 4);
  HIP_TRY(hipMemcpy(i.ptr, in, n * 2, hipMemcpyHostToDevice));
  HIP_TRY(launch_f16_to_f32((const uint16_t *)i.ptr, n, (float *)o.ptr, nullptr));
  HIP_TRY(hipMemcpy(out, o.ptr, n * 4, hipMemcpyDeviceToHost));
  return GL3_OK;
}

extern "C" int gl3_op_gemv(int ggml_type, const void *w, int rows, int cols, const float *x, const float *norm_w,
                           float eps, int mode, float *y) {
  const int fmt = ggml_to_fmt(ggml_type);
  if (!w || !x || !y || rows <= 0 || cols <= 0) return fail(GL3_ERR_INVALID_ARGUMENT, "bad gemv arguments");
  if ((fmt != FMT_Q8 && fmt != FMT_F16) || !gemv_supported(fmt, cols))
    return fail(GL3_ERR_UNSUPPORTED, "gemv type %d with %d columns is not supported", ggml_type, cols);
  if (mode < GL3_GEMV_STORE || mode > GL3_GEMV_SWIGLU || (mode == GL3_GEMV_SWIGLU && rows % 2))
    return fail(GL3_ERR_INVALID_ARGUMENT, "bad gemv mode %d for %d rows", mode, rows);
  const size_t n = (size_t)rows * cols;
  const int out_rows = mode == GL3_GEMV_SWIGLU ? rows / 2 : rows;
  DevBuf raw, q, s, dx, dn, dy;
  DEV_ALLOC(dx, (size_t)cols * 4);
  DEV_ALLOC(dy, (size_t)out_rows * 4);
  if (norm_w) DEV_ALLOC(dn, (size_t)cols * 4);
  if (fmt == FMT_Q8) {
    DEV_ALLOC(raw, n / 32 * 34);
    DEV_ALLOC(q, n);
    DEV_ALLOC(s, n / 32 * 2);
    HIP_TRY(hipMemcpy(raw.ptr, w, n / 32 * 34, hipMemcpyHostToDevice));
    HIP_TRY(launch_repack_q8((const uint8_t *)raw.ptr, n / 32, (uint8_t *)q.ptr, (uint16_t *)s.ptr, nullptr));
  } else {
    DEV_ALLOC(q, n * 2);
    HIP_TRY(hipMemcpy(q.ptr, w, n * 2, hipMemcpyHostToDevice));
  }
  HIP_TRY(hipMemcpy(dx.ptr, x, (size_t)cols * 4, hipMemcpyHostToDevice));
  if (norm_w) HIP_TRY(hipMemcpy(dn.ptr, norm_w, (size_t)cols * 4, hipMemcpyHostToDevice));
  if (mode == GL3_GEMV_RESIDUAL) HIP_TRY(hipMemcpy(dy.ptr, y, (size_t)out_rows * 4, hipMemcpyHostToDevice));
  Mat W{(const uint8_t *)q.ptr, (const uint16_t *)s.ptr, rows, cols};
  const int kmode = mode == GL3_GEMV_STORE ? MODE_STORE : mode == GL3_GEMV_RESIDUAL ? MODE_RESIDUAL : MODE_SWIGLU;
  HIP_TRY(launch_gemv(fmt, kmode, W, out_rows, (const float *)dx.ptr, norm_w ? (const float *)dn.ptr : nullptr, eps,
                      (float *)dy.ptr, nullptr, 0, nullptr));
  HIP_TRY(hipMemcpy(y, dy.ptr, (size_t)out_rows * 4, hipMemcpyDeviceToHost));
  return GL3_OK;
}

extern "C" int gl3_op_sample(const float *logits, int32_t n, float temperature, float topp, const float *coins,
                             int32_t n_draws, int32_t *tokens_out) {
  if (!logits || !coins || !tokens_out || n < 2 || n_draws <= 0)
    return fail(GL3_ERR_INVALID_ARGUMENT, "bad sample arguments (n %d, draws %d)", n, n_draws);
  if (!(temperature >= 0.0f) || std::isinf(temperature) || std::isnan(topp))
    return fail(GL3_ERR_INVALID_ARGUMENT, "temperature %g / topp %g", (double)temperature, (double)topp);
  for (int i = 0; i < n_draws; ++i)
    if (!(coins[i] >= 0.0f && coins[i] < 1.0f))
      return fail(GL3_ERR_INVALID_ARGUMENT, "draw %d = %g is not in [0, 1)", i, (double)coins[i]);
  DevBuf dl, dp, dc, dt;
  DEV_ALLOC(dl, (size_t)n * 4);
  DEV_ALLOC(dp, 2 * (size_t)n * 4);  // probabilities, then candidate indices
  DEV_ALLOC(dc, (size_t)n_draws * 4);
  DEV_ALLOC(dt, (size_t)n_draws * 4);
  HIP_TRY(hipMemcpy(dl.ptr, logits, (size_t)n * 4, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(dc.ptr, coins, (size_t)n_draws * 4, hipMemcpyHostToDevice));
  for (int k = 0; k < n_draws; ++k)
    HIP_TRY(launch_sample((const float *)dl.ptr, n, temperature, topp, (const float *)dc.ptr, k, (float *)dp.ptr,
                          nullptr, nullptr, (int *)dt.ptr, nullptr, nullptr));
  HIP_TRY(hipMemcpy(tokens_out, dt.ptr, (size_t)n_draws * 4, hipMemcpyDeviceToHost));
  return GL3_OK;
}

extern "C" int gl3_op_attention(const float *q, const uint16_t *kcache, const uint16_t *vcache, int n_heads,
                                int n_kv_heads, int head_dim, int pos, float *out) {
  if (!q || !kcache || !vcache || !out || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || pos < 0 ||
      head_dim <= 0)
    return fail(GL3_ERR_INVALID_ARGUMENT, "bad attention arguments");
  const int G = n_heads / n_kv_heads, hd = head_dim, ctx = pos + 1;
  if (!attention_supported(hd, G)) return fail(GL3_ERR_UNSUPPORTED, "head_dim %d / GQA group %d not supported", hd, G);
  const int q_dim = n_heads * hd, kv_dim = n_kv_heads * hd;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  int n_cu = 0;
  HIP_TRY(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
  ModelDev m{};
  m.family = FAM_LLAMA;
  m.n_layers = 1;
  m.n_heads = n_heads;
  m.n_kv = n_kv_heads;
  m.hd = hd;
  m.q_dim = q_dim;
  m.kv_dim = kv_dim;
  m.ctx = ctx;
  m.ctxp = (ctx + 15) / 16 * 16;
  m.sqrt_hd = (float)std::sqrt((double)hd);
  int ms = n_cu / n_kv_heads;
  m.max_split = ms < 1 ? 1 : (ms > 256 ? 256 : ms);
  DevBuf layers, kc, vc, qkv, att, part, ctr, st;
  DEV_ALLOC(layers, sizeof(LayerDev));
  DEV_ALLOC(kc, (size_t)n_kv_heads * m.ctxp * hd * 2);
  DEV_ALLOC(vc, (size_t)n_kv_heads * m.ctxp * hd * 2);
  DevBuf vstage;
  DEV_ALLOC(vstage, (size_t)ctx * hd * 2);
  DEV_ALLOC(qkv, (size_t)(q_dim + 2 * kv_dim) * 4);
  DEV_ALLOC(att, (size_t)q_dim * 4);
  DEV_ALLOC(part, (size_t)n_heads * m.max_split * (hd + 4) * 4);
  DEV_ALLOC(ctr, (size_t)n_kv_heads * 4);
  DEV_ALLOC(st, sizeof(DecodeState));
  LayerDev L{};
  HIP_TRY(hipMemcpy(layers.ptr, &L, sizeof L, hipMemcpyHostToDevice));
  // cache [pos+1][n_kv][hd] (host) -> K [n_kv][ctxp][hd], V [n_kv][ctxp/16][hd][16] (device)
  for (int h = 0; h < n_kv_heads; ++h) {
    HIP_TRY(hipMemcpy2D((uint16_t *)kc.ptr + (size_t)h * m.ctxp * hd, hd * 2, kcache + (size_t)h * hd,
                        (size_t)kv_dim * 2, hd * 2, ctx, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy2D(vstage.ptr, hd * 2, vcache + (size_t)h * hd, (size_t)kv_dim * 2, hd * 2, ctx,
                        hipMemcpyHostToDevice));
    HIP_TRY(launch_vt_copy((uint16_t *)vc.ptr + (size_t)h * hd * m.ctxp, (uint16_t *)vstage.ptr, hd, 0, ctx, true,
                           nullptr));
    HIP_TRY(hipDeviceSynchronize());
  }
  // qkv = [q, k(pos), v(pos)]: the kernel re-appends row pos of the cache unchanged
  std::vector<float> hq((size_t)q_dim + 2 * kv_dim);
  memcpy(hq.data(), q, (size_t)q_dim * 4);
  for (int i = 0; i < kv_dim; ++i) {
    uint16_t kb = kcache[(size_t)pos * kv_dim + i], vb = vcache[(size_t)pos * kv_dim + i];
    _Float16 kh, vh;
    memcpy(&kh, &kb, 2);
    memcpy(&vh, &vb, 2);
    hq[q_dim + i] = (float)kh;
    hq[q_dim + kv_dim + i] = (float)vh;
  }
  HIP_TRY(hipMemcpy(qkv.ptr, hq.data(), hq.size() * 4, hipMemcpyHostToDevice));
  HIP_TRY(hipMemset(ctr.ptr, 0, (size_t)n_kv_heads * 4));
  DecodeState hs{};
  hs.pos = pos;
  HIP_TRY(hipMemcpy(st.ptr, &hs, sizeof hs, hipMemcpyHostToDevice));
  m.layers = (const LayerDev *)layers.ptr;
  m.kc = (uint16_t *)kc.ptr;
  m.vc = (uint16_t *)vc.ptr;
  m.rope_cos = nullptr;  // q is already rotated: no RoPE tables, q and k used as given
  m.rope_sin = nullptr;
  m.qkv = (float *)qkv.ptr;
  m.att = (float *)att.ptr;
  m.part = (float *)part.ptr;
  m.att_ctr = (unsigned *)ctr.ptr;
  m.st = (DecodeState *)st.ptr;
  HIP_TRY(launch_attention(m, 0, nullptr));
  HIP_TRY(hipMemcpy(out, att.ptr, (size_t)q_dim * 4, hipMemcpyDeviceToHost));
  return GL3_OK;
}
