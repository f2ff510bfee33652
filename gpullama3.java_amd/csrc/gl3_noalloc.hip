// gl3_op_attention_noalloc: decode attention over device-resident buffers that
// allocates nothing.  The kernels' scratch (split partials, split-merge
// counters, the step control block and an empty layer descriptor) lives in a
// file-scope device array of fixed size, one copy per GPU, resolved once per
// device with hipGetSymbolAddress.  For callers that cannot allocate device
// memory: code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc.  Calls that overlap on one GPU share its array and race.
#include <cmath>
#include <mutex>

#include "../../include/gl3.h"
#include "gl3_host.h"
#include "gl3_internal.h"

using namespace gl3;

namespace {

// Layout: [0, 256) DecodeState; [256, 512) LayerDev (all zero); [512, 768)
// split-merge counters (one per kv head, <= 64); [1024, ...) partials
// [n_heads][max_split][head_dim + 4] floats.
constexpr size_t kScratchBytes = GL3_NOALLOC_SCRATCH_BYTES;
constexpr size_t kOffState = 0, kOffLayer = 256, kOffCtr = 512, kOffPart = 1024;
constexpr int kMaxKvHeads = 64;
constexpr int kMaxDevices = 64;
static_assert(sizeof(DecodeState) <= kOffLayer - kOffState, "control block");
static_assert(sizeof(LayerDev) <= kOffCtr - kOffLayer, "layer descriptor");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void *g_scratch[kMaxDevices];  // device address of `scratch` per device (nullptr: not resolved yet)
int g_n_cu[kMaxDevices];

// Zeroes the control block, the layer descriptor and the counters (the first
// 1024 bytes) and sets the position.  A kernel, not hipMemsetAsync: callers may
// capture this entry point in a graph.
__global__ void noalloc_init_kernel(unsigned *scr, int pos) {
  const int t = threadIdx.x;
  if (t < 256) scr[t] = t == 0 ? (unsigned)pos : 0u;
}

// The scratch address and CU count of the current device, resolved on its first call.
int device_scratch(unsigned char **out, int *n_cu) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return host_fail(GL3_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return host_fail(GL3_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return host_fail(GL3_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    int cu = 0;
    e = hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || cu <= 0) return host_fail(GL3_ERR_DEVICE, "CU count: %s", hipGetErrorString(e));
    g_n_cu[dev] = cu;
    g_scratch[dev] = p;
  }
  *out = (unsigned char *)g_scratch[dev];
  *n_cu = g_n_cu[dev];
  return GL3_OK;
}

}  // namespace

extern "C" int gl3_op_attention_noalloc(const float *qkv, uint16_t *kcache, uint16_t *vcache, int n_heads,
                                        int n_kv_heads, int head_dim, int ctxp, int pos, float *out, void *stream) {
  if (!qkv || !kcache || !vcache || !out)
    return host_fail(GL3_ERR_INVALID_ARGUMENT, "null buffer");
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim <= 0)
    return host_fail(GL3_ERR_INVALID_ARGUMENT, "bad head counts %d / %d or head_dim %d", n_heads, n_kv_heads,
                     head_dim);
  if (ctxp <= 0 || ctxp % 16 || pos < 0 || pos >= ctxp)
    return host_fail(GL3_ERR_INVALID_ARGUMENT, "ctxp %d must be a positive multiple of 16 above pos %d", ctxp, pos);
  const int G = n_heads / n_kv_heads, hd = head_dim;
  if (!attention_supported(hd, G))
    return host_fail(GL3_ERR_UNSUPPORTED, "head_dim %d / GQA group %d not supported", hd, G);
  if (n_kv_heads > kMaxKvHeads)
    return host_fail(GL3_ERR_INVALID_ARGUMENT, "%d kv heads exceed the scratch's %d counters", n_kv_heads,
                     kMaxKvHeads);
  unsigned char *scr = nullptr;
  int n_cu = 0;
  int rc = device_scratch(&scr, &n_cu);
  if (rc) return rc;
  ModelDev m{};
  m.family = FAM_LLAMA;
  m.n_layers = 1;
  m.n_heads = n_heads;
  m.n_kv = n_kv_heads;
  m.hd = hd;
  m.q_dim = n_heads * hd;
  m.kv_dim = n_kv_heads * hd;
  m.ctx = ctxp;
  m.ctxp = ctxp;
  m.sqrt_hd = (float)std::sqrt((double)hd);  // (float) Math.sqrt(headSize), InferenceCore.java:64
  const int ms = n_cu / n_kv_heads;           // the split count of gl3_op_attention
  m.max_split = ms < 1 ? 1 : (ms > 256 ? 256 : ms);
  const size_t need = kOffPart + (size_t)n_heads * m.max_split * (hd + 4) * sizeof(float);
  if (need > kScratchBytes)
    return host_fail(GL3_ERR_INVALID_ARGUMENT, "%d heads x %d splits x head_dim %d need %zu bytes of scratch, above "
                     "the %zu of this entry point", n_heads, m.max_split, hd, need, kScratchBytes);
  m.st = (DecodeState *)(scr + kOffState);
  m.layers = (const LayerDev *)(scr + kOffLayer);
  m.att_ctr = (unsigned *)(scr + kOffCtr);
  m.part = (float *)(scr + kOffPart);
  m.kc = kcache;
  m.vc = vcache;
  m.qkv = (float *)qkv;  // read only: q, then the new k and v (appended to the cache at pos)
  m.att = out;
  m.rope_cos = nullptr;  // q and k as given
  m.rope_sin = nullptr;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(noalloc_init_kernel, dim3(1), dim3(256), 0, s, (unsigned *)scr, pos);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = launch_attention(m, 0, s);
  if (e != hipSuccess) return host_fail(GL3_ERR_DEVICE, "attention launch: %s", hipGetErrorString(e));
  return GL3_OK;
}
