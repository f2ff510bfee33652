// Kernels of the decode path and their launch helpers.
//
//  * per-phase kernels: embed, GEMV (store / residual / SwiGLU / logits),
//    attention, step advance — one launch each, captured once per plan in a
//    hipGraph and replayed per token;
//  * decode_step_kernel<Shape>: the whole token in one cooperative launch, one
//    workgroup per CU, phases separated by fence-free grid barriers;
//  * op kernels for the op-level C-ABI entry points.
#include "gl3_internal.h"

namespace gl3 {

// ------------------------------------------------------------ GEMV tables
// Choice of (chunks per lane KC, K-split KS, rows per wave NR) for a GEMV of
// K columns.  n = K / (elements per 16-byte chunk * 64 lanes).

#define GL3_GEMV_LIST(X)                                      \
  X(FMT_Q8, 1, 1, 1) X(FMT_Q8, 2, 2, 1) X(FMT_Q8, 3, 3, 1)     \
  X(FMT_Q8, 4, 4, 1) X(FMT_Q8, 8, 4, 2) X(FMT_Q8, 14, 7, 2)    \
  X(FMT_F16, 2, 2, 1) X(FMT_F16, 4, 4, 1) X(FMT_F16, 6, 6, 1)  \
  X(FMT_F16, 8, 8, 1) X(FMT_F16, 16, 8, 2) X(FMT_F16, 28, 7, 4)

template <int KC, int NP>
struct DefaultNR {
  static constexpr int v = (8 / (KC * NP)) > 0 ? (8 / (KC * NP)) : 1;
};

template <class P>
__global__ __launch_bounds__(GL3_BLOCK) void gemv_kernel(Mat W, int out_rows, const float *x, const float *normw,
                                                         float eps, float *y, unsigned long long *best) {
  extern __shared__ float lds[];
  P::run(W, out_rows, x, normw, eps, y, best, blockIdx.x, gridDim.x, lds);
}

template <class P>
static hipError_t launch_gemv_t(const Mat &W, int out_rows, const float *x, const float *normw, float eps, float *y,
                                unsigned long long *best, int grid, hipStream_t s) {
  const int items = (out_rows + P::ROWS_PER_ITEM - 1) / P::ROWS_PER_ITEM;
  if (grid <= 0) grid = items < 2048 ? items : 2048;
  size_t lds = P::lds_bytes(W.cols);
  hipLaunchKernelGGL(gemv_kernel<P>, dim3(grid), dim3(GL3_BLOCK), lds, s, W, out_rows, x, normw, eps, y, best);
  return hipGetLastError();
}

int gemv_n(int fmt, int K) {
  const int per = (fmt == FMT_Q8 ? 16 : 8) * GL3_WAVE;
  return (K % per == 0) ? K / per : -1;
}

bool gemv_supported(int fmt, int K) {
  const int n = gemv_n(fmt, K);
#define GL3_SUP(F, N, KC, KS) if (fmt == F && n == N) return true;
  GL3_GEMV_LIST(GL3_SUP)
#undef GL3_SUP
  return false;
}

hipError_t launch_gemv(int fmt, int mode, const Mat &W, int out_rows, const float *x, const float *normw, float eps,
                       float *y, unsigned long long *best, int grid, hipStream_t s) {
  const int n = gemv_n(fmt, W.cols);
#define GL3_DISPATCH(F, N, KC, KS)                                                                                 \
  if (fmt == F && n == N) {                                                                                         \
    switch (mode) {                                                                                                 \
      case MODE_STORE:                                                                                              \
        return launch_gemv_t<GemvPhase<F, KC, KS, DefaultNR<KC, 1>::v, MODE_STORE>>(W, out_rows, x, normw, eps, y,  \
                                                                                    best, grid, s);                 \
      case MODE_RESIDUAL:                                                                                           \
        return launch_gemv_t<GemvPhase<F, KC, KS, DefaultNR<KC, 1>::v, MODE_RESIDUAL>>(W, out_rows, x, normw, eps, \
                                                                                       y, best, grid, s);           \
      case MODE_SWIGLU:                                                                                             \
        return launch_gemv_t<GemvPhase<F, KC, KS, DefaultNR<KC, 2>::v, MODE_SWIGLU>>(W, out_rows, x, normw, eps, y, \
                                                                                     best, grid, s);                \
      default:                                                                                                      \
        return launch_gemv_t<GemvPhase<F, KC, KS, DefaultNR<KC, 1>::v, MODE_LOGITS>>(W, out_rows, x, normw, eps, y, \
                                                                                     best, grid, s);                \
    }                                                                                                               \
  }
  GL3_GEMV_LIST(GL3_DISPATCH)
#undef GL3_DISPATCH
  return hipErrorInvalidValue;
}

template <class P>
__global__ __launch_bounds__(GL3_BLOCK) void logits_kernel(ModelDev m) {
  extern __shared__ float lds[];
  const int parity = ld_coherent_i32(&m.st->parity);
  const int nbest = ld_coherent_i32(&m.st->nbest);
  P::run(m.cls, m.vocab, m.x, m.out_norm, m.eps, m.logits, m.best + (size_t)parity * nbest, blockIdx.x, gridDim.x,
         lds);
}

hipError_t launch_logits(const ModelDev &m, int grid, hipStream_t s) {
  const int n = gemv_n(m.cls_fmt, m.dim);
#define GL3_LOGITS(F, N, KC, KS)                                                                     \
  if (m.cls_fmt == F && n == N) {                                                                    \
    typedef GemvPhase<F, KC, KS, DefaultNR<KC, 1>::v, MODE_LOGITS> P;                                \
    hipLaunchKernelGGL(logits_kernel<P>, dim3(grid), dim3(GL3_BLOCK), P::lds_bytes(m.dim), s, m);    \
    return hipGetLastError();                                                                        \
  }
  GL3_GEMV_LIST(GL3_LOGITS)
#undef GL3_LOGITS
  return hipErrorInvalidValue;
}

// ------------------------------------------------------ per-phase kernels

__global__ __launch_bounds__(GL3_BLOCK) void embed_kernel(ModelDev m) {
  __shared__ int si_lds[8];
  StepInfo si = read_step(m, si_lds);
  phase_embed(m, si.token, blockIdx.x, gridDim.x);
}

__global__ __launch_bounds__(GL3_BLOCK) void attention_kernel(ModelDev m, int layer) {
  extern __shared__ float lds[];
  __shared__ int si_lds[8];
  StepInfo si = read_step(m, si_lds);
  phase_attention(m, layer, si.pos, blockIdx.x, gridDim.x, lds);
}

// Last kernel of a step: records the previous token and advances the control block.
__global__ __launch_bounds__(GL3_BLOCK) void advance_kernel(ModelDev m) {
  __shared__ int si_lds[8];
  StepInfo si = read_step(m, si_lds);
  advance_step(m, si);
}

// Records the argmax of the last step of a generate call.
__global__ __launch_bounds__(GL3_BLOCK) void finish_kernel(ModelDev m) {
  __shared__ int si_lds[8];
  StepInfo si = read_step(m, si_lds);
  if (threadIdx.x == 0 && si.from_best && si.step > 0) m.tokens_out[si.step - 1] = si.token;
}

size_t attention_lds_bytes(int hd, int G) {
  return ((size_t)G * hd + 2 * hd + ATT_TILE * (hd + 1) + ATT_TILE * hd + G * ATT_TILE + 3 * ATT_MAX_G + 16 + 8 + 16) *
         sizeof(float);
}

hipError_t launch_embed(const ModelDev &m, hipStream_t s) {
  int grid = (m.dim + GL3_BLOCK - 1) / GL3_BLOCK;
  hipLaunchKernelGGL(embed_kernel, dim3(grid), dim3(GL3_BLOCK), 0, s, m);
  return hipGetLastError();
}
hipError_t launch_attention(const ModelDev &m, int layer, hipStream_t s) {
  const int grid = m.n_kv * m.max_split;
  hipLaunchKernelGGL(attention_kernel, dim3(grid), dim3(GL3_BLOCK), attention_lds_bytes(m.hd, m.n_heads / m.n_kv), s,
                     m, layer);
  return hipGetLastError();
}
hipError_t launch_advance(const ModelDev &m, hipStream_t s) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(GL3_BLOCK), 0, s, m);
  return hipGetLastError();
}
hipError_t launch_finish(const ModelDev &m, hipStream_t s) {
  hipLaunchKernelGGL(finish_kernel, dim3(1), dim3(GL3_BLOCK), 0, s, m);
  return hipGetLastError();
}

// --------------------------------------------------- persistent step kernel

// Compile-time GEMV shapes of the model families the persistent kernel is
// built for.  NR is chosen so that every phase has >= 256 work items.
template <int FMT, int CLSF, int DIM, int QD, int KVD, int HID, int NRQKV, int NRWO, int NRGU, int NRDN, int NRCLS>
struct Shape {
  static constexpr int fmt = FMT, cls_fmt = CLSF, dim = DIM, q_dim = QD, kv_dim = KVD, hidden = HID;
  static constexpr int EPC = FMT == FMT_Q8 ? 16 : 8;
  static constexpr int CEPC = CLSF == FMT_Q8 ? 16 : 8;
  static constexpr int nd = DIM / (EPC * 64), nq = QD / (EPC * 64), nh = HID / (EPC * 64), nc = DIM / (CEPC * 64);
  // split K so that a lane holds at most 64 (Q8: 7*16=112 for n=14) x values
  static constexpr int ks(int n, int kcmax) { return n <= kcmax ? 1 : (n / 2 <= kcmax ? 2 : 4); }
  static constexpr int KCMAX = FMT == FMT_Q8 ? 7 : 8;
  static constexpr int CKCMAX = CLSF == FMT_Q8 ? 7 : 8;
  typedef GemvPhase<FMT, nd / ks(nd, KCMAX), ks(nd, KCMAX), NRQKV, MODE_STORE> QKV;
  typedef GemvPhase<FMT, nq / ks(nq, KCMAX), ks(nq, KCMAX), NRWO, MODE_RESIDUAL> WO;
  typedef GemvPhase<FMT, nd / ks(nd, KCMAX), ks(nd, KCMAX), NRGU, MODE_SWIGLU> GU;
  typedef GemvPhase<FMT, nh / ks(nh, KCMAX), ks(nh, KCMAX), NRDN, MODE_RESIDUAL> DOWN;
  typedef GemvPhase<CLSF, nc / ks(nc, CKCMAX), ks(nc, CKCMAX), NRCLS, MODE_LOGITS> CLS;
};

// Llama-3.2-1B (Q8_0 and F16), Qwen3-0.6B (Q8_0), Phi-3-mini (F16), Llama-3.1-8B (Q8_0)
typedef Shape<FMT_Q8, FMT_Q8, 2048, 2048, 512, 8192, 3, 2, 4, 2, 4> ShapeLlama1BQ8;
typedef Shape<FMT_F16, FMT_F16, 2048, 2048, 512, 8192, 2, 2, 2, 2, 2> ShapeLlama1BF16;
typedef Shape<FMT_Q8, FMT_Q8, 1024, 2048, 1024, 3072, 4, 1, 3, 1, 4> ShapeQwen3_06BQ8;
typedef Shape<FMT_F16, FMT_F16, 3072, 3072, 3072, 8192, 2, 2, 1, 2, 2> ShapePhi3MiniF16;
typedef Shape<FMT_Q8, FMT_Q8, 4096, 4096, 1024, 14336, 2, 2, 1, 1, 2> ShapeLlama8BQ8;

template <class SH>
__global__ __launch_bounds__(GL3_BLOCK, 1) void decode_step_kernel(ModelDev m, GridBarrier gb, unsigned epoch) {
  extern __shared__ float lds[];
  __shared__ int si_lds[8];
  const int blk = blockIdx.x, nblk = gridDim.x;
  StepInfo si = read_step(m, si_lds);
  phase_embed(m, si.token, blk, nblk);
  if (!grid_barrier(gb, ++epoch)) return;
  if (blk == 0) advance_step(m, si);
  const int rows_qkv = SH::q_dim + 2 * SH::kv_dim;
  for (int l = 0; l < m.n_layers; ++l) {
    const LayerDev &L = m.layers[l];
    SH::QKV::run(L.qkv, rows_qkv, m.x, L.attn_norm, m.eps, m.qkv, nullptr, blk, nblk, lds);
    if (!grid_barrier(gb, ++epoch)) return;
    phase_attention(m, l, si.pos, blk, nblk, lds);
    if (!grid_barrier(gb, ++epoch)) return;
    SH::WO::run(L.wo, SH::dim, m.att, nullptr, m.eps, m.x, nullptr, blk, nblk, lds);
    if (!grid_barrier(gb, ++epoch)) return;
    SH::GU::run(L.gu, SH::hidden, m.x, L.ffn_norm, m.eps, m.hb, nullptr, blk, nblk, lds);
    if (!grid_barrier(gb, ++epoch)) return;
    SH::DOWN::run(L.down, SH::dim, m.hb, nullptr, m.eps, m.x, nullptr, blk, nblk, lds);
    if (!grid_barrier(gb, ++epoch)) return;
  }
  SH::CLS::run(m.cls, m.vocab, m.x, m.out_norm, m.eps, m.logits, m.best + (size_t)si.parity * si.nbest, blk, nblk,
               lds);
}

template <class SH>
static bool shape_matches(const ModelDev &m) {
  return m.fmt == SH::fmt && m.cls_fmt == SH::cls_fmt && m.dim == SH::dim && m.q_dim == SH::q_dim &&
         m.kv_dim == SH::kv_dim && m.hidden == SH::hidden;
}

template <class SH>
static size_t step_lds_bytes(const ModelDev &m) {
  size_t b = attention_lds_bytes(m.hd, m.n_heads / m.n_kv);
  size_t g[5] = {SH::QKV::lds_bytes(SH::dim), SH::WO::lds_bytes(SH::q_dim), SH::GU::lds_bytes(SH::dim),
                 SH::DOWN::lds_bytes(SH::hidden), SH::CLS::lds_bytes(SH::dim)};
  for (size_t v : g) b = v > b ? v : b;
  return b;
}

template <class SH>
static StepKernel make_step_kernel(const ModelDev &m) {
  StepKernel k;
  k.fn = (const void *)decode_step_kernel<SH>;
  k.lds_bytes = step_lds_bytes<SH>(m);
  k.barriers_per_step = 1 + 5 * m.n_layers;
  return k;
}

bool find_step_kernel(const ModelDev &m, StepKernel *out) {
  if (shape_matches<ShapeLlama1BQ8>(m)) { *out = make_step_kernel<ShapeLlama1BQ8>(m); return true; }
  if (shape_matches<ShapeLlama1BF16>(m)) { *out = make_step_kernel<ShapeLlama1BF16>(m); return true; }
  if (shape_matches<ShapeQwen3_06BQ8>(m)) { *out = make_step_kernel<ShapeQwen3_06BQ8>(m); return true; }
  if (shape_matches<ShapePhi3MiniF16>(m)) { *out = make_step_kernel<ShapePhi3MiniF16>(m); return true; }
  if (shape_matches<ShapeLlama8BQ8>(m)) { *out = make_step_kernel<ShapeLlama8BQ8>(m); return true; }
  return false;
}

hipError_t launch_step_kernel(const StepKernel &k, const ModelDev &m, const GridBarrier &gb, unsigned epoch, int grid,
                              hipStream_t s) {
  ModelDev mm = m;
  GridBarrier gg = gb;
  unsigned e = epoch;
  void *args[] = {&mm, &gg, &e};
  return hipLaunchCooperativeKernel(k.fn, dim3(grid), dim3(GL3_BLOCK), args, (unsigned)k.lds_bytes, s);
}

// -------------------------------------------------------------- op kernels

__global__ void dequant_q8_kernel(const uint8_t *q, const uint16_t *s, size_t n, float *out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = (float)(int8_t)q[i] * h2f(s[i / 32]);
}
__global__ void f16_to_f32_kernel(const uint16_t *in, size_t n, float *out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = h2f(in[i]);
}
// GGUF Q8_0 blocks {fp16 scale, int8 q[32]} -> int8 quants + fp16 scales (structure of arrays)
__global__ void repack_q8_kernel(const uint8_t *blocks, size_t nblocks, uint8_t *q, uint16_t *s) {
  for (size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks; b += (size_t)gridDim.x * blockDim.x) {
    const uint8_t *src = blocks + b * 34;
    s[b] = (uint16_t)(src[0] | (src[1] << 8));
#pragma unroll
    for (int i = 0; i < 32; ++i) q[b * 32 + i] = src[2 + i];
  }
}
// counter-based N(0,1) -> fp16 (Box-Muller on two 24-bit uniforms of a splitmix64 hash)
__device__ __forceinline__ unsigned long long splitmix64(unsigned long long z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__global__ void fill_normal_f16_kernel(uint16_t *dst, size_t n, unsigned long long seed) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    unsigned long long h = splitmix64(seed ^ splitmix64(i));
    float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    float u2 = (float)((h >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);
    float r = sqrtf(-2.0f * logf(u1));
    dst[i] = f2h(r * cospif(2.0f * u2));
  }
}

hipError_t launch_repack_q8(const uint8_t *blocks, size_t nblocks, uint8_t *q, uint16_t *s, hipStream_t st) {
  size_t grid = (nblocks + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (grid == 0) grid = 1;
  hipLaunchKernelGGL(repack_q8_kernel, dim3((unsigned)grid), dim3(256), 0, st, blocks, nblocks, q, s);
  return hipGetLastError();
}
hipError_t launch_dequant_q8(const uint8_t *q, const uint16_t *s, size_t n, float *out, hipStream_t st) {
  size_t grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (grid == 0) grid = 1;
  hipLaunchKernelGGL(dequant_q8_kernel, dim3((unsigned)grid), dim3(256), 0, st, q, s, n, out);
  return hipGetLastError();
}
hipError_t launch_f16_to_f32(const uint16_t *in, size_t n, float *out, hipStream_t st) {
  size_t grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (grid == 0) grid = 1;
  hipLaunchKernelGGL(f16_to_f32_kernel, dim3((unsigned)grid), dim3(256), 0, st, in, n, out);
  return hipGetLastError();
}
hipError_t launch_fill_normal_f16(uint16_t *dst, size_t n, unsigned long long seed, hipStream_t st) {
  size_t grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (grid == 0) grid = 1;
  hipLaunchKernelGGL(fill_normal_f16_kernel, dim3((unsigned)grid), dim3(256), 0, st, dst, n, seed);
  return hipGetLastError();
}

}  // namespace gl3
