// Batched prefill: a block of prompt tokens through every layer at once.
//
// The reference ingests a prompt one token per forward, the logits of all but
// the last token unused (InferenceEngine.java:88-131 for Llama / Phi-3,
// :162-187 for Qwen3).  What a prompt token leaves behind is its K and V in
// every layer; a block of rows computes the same function of the same weights:
// per layer RMSNorm of every row, the QKV, Wo, gate/up and down projections as
// matrix products on the matrix cores, Qwen3's per-head QK-norm and RoPE with
// the KV append for every position, and causal attention of every row over the
// cache.  The last prompt token is forwarded by the decode step, which also
// produces its logits.
//
// Activations that feed a matrix product are kept as two fp16 planes, hi =
// fp16(x) and lo = fp16(x - hi) (~22 significant bits of x, |x| < 65504), and
// both are multiplied: v_mfma_f32_16x16x32_f16, fp32 accumulation.  Q8_0
// weights enter as their int8 quants (exact in fp16), one MFMA pair per
// 32-column block, and the block's scale multiplies the pair's fp32 result;
// FP16 weights enter as they are.
#include "gl3_internal.h"

namespace gl3 {

typedef _Float16 ph8 __attribute__((ext_vector_type(8)));
typedef float pf4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int PBS = 256;  // threads per workgroup

__device__ __forceinline__ void put_split(_Float16 *hi, _Float16 *lo, size_t i, float x) {
  const _Float16 h = (_Float16)x;
  hi[i] = h;
  lo[i] = (_Float16)(x - (float)h);
}

// 8 int8 quants (two dwords) as exact fp16 values
__device__ __forceinline__ ph8 q8_to_h8(unsigned w0, unsigned w1) {
  ph8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = (_Float16)(float)(signed char)((w0 >> (8 * i)) & 0xffu);
    r[4 + i] = (_Float16)(float)(signed char)((w1 >> (8 * i)) & 0xffu);
  }
  return r;
}

}  // namespace

// Y[T][N] = X[T][K] . W[N][K]^T.  One wave computes a 16 (rows of X) x 64
// (rows of W) tile as four 16 x 16 MFMA tiles; the four waves of a workgroup
// take four consecutive 16-row groups of X over the same 64 rows of W (the
// weights come through L1 once per workgroup).  MFMA operands: lane (hh, kb)
// holds row hh of the A tile (a row of X) and column hh of the B tile (a row
// of W), elements 8 kb .. 8 kb + 7 of the 32-column step; the result lane holds
// rows 4 kb .. 4 kb + 3 of column hh.
// MODE_STORE: Y = fp32; MODE_RESIDUAL: Y += fp32; MODE_SWIGLU: W holds gate
// rows then up rows ([2N][K]) and the output is silu(gate) * up as hi / lo
// fp16 planes Yh, Yl.
template <int FMT, int MODE>
__global__ __launch_bounds__(PBS) void gemm_kernel(const uint8_t *wq, const uint16_t *ws, int N, int K,
                                                   const _Float16 *Xh, const _Float16 *Xl, int T, float *Y,
                                                   _Float16 *Yh, _Float16 *Yl) {
  constexpr int NP = MODE == MODE_SWIGLU ? 2 : 1;
  const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
  const int hh = lane % 16, kb = lane / 16;
  const int n0 = blockIdx.x * 64, t0 = blockIdx.y * 64 + wave * 16;
  if (t0 >= T) return;  // no row of this wave is in the block (nothing below synchronizes)
  const size_t trow = (size_t)min(t0 + hh, T - 1);  // rows past T repeat the last; their results are dropped
  const _Float16 *xh = Xh + trow * K + 8 * kb, *xl = Xl + trow * K + 8 * kb;
  size_t wrow[NP][4];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int j = 0; j < 4; ++j) wrow[p][j] = (size_t)min(n0 + 16 * j + hh, N - 1) + (size_t)p * N;
  pf4 acc[NP][4];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[p][j] = pf4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < K; k0 += 32) {
    const ph8 ahi = *(const ph8 *)(xh + k0), alo = *(const ph8 *)(xl + k0);
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const size_t n = wrow[p][j];
        if (FMT == FMT_Q8) {
          const uint2 w = *(const uint2 *)(wq + n * K + k0 + 8 * kb);
          const ph8 b = q8_to_h8(w.x, w.y);
          pf4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, pf4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
          tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, tmp, 0, 0, 0);
          const float sc = h2f(ws[n * (K / 32) + k0 / 32]);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[p][j][v] = fmaf(tmp[v], sc, acc[p][j][v]);
        } else {
          const ph8 b = *(const ph8 *)(wq + (n * K + k0 + 8 * kb) * 2);
          acc[p][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, acc[p][j], 0, 0, 0);
          acc[p][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, acc[p][j], 0, 0, 0);
        }
      }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int t = t0 + 4 * kb + v, n = n0 + 16 * j + hh;
      if (t >= T || n >= N) continue;
      const size_t i = (size_t)t * N + n;
      if (MODE == MODE_STORE)
        Y[i] = acc[0][j][v];
      else if (MODE == MODE_RESIDUAL)
        Y[i] += acc[0][j][v];
      else
        put_split(Yh, Yl, i, silu_ref(acc[0][j][v]) * acc[NP - 1][j][v]);  // InferenceCore.java:162-166
    }
}

// Residual-stream rows of the block: the embedding rows of its tokens (InferenceCore.java:68)
__global__ __launch_bounds__(PBS) void embed_rows_kernel(ModelDev m, const int *tokens, int T, float *X) {
  const int t = blockIdx.x;
  if (t >= T) return;
  const size_t row = (size_t)tokens[t] * m.dim;
  for (int i = threadIdx.x; i < m.dim; i += PBS) {
    const size_t e = row + i;
    float v;
    if (m.embd_fmt == FMT_F32)
      v = ((const float *)m.embd.q)[e];
    else if (m.embd_fmt == FMT_Q8)
      v = (float)(int8_t)m.embd.q[e] * h2f(m.embd.s[e / 32]);
    else
      v = h2f(((const uint16_t *)m.embd.q)[e]);
    X[(size_t)t * m.dim + i] = v;
  }
}

// RMSNorm of every row (InferenceCore.java:46-55: mean of squares in fp32, plus
// eps, 1/sqrt in double), written as hi / lo planes.  One workgroup per row.
__global__ __launch_bounds__(PBS) void rmsnorm_rows_kernel(const float *X, const float *w, float eps, int dim, int T,
                                                            _Float16 *Yh, _Float16 *Yl) {
  __shared__ float red[PBS / GL3_WAVE];
  const int t = blockIdx.x;
  if (t >= T) return;
  const float *x = X + (size_t)t * dim;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < dim; i += PBS) ss += x[i] * x[i];
  ss = block_sum<PBS>(ss, red);
  ss /= (float)dim;
  ss += eps;
  ss = (float)(1.0 / sqrt((double)ss));
  for (int i = threadIdx.x; i < dim; i += PBS) put_split(Yh, Yl, (size_t)t * dim + i, w[i] * (ss * x[i]));
}

// Per-head work of every row, one wave per (row, head) with the q heads first:
// Qwen3's per-head RMSNorm of q and k (InferenceCore.java:341-347), RoPE
// (:82-100, interleaved pairs, Llama; :472-491, NeoX halves, Qwen3 / Phi-3) in
// place in the QKV rows, and k and v appended to the cache at position p0 + t
// (copyToCache, TransformerComputeKernelsLayered.java:129-139).  Lane i takes
// the rotation pair i (head_dim <= 128: one pair per lane), so no lane reads a
// value another lane writes.
__global__ __launch_bounds__(PBS) void rope_kv_rows_kernel(ModelDev m, int layer, float *QKV, int p0, int T) {
  const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
  const int nh = m.n_heads + m.n_kv;
  const int item = blockIdx.x * (PBS / GL3_WAVE) + wave;
  const int t = item / nh, h = item % nh;
  if (t >= T) return;
  const int hd = m.hd, half = hd / 2, pos = p0 + t;
  float *row = QKV + (size_t)t * (m.q_dim + 2 * m.kv_dim);
  const bool isq = h < m.n_heads, neox = m.family != FAM_LLAMA;
  float *v = isq ? row + h * hd : row + m.q_dim + (h - m.n_heads) * hd;
  const bool act = lane < half;
  const int d0 = neox ? lane : 2 * lane, d1 = neox ? lane + half : 2 * lane + 1;
  float a = act ? v[d0] : 0.0f, b = act ? v[d1] : 0.0f;
  if (m.family == FAM_QWEN3) {
    const LayerDev L = ld_layer(m.layers, layer);
    const float *nw = isq ? L.q_norm : L.k_norm;
    float ss = wave_sum(a * a + b * b);
    ss /= (float)hd;
    ss += m.eps;
    ss = (float)(1.0 / sqrt((double)ss));
    if (act) {
      a = nw[d0] * (ss * a);
      b = nw[d1] * (ss * b);
    }
  }
  if (act) {
    const float c = m.rope_cos[(size_t)pos * half + lane], s = m.rope_sin[(size_t)pos * half + lane];
    const float r0 = a * c - b * s, r1 = a * s + b * c;
    v[d0] = r0;
    v[d1] = r1;
    if (!isq) {
      const int kvh = h - m.n_heads;
      uint16_t *kc = m.kc + (((size_t)layer * m.n_kv + kvh) * m.ctxp + pos) * hd;
      kc[d0] = f2h(r0);
      kc[d1] = f2h(r1);
    }
  }
  if (!isq) {
    const int kvh = h - m.n_heads;
    uint16_t *vt = m.vc + ((size_t)layer * m.n_kv + kvh) * hd * m.ctxp;
    const float *vv = row + m.q_dim + m.kv_dim + kvh * hd;
    for (int d = lane; d < hd; d += GL3_WAVE) vt[((size_t)(pos / 16) * hd + d) * 16 + pos % 16] = f2h(vv[d]);
  }
}

// Causal attention of the block's rows, one wave per (row, query head), over
// positions 0 .. p0 + t of the cache (InferenceCore.java:105-144: scores
// q.k / sqrt(head_dim), softmax, weighted sum of v), as an online softmax over
// chunks of 64 positions: lane j scores position c0 + j; then lane d
// accumulates output dims d and d + 64 over the chunk, 16 positions of its V
// dims per 32-byte read of the transposed V blocks.  Output as hi / lo planes.
template <int HD>
__global__ __launch_bounds__(PBS) void attn_rows_kernel(ModelDev m, int layer, const float *QKV, int p0, int T,
                                                        _Float16 *Oh, _Float16 *Ol) {
  __shared__ float qs[PBS / GL3_WAVE][HD];
  constexpr int DPL = (HD + GL3_WAVE - 1) / GL3_WAVE;  // output dims per lane
  const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
  const int item = blockIdx.x * (PBS / GL3_WAVE) + wave;
  const int t = min(item / m.n_heads, T - 1), h = item % m.n_heads;
  const bool valid = item < T * m.n_heads;
  const float *q = QKV + (size_t)t * (m.q_dim + 2 * m.kv_dim) + h * HD;
  for (int d = lane; d < HD; d += GL3_WAVE) qs[wave][d] = q[d];
  __syncthreads();  // every wave reaches it: invalid items are cut below
  if (!valid) return;
  const int kvh = h / (m.n_heads / m.n_kv), pos = p0 + t;
  const uint16_t *kc = m.kc + ((size_t)layer * m.n_kv + kvh) * m.ctxp * HD;
  const uint16_t *vt = m.vc + ((size_t)layer * m.n_kv + kvh) * HD * m.ctxp;
  float o[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) o[i] = 0.0f;
  float mrun = -INFINITY, lrun = 0.0f;
  for (int c0 = 0; c0 <= pos; c0 += GL3_WAVE) {
    const int p = c0 + lane;
    float s = -INFINITY;
    if (p <= pos) {
      const uint16_t *kr = kc + (size_t)p * HD;
      float a = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; d += 8) {
        const u32x4 w = *(const u32x4 *)(kr + d);
        a = fmaf(qs[wave][d + 0], h2f_lo(w.x), a);
        a = fmaf(qs[wave][d + 1], h2f_hi(w.x), a);
        a = fmaf(qs[wave][d + 2], h2f_lo(w.y), a);
        a = fmaf(qs[wave][d + 3], h2f_hi(w.y), a);
        a = fmaf(qs[wave][d + 4], h2f_lo(w.z), a);
        a = fmaf(qs[wave][d + 5], h2f_hi(w.z), a);
        a = fmaf(qs[wave][d + 6], h2f_lo(w.w), a);
        a = fmaf(qs[wave][d + 7], h2f_hi(w.w), a);
      }
      s = a / m.sqrt_hd;
    }
    const float mn = fmaxf(mrun, wave_max(s));
    const float cf = mrun == -INFINITY ? 0.0f : __expf(mrun - mn);
    const float e = s == -INFINITY ? 0.0f : __expf(s - mn);
    lrun = lrun * cf + wave_sum(e);
    mrun = mn;
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[i] *= cf;
    const int ng = (min(GL3_WAVE, pos + 1 - c0) + 15) / 16;  // 16-position groups of the chunk
    for (int g = 0; g < ng; ++g) {
      const int pb = c0 + 16 * g;  // first position of the group (a multiple of 16)
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const int d = lane + GL3_WAVE * i;
        if (d >= HD) continue;
        const u32x4 *src = (const u32x4 *)(vt + ((size_t)(pb / 16) * HD + d) * 16);
        const u32x4 w0 = src[0], w1 = src[1];
        const unsigned wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float acc = o[i];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          // positions past pos (e = 0) are skipped: their cache entries may be anything, inf or nan included
          const float pk = readlane_f(e, 16 * g + k);
          if (pb + k <= pos) acc = fmaf(pk, k % 2 ? h2f_hi(wv[k / 2]) : h2f_lo(wv[k / 2]), acc);
        }
        o[i] = acc;
      }
    }
  }
  const size_t ob = (size_t)t * m.q_dim + (size_t)h * HD;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + GL3_WAVE * i;
    if (d < HD) put_split(Oh, Ol, ob + d, o[i] / lrun);
  }
}

bool prefill_supported(const ModelDev &m) {
  return (m.hd == 64 || m.hd == 96 || m.hd == 128) && m.dim % 32 == 0 && m.q_dim % 32 == 0 && m.hidden % 32 == 0 &&
         m.rope_cos != nullptr;
}

hipError_t launch_prefill_gemm(int fmt, int mode, const Mat &W, int N, const _Float16 *Xh, const _Float16 *Xl, int T,
                               float *Y, _Float16 *Yh, _Float16 *Yl, hipStream_t s) {
  if (W.cols % 32 != 0 || T <= 0 || N <= 0) return hipErrorInvalidValue;
  const dim3 grid((N + 63) / 64, (T + 63) / 64);
#define GL3_GEMM(F, M)                                                                                          \
  if (fmt == F && mode == M) {                                                                                  \
    hipLaunchKernelGGL((gemm_kernel<F, M>), grid, dim3(PBS), 0, s, W.q, W.s, N, W.cols, Xh, Xl, T, Y, Yh, Yl);  \
    return hipGetLastError();                                                                                   \
  }
  GL3_GEMM(FMT_Q8, MODE_STORE) GL3_GEMM(FMT_Q8, MODE_RESIDUAL) GL3_GEMM(FMT_Q8, MODE_SWIGLU)
  GL3_GEMM(FMT_F16, MODE_STORE) GL3_GEMM(FMT_F16, MODE_RESIDUAL) GL3_GEMM(FMT_F16, MODE_SWIGLU)
#undef GL3_GEMM
  return hipErrorInvalidValue;
}

hipError_t launch_embed_rows(const ModelDev &m, const int *tokens, int T, float *X, hipStream_t s) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3(T), dim3(PBS), 0, s, m, tokens, T, X);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float *X, const float *w, float eps, int dim, int T, _Float16 *Yh, _Float16 *Yl,
                               hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(T), dim3(PBS), 0, s, X, w, eps, dim, T, Yh, Yl);
  return hipGetLastError();
}

hipError_t launch_rope_kv_rows(const ModelDev &m, int layer, float *QKV, int p0, int T, hipStream_t s) {
  if (m.hd > 2 * GL3_WAVE || m.hd % 2) return hipErrorInvalidValue;
  const int waves = T * (m.n_heads + m.n_kv);
  hipLaunchKernelGGL(rope_kv_rows_kernel, dim3((waves + 3) / 4), dim3(PBS), 0, s, m, layer, QKV, p0, T);
  return hipGetLastError();
}

hipError_t launch_attn_rows(const ModelDev &m, int layer, const float *QKV, int p0, int T, _Float16 *Oh, _Float16 *Ol,
                            hipStream_t s) {
  const int grid = (T * m.n_heads + 3) / 4;
#define GL3_AR(HD_)                                                                                          \
  if (m.hd == HD_) {                                                                                         \
    hipLaunchKernelGGL((attn_rows_kernel<HD_>), dim3(grid), dim3(PBS), 0, s, m, layer, QKV, p0, T, Oh, Ol); \
    return hipGetLastError();                                                                                \
  }
  GL3_AR(64) GL3_AR(96) GL3_AR(128)
#undef GL3_AR
  return hipErrorInvalidValue;
}

}  // namespace gl3
