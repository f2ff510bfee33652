// GEMV for any row length: the per-phase schedule's kernel for widths outside
// the compiled tiles of the GemvPhase kernels (e.g. Qwen3-4B's dim 2560 and
// hidden 9728), with the same four epilogues (matrixVectorGeneric,
// matrixVectorGenericWithResidual, fusedFeedForwardWithSiLUAndGLUActivation and
// the logits with their argmax key: kernels/TransformerComputeKernelsLayered.java:650-1057,
// layers/type/q8_0/LogitsQ8_0Layer.java:58-73).
//
// A workgroup stages the input vector in LDS once (RMSNorm applied: mean of
// squares in fp32, 1/sqrt in double, w * (ss * x), InferenceCore.java:46-55);
// each wave then takes 4 rows at a time and streams them in 16-byte chunks,
// 64 lanes side by side along the row (coalesced), all rows' loads of a step
// issued before any is used.  Q8_0: 16 int8 weights per chunk, one fp16 block
// scale per chunk (K is a multiple of 32, so a chunk never straddles a block);
// FP16: 8 weights per chunk.  fp32 accumulation, wavefront reduction.
#include <algorithm>

#include "gl3_internal.h"

namespace gl3 {

namespace {

constexpr int AB = GL3_BLOCK;         // threads per workgroup
constexpr int AWPB = AB / GL3_WAVE;   // waves per workgroup
constexpr int ARB = 4;                // rows per wave per pass

template <int FMT, int MODE>
__device__ void gemv_any_body(const Mat &W, int out_rows, const float *x, const float *normw, float eps, float *y,
                              unsigned long long *best, float *xs) {
  constexpr int EPC = FMT == FMT_Q8 ? 16 : 8;  // weights per 16-byte chunk
  constexpr int NP = MODE == MODE_SWIGLU ? 2 : 1;
  __shared__ float red[AWPB];
  __shared__ unsigned long long bk[AWPB];
  const int K = W.cols;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < K; i += AB) {
    const float v = x[i];
    xs[i] = v;
    ss += v * v;
  }
  if (normw) {
    ss = block_sum<AB>(ss, red);
    ss /= (float)K;
    ss += eps;
    ss = (float)(1.0 / sqrt((double)ss));
    for (int i = threadIdx.x; i < K; i += AB) xs[i] = normw[i] * (ss * xs[i]);
  }
  __syncthreads();
  const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
  unsigned long long kbest = 0ull;
  const int stride = gridDim.x * AWPB * ARB;
  for (int r0 = (blockIdx.x * AWPB + wave) * ARB; r0 < out_rows; r0 += stride) {  // uniform over the wave
    float acc[ARB][NP];
#pragma unroll
    for (int r = 0; r < ARB; ++r)
#pragma unroll
      for (int p = 0; p < NP; ++p) acc[r][p] = 0.0f;
    for (int c0 = EPC * lane; c0 < K; c0 += GL3_WAVE * EPC) {
      u32x4 w[ARB][NP];
      float sc[ARB][NP];
#pragma unroll
      for (int r = 0; r < ARB; ++r)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const size_t row = (size_t)min(r0 + r, out_rows - 1) + (size_t)p * out_rows;
          if (FMT == FMT_Q8) {
            w[r][p] = *(const u32x4 *)(W.q + row * K + c0);
            sc[r][p] = h2f(W.s[row * (K / 32) + c0 / 32]);
          } else {
            w[r][p] = *(const u32x4 *)(W.q + (row * K + c0) * 2);
            sc[r][p] = 1.0f;
          }
        }
      float xv[EPC];
#pragma unroll
      for (int i = 0; i < EPC; ++i) xv[i] = xs[c0 + i];
#pragma unroll
      for (int r = 0; r < ARB; ++r)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const unsigned wd[4] = {w[r][p].x, w[r][p].y, w[r][p].z, w[r][p].w};
          float d = 0.0f;
          if (FMT == FMT_Q8) {
#pragma unroll
            for (int i = 0; i < 16; ++i) d = fmaf((float)(signed char)((wd[i / 4] >> (8 * (i % 4))) & 0xffu), xv[i], d);
            acc[r][p] = fmaf(d, sc[r][p], acc[r][p]);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(i % 2 ? h2f_hi(wd[i / 2]) : h2f_lo(wd[i / 2]), xv[i], d);
            acc[r][p] += d;
          }
        }
    }
#pragma unroll
    for (int r = 0; r < ARB; ++r) {
      const int row = r0 + r;
      if (row >= out_rows) break;  // uniform over the wave
      const float a = wave_sum(acc[r][0]);
      const float u = NP == 2 ? wave_sum(acc[r][NP - 1]) : 0.0f;
      if (lane == 0) {
        if (MODE == MODE_STORE)
          y[row] = a;
        else if (MODE == MODE_RESIDUAL)
          y[row] += a;
        else if (MODE == MODE_SWIGLU)
          y[row] = silu_ref(a) * u;  // InferenceCore.java:162-166
        else {
          y[row] = a;
          const unsigned long long k = argmax_key(a, row);
          kbest = k > kbest ? k : kbest;
        }
      }
    }
  }
  if (MODE == MODE_LOGITS) {
    // the workgroup's best key (FloatTensor.argmax: the larger value, then the smaller row)
    if (lane == 0) bk[wave] = kbest;
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned long long b = 0ull;
      for (int i = 0; i < AWPB; ++i) b = bk[i] > b ? bk[i] : b;
      best[blockIdx.x] = b;
    }
  }
}

template <int FMT, int MODE>
__global__ __launch_bounds__(AB) void gemv_any_kernel(Mat W, int out_rows, const float *x, const float *normw, float eps,
                                                      float *y, unsigned long long *best) {
  extern __shared__ float xs[];
  gemv_any_body<FMT, MODE>(W, out_rows, x, normw, eps, y, best, xs);
}

template <int FMT>
__global__ __launch_bounds__(AB) void logits_any_kernel(ModelDev m) {
  extern __shared__ float xs[];
  const int parity = ld_coherent_i32(&m.st->parity);
  const int nbest = ld_coherent_i32(&m.st->nbest);
  gemv_any_body<FMT, MODE_LOGITS>(m.cls, m.vocab, m.x, m.out_norm, m.eps, m.logits, m.best + (size_t)parity * nbest,
                                  xs);
}

}  // namespace

bool gemv_any_supported(int fmt, int K) {
  return K > 0 && K <= GL3_GEMV_ANY_MAX_K && K % (fmt == FMT_Q8 ? 32 : 8) == 0;
}

hipError_t launch_gemv_any(int fmt, int mode, const Mat &W, int out_rows, const float *x, const float *normw,
                           float eps, float *y, unsigned long long *best, int grid, hipStream_t s) {
  if (!gemv_any_supported(fmt, W.cols) || out_rows <= 0) return hipErrorInvalidValue;
  if (grid <= 0) grid = std::min((out_rows + AWPB * ARB - 1) / (AWPB * ARB), 2048);
  const size_t lds = (size_t)W.cols * sizeof(float);
#define GL3_ANY(F, M)                                                                                          \
  if (fmt == F && mode == M) {                                                                                 \
    hipLaunchKernelGGL((gemv_any_kernel<F, M>), dim3(grid), dim3(AB), lds, s, W, out_rows, x, normw, eps, y, best); \
    return hipGetLastError();                                                                                  \
  }
  GL3_ANY(FMT_Q8, MODE_STORE) GL3_ANY(FMT_Q8, MODE_RESIDUAL) GL3_ANY(FMT_Q8, MODE_SWIGLU) GL3_ANY(FMT_Q8, MODE_LOGITS)
  GL3_ANY(FMT_F16, MODE_STORE) GL3_ANY(FMT_F16, MODE_RESIDUAL) GL3_ANY(FMT_F16, MODE_SWIGLU) GL3_ANY(FMT_F16, MODE_LOGITS)
#undef GL3_ANY
  return hipErrorInvalidValue;
}

hipError_t launch_logits_any(const ModelDev &m, int grid, hipStream_t s) {
  if (!gemv_any_supported(m.cls_fmt, m.dim) || grid <= 0) return hipErrorInvalidValue;
  const size_t lds = (size_t)m.dim * sizeof(float);
  if (m.cls_fmt == FMT_Q8)
    hipLaunchKernelGGL(logits_any_kernel<FMT_Q8>, dim3(grid), dim3(AB), lds, s, m);
  else if (m.cls_fmt == FMT_F16)
    hipLaunchKernelGGL(logits_any_kernel<FMT_F16>, dim3(grid), dim3(AB), lds, s, m);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace gl3
