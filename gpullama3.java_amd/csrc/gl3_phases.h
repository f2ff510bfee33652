// The phases of one decode step, written once and used by both schedules:
// the per-phase kernels (one launch per phase, captured in a hipGraph) and the
// persistent per-token kernel (all phases in one launch, separated by grid
// barriers).  Every phase is a grid-stride loop over its work items, so it runs
// on any number of workgroups of GL3_BLOCK threads.
//
// Reference paths are relative to src/main/java/org/beehive/gpullama3/.
#pragma once

#include "gl3_device.h"

namespace gl3 {

enum { FMT_Q8 = 0, FMT_F16 = 1, FMT_F32 = 2 };
enum { MODE_STORE = 0, MODE_RESIDUAL = 1, MODE_SWIGLU = 2, MODE_LOGITS = 3 };
enum { FAM_LLAMA = 0, FAM_QWEN3 = 2, FAM_PHI3 = 3 };

// A weight matrix in the device layout.
//  Q8_0: q = int8 quants row-major [rows][cols]; s = fp16 block scales [rows][cols/32].
//        Same structure-of-arrays split as the reference's device tensor
//        (tensor/tornado/Q8_0TornadoTensor.java:74-117).
//  F16:  q = binary16 row-major [rows][cols] (as bytes); s unused.
struct Mat {
  const uint8_t *q;
  const uint16_t *s;
  int rows, cols;
};

struct LayerDev {
  Mat qkv;    // [q_dim + 2 kv_dim][dim]: Wq, Wk, Wv stacked (Phi3: attn_qkv as is)
  Mat wo;     // [dim][q_dim]
  Mat gu;     // [2 hidden][dim]: gate rows then up rows (Phi3: ffn_up as is)
  Mat down;   // [dim][hidden]
  const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
};

// Per-step control block in device memory.
struct DecodeState {
  int pos;        // position of the token being forwarded
  int token;      // token to forward when from_best == 0
  int from_best;  // 1: forward the argmax of the previous step (best[parity ^ 1])
  int parity;     // which half of best[] this step writes
  int step;       // steps run since the start of the current generate call
  int nbest;      // number of entries per half of best[]
  int pad[2];
};

struct ModelDev {
  int family, fmt, embd_fmt, cls_fmt;  // embd_fmt: FMT_Q8 / FMT_F16 / FMT_F32
  int dim, hidden, n_layers, n_heads, n_kv, hd, q_dim, kv_dim, vocab, ctx;
  int max_split;
  float eps, sqrt_hd;
  const LayerDev *layers;
  Mat embd;                 // token_embd in GEMV layout (Q8_0 / F16), or F32 rows in embd.q
  Mat cls;                  // classifier [vocab][dim]
  const float *out_norm;
  const float *rope_cos, *rope_sin;  // [ctx][hd/2]
  uint16_t *kc, *vc;        // fp16 [L][n_kv][ctx][hd]
  float *x;                 // residual stream [dim]
  float *qkv;               // raw q,k,v [q_dim + 2 kv_dim]
  float *att;               // attention output [q_dim]
  float *hb;                // SwiGLU output [hidden]
  float *logits;            // [vocab]
  float *part;              // attention partials [n_heads][max_split][hd + 2]
  unsigned *att_ctr;        // split-merge counters [L][n_kv]
  unsigned long long *best; // argmax keys [2][nbest]
  DecodeState *st;
  int *tokens_out;          // device copy of generated tokens
};

// ------------------------------------------------------------ step control

struct StepInfo {
  int pos, token, from_best, parity, step, nbest;
};

// Orderable key of (value, row): larger value wins, then the smaller row, as in
// FloatTensor.argmax (tensor/standard/FloatTensor.java:138-151).
__device__ __forceinline__ unsigned long long argmax_key(float v, int row) {
  unsigned b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)row);
}
__device__ __forceinline__ int argmax_key_row(unsigned long long k) { return (int)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFu)); }

// Read the control block and resolve the input token (block-uniform result).
__device__ inline StepInfo read_step(const ModelDev &m, int *lds_i) {
  if (threadIdx.x < GL3_WAVE) {
    const int *s = (const int *)m.st;
    int v = threadIdx.x < 6 ? ld_coherent_i32(s + threadIdx.x) : 0;
    int from_best = __shfl(v, 2), parity = __shfl(v, 3), nbest = __shfl(v, 5);
    unsigned long long best = 0;
    if (from_best) {
      const unsigned long long *src = m.best + (size_t)(parity ^ 1) * nbest;
      for (int i = threadIdx.x; i < nbest; i += GL3_WAVE) {
        unsigned long long k = ld_coherent_u64(src + i);
        best = k > best ? k : best;
      }
      for (int o = 32; o >= 1; o >>= 1) {
        unsigned long long other = __shfl_xor(best, o);
        best = other > best ? other : best;
      }
    }
    if (threadIdx.x < 6) lds_i[threadIdx.x] = v;
    if (threadIdx.x == 0 && from_best) {
      int row = argmax_key_row(best);
      lds_i[1] = (row >= 0 && row < m.vocab) ? row : 0;  // an empty key set cannot index past the table
    }
  }
  __syncthreads();
  StepInfo si;
  si.pos = lds_i[0];
  si.token = lds_i[1];
  si.from_best = lds_i[2];
  si.parity = lds_i[3];
  si.step = lds_i[4];
  si.nbest = lds_i[5];
  __syncthreads();
  return si;
}

// Advance the control block after every workgroup has read it.
__device__ inline void advance_step(const ModelDev &m, const StepInfo &si) {
  if (threadIdx.x == 0) {
    if (si.from_best && si.step > 0) m.tokens_out[si.step - 1] = si.token;
    int *s = (int *)m.st;
    __hip_atomic_store(s + 0, si.pos + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(s + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(s + 3, si.parity ^ 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(s + 4, si.step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// -------------------------------------------------------------- embedding
// x = token_embedding_table[token] (InferenceCore.java:68; the GPU path copies
// the fp32-converted row on the host, InferenceCore.java:586).
__device__ inline void phase_embed(const ModelDev &m, int token, int blk, int nblk) {
  const int dim = m.dim;
  for (int i = blk * GL3_BLOCK + threadIdx.x; i < dim; i += nblk * GL3_BLOCK) {
    size_t e = (size_t)token * dim + i;
    float v;
    if (m.embd_fmt == FMT_F32) {
      v = ((const float *)m.embd.q)[e];
    } else if (m.embd_fmt == FMT_Q8) {
      v = (float)(int8_t)m.embd.q[e] * h2f(m.embd.s[e / 32]);
    } else {
      v = h2f(((const uint16_t *)m.embd.q)[e]);
    }
    st_coherent(m.x + i, v);
  }
}

// ------------------------------------------------------------------ GEMV
// y = W · n(x): one wavefront computes NR rows (NR row pairs for SwiGLU) over
// its K-slice; KS waves of a workgroup split K.  Each lane owns fixed 16-byte
// chunks of every row, so its slice of x stays in registers for all rows.
// Weights stream with 128-bit non-temporal loads, are converted in registers
// (Q8_0: one sign-extending byte->float conversion per element, per 16-element
// chunk acc += s * sum(q*x); F16: exact half->float), and accumulate in fp32.  No MFMA: batch-1 GEMV is
// bound by HBM bandwidth.
//
// Follows matrixVectorGeneric / matrixVectorGenericWithResidual /
// fusedFeedForwardWithSiLUAndGLUActivation (kernels/TransformerComputeKernelsLayered.java:650-1057).

template <int FMT>
struct ChunkTraits;
template <>
struct ChunkTraits<FMT_Q8> {
  static constexpr int EPC = 16;  // elements per 16-byte chunk
  static constexpr int ESZ = 1;   // bytes per element
};
template <>
struct ChunkTraits<FMT_F16> {
  static constexpr int EPC = 8;
  static constexpr int ESZ = 2;
};

// Load x (coherently) into LDS, applying RMSNorm when normw != nullptr:
// xs[i] = normw[i] * (ss * x[i]), ss = 1/sqrt(mean(x^2) + eps) (InferenceCore.java:46-55).
__device__ inline void load_x_lds(const float *x, const float *normw, float eps, int K, float *xs, float *red) {
  float ss = 0.0f;
  for (int i = threadIdx.x; i < K; i += GL3_BLOCK) {
    float v = ld_coherent(x + i);
    xs[i] = v;
    ss += v * v;
  }
  if (normw) {
    ss = block_sum(ss, red);
    ss /= (float)K;
    ss += eps;
    ss = (float)(1.0 / sqrt((double)ss));
    for (int i = threadIdx.x; i < K; i += GL3_BLOCK) xs[i] = normw[i] * (ss * xs[i]);
  }
  __syncthreads();
}

__device__ __forceinline__ float silu_ref(float v) { return v / (float)(1.0 + exp((double)(-v))); }

template <int FMT, int KC, int KS, int NR, int MODE>
struct GemvPhase {
  typedef ChunkTraits<FMT> T;
  static constexpr int EPC = T::EPC;
  static constexpr int XPL = KC * EPC;                   // x floats per lane
  static constexpr int RG = GL3_WAVES_PER_BLOCK / KS;    // row groups per workgroup
  static constexpr int NP = (MODE == MODE_SWIGLU) ? 2 : 1;
  static constexpr int ROWS_PER_ITEM = RG * NR;          // output rows per work item

  struct Tile {
    u32x4 w[NR][NP][KC];
    float s[NR][NP][KC];
  };

  // K-slice of this wave and the element offset of lane chunk j.
  static __device__ __forceinline__ int elem(int K, int ks, int lane, int j) {
    return ks * (K / KS) + EPC * (lane + GL3_WAVE * j);
  }

  static __device__ __forceinline__ void load_tile(const Mat &W, int out_rows, int item, int rg, int ks, int lane,
                                                   Tile &t) {
    const int K = W.cols;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      int row = item * ROWS_PER_ITEM + rg * NR + r;
      row = row < out_rows ? row : out_rows - 1;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const size_t wrow = (size_t)(row + p * out_rows);
#pragma unroll
        for (int j = 0; j < KC; ++j) {
          const int e = elem(K, ks, lane, j);
          t.w[r][p][j] = ld_stream(W.q + (wrow * K + e) * T::ESZ);
          if (FMT == FMT_Q8) t.s[r][p][j] = h2f(W.s[wrow * (K / 32) + e / 32]);
        }
      }
    }
  }

  // Partial dot products of the lane for every (row, pair).
  static __device__ __forceinline__ void dot_tile(const Tile &t, const float (&xr)[KC][EPC], float (&acc)[NR][NP]) {
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < KC; ++j) {
          const u32x4 w = t.w[r][p][j];
          if (FMT == FMT_Q8) {
            float c = 0.0f;
            const unsigned ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              c = fmaf(sbyte<0>(ww[d]), xr[j][4 * d + 0], c);
              c = fmaf(sbyte<1>(ww[d]), xr[j][4 * d + 1], c);
              c = fmaf(sbyte<2>(ww[d]), xr[j][4 * d + 2], c);
              c = fmaf(sbyte<3>(ww[d]), xr[j][4 * d + 3], c);
            }
            a = fmaf(t.s[r][p][j], c, a);
          } else {
            const unsigned ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              a = fmaf(h2f_lo(ww[d]), xr[j][2 * d + 0], a);
              a = fmaf(h2f_hi(ww[d]), xr[j][2 * d + 1], a);
            }
          }
        }
        acc[r][p] = a;
      }
  }

  // Runs the phase.  x: input vector (K floats, coherent); normw: RMSNorm
  // weights or nullptr; y: output (MODE_RESIDUAL: y += W n(x)); for
  // MODE_LOGITS, y gets the rows and best_out[blk] the argmax key of the rows
  // this workgroup produced.
  static __device__ void run(const Mat &W, int out_rows, const float *x, const float *normw, float eps, float *y,
                             unsigned long long *best_out, int blk, int nblk, float *lds) {
    const int K = W.cols;
    float *xs = lds;                 // K floats
    float *red = lds + K;            // reduction scratch
    float *kpart = red + 16;         // [RG][NR][NP][KS] cross-wave partials
    load_x_lds(x, normw, eps, K, xs, red);

    const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
    const int ks = wave % KS, rg = wave / KS;
    float xr[KC][EPC];
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int e = elem(K, ks, lane, j);
#pragma unroll
      for (int i = 0; i < EPC; ++i) xr[j][i] = xs[e + i];
    }

    const int n_items = (out_rows + ROWS_PER_ITEM - 1) / ROWS_PER_ITEM;
    unsigned long long best = 0;
    int item = blk;
    Tile cur;
    if (item < n_items) load_tile(W, out_rows, item, rg, ks, lane, cur);
    for (; item < n_items; item += nblk) {
      Tile nxt;
      const int next = item + nblk;
      if (next < n_items) load_tile(W, out_rows, next, rg, ks, lane, nxt);
      float acc[NR][NP];
      dot_tile(cur, xr, acc);
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int p = 0; p < NP; ++p) acc[r][p] = wave_sum(acc[r][p]);
      if (KS > 1) {
        if (lane == 0) {
#pragma unroll
          for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int p = 0; p < NP; ++p) kpart[((rg * NR + r) * NP + p) * KS + ks] = acc[r][p];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < KS; ++q) s += kpart[((rg * NR + r) * NP + p) * KS + q];
            acc[r][p] = s;
          }
        __syncthreads();
      }
      if (lane == 0 && ks == 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int row = item * ROWS_PER_ITEM + rg * NR + r;
          if (row < out_rows) {
            if (MODE == MODE_STORE) {
              st_coherent(y + row, acc[r][0]);
            } else if (MODE == MODE_RESIDUAL) {
              st_coherent(y + row, ld_coherent(y + row) + acc[r][0]);
            } else if (MODE == MODE_SWIGLU) {
              st_coherent(y + row, silu_ref(acc[r][0]) * acc[r][NP - 1]);
            } else {
              y[row] = acc[r][0];
              unsigned long long k = argmax_key(acc[r][0], row);
              best = k > best ? k : best;
            }
          }
        }
      }
      if (next < n_items) cur = nxt;
    }
    if (MODE == MODE_LOGITS) {
      __shared__ unsigned long long bred[GL3_WAVES_PER_BLOCK];
      if (lane == 0) bred[wave] = best;
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned long long b = 0;
        for (int w = 0; w < GL3_WAVES_PER_BLOCK; ++w) b = bred[w] > b ? bred[w] : b;
        __hip_atomic_store(best_out + blk, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();  // LDS is reused by the next phase
  }

  static constexpr size_t lds_bytes(int K) { return (size_t)(K + 16 + RG * NR * NP * KS + 16) * sizeof(float); }
};

// -------------------------------------------------------------- attention
// Flash-decode over the fp16 KV cache [L][n_kv][ctx][hd].  Work item = (kv head,
// split of positions); the workgroup serves every query head of the kv head's
// GQA group, so each K/V row is read from HBM once per group.  K and V tiles of
// ATT_TILE positions are staged in LDS (converted to fp32 once); scores use the
// reference's order of operations (sequential dot, then / sqrt(hd), InferenceCore.java:114-121),
// softmax is online within the split and splits merge by log-sum-exp in the
// workgroup that finishes last.  The same workgroup applies the Qwen3 per-head
// RMSNorm and RoPE to q and, for the split holding `pos`, to k, and appends k,v
// to the cache (InferenceCore.java:82-100, :341-372, :472-491).

#define ATT_TILE 64
#define ATT_MAX_G 8

__device__ __forceinline__ void rope_pair(float &v0, float &v1, float c, float s) {
  float a = v0 * c - v1 * s;
  float b = v0 * s + v1 * c;
  v0 = a;
  v1 = b;
}

// Prepare `nvec` head vectors of length hd from src (coherent) into dst (LDS):
// optional per-head RMSNorm, then RoPE at pos.  Caller must __syncthreads() after.
__device__ inline void prep_heads(const ModelDev &m, const float *src, int nvec, const float *normw, int pos,
                                  float *dst, float *red) {
  const int hd = m.hd, half = hd / 2;
  for (int i = threadIdx.x; i < nvec * hd; i += GL3_BLOCK) dst[i] = ld_coherent(src + i);
  __syncthreads();
  if (normw) {
    // one wave per head vector: ss = sum x^2; x = w * (ss * x)   (Qwen3Kernels / InferenceCore.java:341-347)
    const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
    for (int g = wave; g < nvec; g += GL3_WAVES_PER_BLOCK) {
      float ss = 0.0f;
      for (int d = lane; d < hd; d += GL3_WAVE) ss += dst[g * hd + d] * dst[g * hd + d];
      ss = wave_sum(ss);
      ss /= (float)hd;
      ss += m.eps;
      ss = (float)(1.0 / sqrt((double)ss));
      for (int d = lane; d < hd; d += GL3_WAVE) dst[g * hd + d] = normw[d] * (ss * dst[g * hd + d]);
    }
    __syncthreads();
  }
  const float *cr = m.rope_cos + (size_t)pos * half, *ci = m.rope_sin + (size_t)pos * half;
  for (int t = threadIdx.x; t < nvec * half; t += GL3_BLOCK) {
    const int g = t / half, i = t % half;
    int i0, i1;
    if (m.family == FAM_LLAMA) { i0 = 2 * i; i1 = 2 * i + 1; }
    else { i0 = i; i1 = i + half; }
    float v0 = dst[g * hd + i0], v1 = dst[g * hd + i1];
    rope_pair(v0, v1, cr[i], ci[i]);
    dst[g * hd + i0] = v0;
    dst[g * hd + i1] = v1;
  }
}

__device__ inline int att_split_len(const ModelDev &m, int pos) {
  const int n = pos + 1;
  int s = (n + m.max_split - 1) / m.max_split;
  s = (s + ATT_TILE - 1) / ATT_TILE * ATT_TILE;
  return s < ATT_TILE ? ATT_TILE : s;
}

__device__ inline size_t att_lds_floats(int hd, int G) {
  return (size_t)G * hd            // q
         + 2 * hd                  // new k, v
         + ATT_TILE * (hd + 1)     // K tile (padded rows)
         + ATT_TILE * hd           // V tile
         + G * ATT_TILE            // p
         + 3 * ATT_MAX_G + 16;     // m, l, scale, flags
}

__device__ void phase_attention(const ModelDev &m, int layer, int pos, int blk, int nblk, float *lds) {
  const int hd = m.hd, G = m.n_heads / m.n_kv, kv_dim = m.kv_dim;
  const int S = att_split_len(m, pos);
  const int n = pos + 1;
  const int nsplit = (n + S - 1) / S;
  const int items = m.n_kv * nsplit;
  const int hdp = hd + 1;
  float *qs = lds;
  float *knew = qs + G * hd;
  float *vnew = knew + hd;
  float *kt = vnew + hd;
  float *vt = kt + ATT_TILE * hdp;
  float *ps = vt + ATT_TILE * hd;
  float *ml = ps + G * ATT_TILE;   // m[G], l[G], scale[G]
  int *flag = (int *)(ml + 3 * ATT_MAX_G);
  float *red = (float *)(flag + 8);
  const LayerDev &L = m.layers[layer];
  const size_t head_stride = (size_t)m.ctx * hd;
  uint16_t *kc_l = m.kc + (size_t)layer * m.n_kv * head_stride;
  uint16_t *vc_l = m.vc + (size_t)layer * m.n_kv * head_stride;

  for (int item = blk; item < items; item += nblk) {
    const int kvh = item / nsplit, sp = item % nsplit;
    const int t0 = sp * S, t1 = min(n, t0 + S);
    uint16_t *kh = kc_l + kvh * head_stride;
    uint16_t *vh = vc_l + kvh * head_stride;
    // q of the group's heads (contiguous in qkv), normalised and rotated
    prep_heads(m, m.qkv + (size_t)kvh * G * hd, G, m.family == FAM_QWEN3 ? L.q_norm : nullptr, pos, qs, red);
    const bool owns_pos = (pos >= t0 && pos < t1);
    if (owns_pos) {
      __syncthreads();
      prep_heads(m, m.qkv + m.q_dim + (size_t)kvh * hd, 1, m.family == FAM_QWEN3 ? L.k_norm : nullptr, pos, knew, red);
      for (int d = threadIdx.x; d < hd; d += GL3_BLOCK) vnew[d] = ld_coherent(m.qkv + m.q_dim + kv_dim + (size_t)kvh * hd + d);
      __syncthreads();
      for (int d = threadIdx.x; d < hd; d += GL3_BLOCK) {
        uint16_t kh16 = f2h(knew[d]), vh16 = f2h(vnew[d]);
        kh[(size_t)pos * hd + d] = kh16;
        vh[(size_t)pos * hd + d] = vh16;
        knew[d] = h2f(kh16);
        vnew[d] = h2f(vh16);
      }
    }
    if (threadIdx.x < G) {
      ml[threadIdx.x] = -INFINITY;
      ml[ATT_MAX_G + threadIdx.x] = 0.0f;
    }
    // output accumulators: thread handles (g, d) pairs idx = threadIdx.x + k*GL3_BLOCK
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int npairs = G * hd;
    __syncthreads();

    for (int tt = t0; tt < t1; tt += ATT_TILE) {
      const int nt = min(ATT_TILE, t1 - tt);
      // stage K and V rows [tt, tt+nt) as fp32; 8 halfs (16 bytes) per load
      const int chunks = ATT_TILE * hd / 8;
      for (int c = threadIdx.x; c < chunks; c += GL3_BLOCK) {
        const int t = (c * 8) / hd, d0 = (c * 8) % hd;
        const int tp = tt + t;
        float kf[8], vf[8];
        if (t < nt && tp != pos) {
          u32x4 kw = ld_stream(kh + (size_t)tp * hd + d0);
          u32x4 vw = ld_stream(vh + (size_t)tp * hd + d0);
          const unsigned ka[4] = {kw.x, kw.y, kw.z, kw.w}, va[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            kf[2 * i] = h2f_lo(ka[i]); kf[2 * i + 1] = h2f_hi(ka[i]);
            vf[2 * i] = h2f_lo(va[i]); vf[2 * i + 1] = h2f_hi(va[i]);
          }
        } else if (t < nt) {
#pragma unroll
          for (int i = 0; i < 8; ++i) { kf[i] = knew[d0 + i]; vf[i] = vnew[d0 + i]; }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) { kf[i] = 0.0f; vf[i] = 0.0f; }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kt[t * hdp + d0 + i] = kf[i];
          vt[t * hd + d0 + i] = vf[i];
        }
      }
      __syncthreads();
      // scores: thread (t, g)
      for (int idx = threadIdx.x; idx < G * ATT_TILE; idx += GL3_BLOCK) {
        const int t = idx % ATT_TILE, g = idx / ATT_TILE;
        float s = -INFINITY;
        if (t < nt) {
          const float *q = qs + g * hd, *k = kt + t * hdp;
          float acc = 0.0f;
          for (int d = 0; d < hd; ++d) acc += q[d] * k[d];
          s = acc / m.sqrt_hd;
        }
        ps[g * ATT_TILE + t] = s;
      }
      __syncthreads();
      // online softmax per head: one wave per head
      {
        const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
        for (int g = wave; g < G; g += GL3_WAVES_PER_BLOCK) {
          float s = ps[g * ATT_TILE + lane];  // ATT_TILE == GL3_WAVE
          float mt = wave_max(s);
          float mold = ml[g];
          float mnew = fmaxf(mold, mt);
          float p = (lane < nt) ? expf(s - mnew) : 0.0f;
          ps[g * ATT_TILE + lane] = p;
          float lsum = wave_sum(p);
          float scale = expf(mold - mnew);  // exp(-inf) = 0 on the first tile
          if (lane == 0) {
            ml[g] = mnew;
            ml[ATT_MAX_G + g] = ml[ATT_MAX_G + g] * scale + lsum;
            ml[2 * ATT_MAX_G + g] = scale;
          }
        }
      }
      __syncthreads();
      // o[g][d] = o * scale + sum_t p[g][t] * V[t][d]
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int idx = threadIdx.x + k * GL3_BLOCK;
        if (idx < npairs) {
          const int g = idx / hd, d = idx % hd;
          float acc = o[k] * ml[2 * ATT_MAX_G + g];
          for (int t = 0; t < nt; ++t) acc += ps[g * ATT_TILE + t] * vt[t * hd + d];
          o[k] = acc;
        }
      }
      __syncthreads();
    }

    // write the result of this split
    const int hpart = hd + 2;
    if (nsplit == 1) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int idx = threadIdx.x + k * GL3_BLOCK;
        if (idx < npairs) {
          const int g = idx / hd, d = idx % hd;
          st_coherent(m.att + (size_t)(kvh * G + g) * hd + d, o[k] / ml[ATT_MAX_G + g]);
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int idx = threadIdx.x + k * GL3_BLOCK;
        if (idx < npairs) {
          const int g = idx / hd, d = idx % hd;
          st_coherent(m.part + ((size_t)(kvh * G + g) * m.max_split + sp) * hpart + d, o[k]);
        }
      }
      if (threadIdx.x < G) {
        float *pp = m.part + ((size_t)(kvh * G + threadIdx.x) * m.max_split + sp) * hpart;
        st_coherent(pp + hd, ml[threadIdx.x]);
        st_coherent(pp + hd + 1, ml[ATT_MAX_G + threadIdx.x]);
      }
      vmem_drain();
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned *ctr = m.att_ctr + layer * m.n_kv + kvh;
        unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = (old == (unsigned)(nsplit - 1));
        flag[0] = last;
        if (last) st_coherent_u32(ctr, 0u);
      }
      __syncthreads();
      if (flag[0]) {
        // log-sum-exp merge of the splits for every head of the group
        for (int idx = threadIdx.x; idx < npairs; idx += GL3_BLOCK) {
          const int g = idx / hd, d = idx % hd;
          const float *base = m.part + (size_t)(kvh * G + g) * m.max_split * hpart;
          float M = -INFINITY;
          for (int s = 0; s < nsplit; ++s) M = fmaxf(M, ld_coherent(base + (size_t)s * hpart + hd));
          float Ls = 0.0f, O = 0.0f;
          for (int s = 0; s < nsplit; ++s) {
            const float *ps_ = base + (size_t)s * hpart;
            float w = expf(ld_coherent(ps_ + hd) - M);
            Ls += w * ld_coherent(ps_ + hd + 1);
            O += w * ld_coherent(ps_ + d);
          }
          st_coherent(m.att + (size_t)(kvh * G + g) * hd + d, O / Ls);
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace gl3
