// The phases of one decode step, written once and used by both schedules:
// the per-phase kernels (one launch per phase, captured in a hipGraph) and the
// persistent per-token kernel (all phases in one launch, separated by grid
// barriers).  Every phase is a grid-stride loop over its work items and is
// templated on the workgroup size BS, so it runs on any number of workgroups.
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
  Mat down_sl;  // Q8_0 down in 32-column slices (fused FFN of the persistent kernel): quants
                // [hidden/32][dim][32], scales [hidden/32][dim]
  const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
};

// Layer descriptors are read through the constant address space: they are
// written by the host only, so the loads are scalar and the matrix pointers
// land in SGPRs (buffer descriptors built from them stay uniform).
typedef __attribute__((address_space(4))) const Mat cMat;
typedef __attribute__((address_space(4))) const LayerDev cLayerDev;
__device__ __forceinline__ Mat ld_mat(const cMat *p) {
  Mat r;
  r.q = p->q;
  r.s = p->s;
  r.rows = p->rows;
  r.cols = p->cols;
  return r;
}
__device__ __forceinline__ LayerDev ld_layer(const LayerDev *layers, int l) {
  const cLayerDev *p = (const cLayerDev *)(layers + l);
  LayerDev r;
  r.qkv = ld_mat(&p->qkv);
  r.wo = ld_mat(&p->wo);
  r.gu = ld_mat(&p->gu);
  r.down = ld_mat(&p->down);
  r.attn_norm = p->attn_norm;
  r.ffn_norm = p->ffn_norm;
  r.q_norm = p->q_norm;
  r.k_norm = p->k_norm;
  return r;
}

// Per-step control block in device memory.
struct DecodeState {
  int pos;        // position of the token being forwarded
  int token;      // token to forward when from_best == 0
  int from_best;  // 1: forward the argmax of the previous step (best[parity ^ 1])
  int parity;     // which half of best[] this step writes
  int step;       // steps run since the start of the current generate call
  int nbest;      // number of entries per half of best[]
  int n_prompt;   // steps 0 .. n_prompt-1 forward the prompt tokens (prompt[step]); later steps the argmax
  int pad;
};

struct ModelDev {
  int family, fmt, embd_fmt, cls_fmt;  // embd_fmt: FMT_Q8 / FMT_F16 / FMT_F32
  int dim, hidden, n_layers, n_heads, n_kv, hd, q_dim, kv_dim, vocab, ctx;
  int ctxp;                 // KV cache position stride: ctx rounded up to a multiple of 16
  int max_split;
  float eps, sqrt_hd;
  const LayerDev *layers;
  Mat embd;                 // token_embd in GEMV layout (Q8_0 / F16), or F32 rows in embd.q
  Mat cls;                  // classifier [vocab][dim]
  const float *out_norm;
  const float *rope_cos, *rope_sin;  // [ctx][hd/2]
  uint16_t *kc;             // fp16 K cache [L][n_kv][ctxp][hd]
  uint16_t *vc;             // fp16 V cache in 16-position blocks, transposed: [L][n_kv][ctxp/16][hd][16]
  float *x;                 // residual stream [dim]
  float *qkv;               // raw q,k,v [q_dim + 2 kv_dim]
  float *att;               // attention output [q_dim]
  float *hb;                // SwiGLU output [hidden]
  // the same vectors as tagged cells, for the persistent kernel: residual
  // stream ping-pong (txa: embedding and FFN outputs, txb: attention block
  // outputs), q/k/v, attention output, SwiGLU output
  uint2 *txa, *txb, *tqkv, *tatt, *thb;
  uint2 *tpart;             // attention partials as tagged cells, laid out as part
  uint2 *tdp;               // fused FFN: down-projection partials [workgroup][dim] as tagged cells
  float *logits;            // [vocab]
  float *part;              // attention partials [n_heads][max_split][hd + 4]: o[hd], m, l, pad
  unsigned *att_ctr;        // split-merge counters [L][n_kv]
  unsigned long long *best; // argmax keys [2][nbest]
  DecodeState *st;
  int *tokens_out;          // device copy of generated tokens
  const int *prompt;        // prompt tokens of the current generate call [context length]
  unsigned long long *tstamp;  // optional phase trace: s_memrealtime at each phase boundary, per workgroup
};

// Phase trace of the persistent kernel: every workgroup stamps the 100 MHz
// real-time counter when it leaves a phase (before the grid barrier) and when
// it enters the next one (after the barrier).
__device__ __forceinline__ void trace(const ModelDev &m, int idx) {
  if (m.tstamp && threadIdx.x == 0) m.tstamp[(size_t)idx * gridDim.x + blockIdx.x] = __builtin_amdgcn_s_memrealtime();
}

// ------------------------------------------------------------ step control

struct StepInfo {
  int pos, token, from_best, parity, step, nbest, n_prompt;
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
    int v = threadIdx.x < 7 ? ld_coherent_i32(s + threadIdx.x) : 0;
    int from_best = __shfl(v, 2), parity = __shfl(v, 3), nbest = __shfl(v, 5);
    unsigned long long best = 0;
    if (from_best) {
      // 4 keys per lane per 256, both 16-byte loads of a round in flight together
      const unsigned long long *src = m.best + (size_t)(parity ^ 1) * nbest;
      for (int i0 = 4 * threadIdx.x; i0 < nbest; i0 += 4 * GL3_WAVE) {
        const u32x4 a = ld_coherent_x4(src, (unsigned)(i0 < nbest ? i0 : 0) * 8u);
        const u32x4 b = ld_coherent_x4(src, (unsigned)(i0 + 2 < nbest ? i0 + 2 : 0) * 8u);
        const unsigned long long k[4] = {((unsigned long long)a.y << 32) | a.x, ((unsigned long long)a.w << 32) | a.z,
                                         ((unsigned long long)b.y << 32) | b.x, ((unsigned long long)b.w << 32) | b.z};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (i0 + j < nbest) best = k[j] > best ? k[j] : best;
      }
      for (int o = 32; o >= 1; o >>= 1) {
        unsigned long long other = __shfl_xor(best, o);
        best = other > best ? other : best;
      }
    }
    if (threadIdx.x < 7) lds_i[threadIdx.x] = v;
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
  si.n_prompt = lds_i[6];
  __syncthreads();
  return si;
}

// Advance the control block after every workgroup has read it.
__device__ inline void advance_step(const ModelDev &m, const StepInfo &si) {
  if (threadIdx.x == 0) {
    if (si.from_best && si.step > 0) m.tokens_out[si.step - 1] = si.token;
    int *s = (int *)m.st;
    __hip_atomic_store(s + 0, si.pos + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the next step forwards the next prompt token while the prompt lasts
    // (InferenceEngine.java:83-131: prompt tokens are forced, their logits unused), then the argmax
    const int next = si.step + 1;
    if (next < si.n_prompt) {
      __hip_atomic_store(s + 1, m.prompt[next], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(s + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      __hip_atomic_store(s + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __hip_atomic_store(s + 3, si.parity ^ 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(s + 4, si.step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// -------------------------------------------------------------- embedding
// x = token_embedding_table[token] (InferenceCore.java:68; the GPU path copies
// the fp32-converted row on the host, InferenceCore.java:586).
template <bool TAG>
__device__ inline void phase_embed(const ModelDev &m, int token, int blk, int nblk, unsigned tag = 0) {
  const int dim = m.dim;
  for (int i = blk * blockDim.x + threadIdx.x; i < dim; i += nblk * blockDim.x) {
    size_t e = (size_t)token * dim + i;
    float v;
    if (m.embd_fmt == FMT_F32) {
      v = ((const float *)m.embd.q)[e];
    } else if (m.embd_fmt == FMT_Q8) {
      v = (float)(int8_t)m.embd.q[e] * h2f(m.embd.s[e / 32]);
    } else {
      v = h2f(((const uint16_t *)m.embd.q)[e]);
    }
    if (TAG)
      st_tagged(m.txa + i, v, tag);
    else
      st_coherent(m.x + i, v);
  }
}

// ------------------------------------------------------------------ GEMV
// y = W · n(x): one wavefront computes NR rows (NR row pairs for SwiGLU) over
// its K-slice; KS waves of a workgroup split K.  Each lane owns fixed 16-byte
// chunks of every row, so its slice of x stays in registers for all rows.
// Weights stream with 128-bit non-temporal loads, are converted in registers
// (Q8_0: one sign-extending byte->float conversion per element, per 16-element
// chunk acc += s * sum(q*x); F16: exact half->float), and accumulate in fp32.
// No MFMA: batch-1 GEMV is bound by HBM bandwidth.  Latency is hidden by many
// resident waves; the first tile of a workgroup can be loaded before the grid
// barrier that precedes the phase (it does not depend on the previous phase).
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
// K must be a multiple of 4.
// Input / output access of a phase.  Plain fp32 arrays serve the per-phase
// kernels and the single-op entry points (ordered by kernel boundaries);
// tagged cells serve the persistent kernel, where each read waits for its
// producer (see TagWait).
struct InPlain {
  const float *p;
  template <int N>
  __device__ __forceinline__ void load4(const int (&e)[N], float4 (&v)[N]) const {
#pragma unroll
    for (int n = 0; n < N; ++n) v[n] = ld_coherent_f4(p, (unsigned)e[n]);
  }
};
struct InTag {
  const uint2 *p;
  unsigned tag;
  TagWait tw;
  template <int N>
  __device__ __forceinline__ void load4(const int (&e)[N], float4 (&v)[N]) const {
    ld_tagged4(p, e, tag, tw, v);
  }
};
// Outputs.  res_issue / res_finish read the residual input of a row in two
// halves, so the read can be in flight during the phase.
struct OutPlain {
  float *y;
  __device__ __forceinline__ unsigned long long res_issue(int row) const { return __float_as_uint(ld_coherent(y + row)); }
  __device__ __forceinline__ float res_finish(unsigned long long r, int) const { return __uint_as_float((unsigned)r); }
  __device__ __forceinline__ void store(int row, float v) const { st_coherent(y + row, v); }
  __device__ __forceinline__ void store_plain(int row, float v) const { y[row] = v; }
};
struct OutTag {
  uint2 *y;
  unsigned tag;
  const uint2 *rin;  // residual input cells (y = rin + W x)
  unsigned rtag;
  TagWait tw;
  __device__ __forceinline__ unsigned long long res_issue(int row) const {
    return ld_coherent_u64((const unsigned long long *)(rin + row));
  }
  __device__ __forceinline__ float res_finish(unsigned long long r, int row) const {
    return (unsigned)(r >> 32) == rtag ? __uint_as_float((unsigned)r) : ld_tagged1(rin, row, rtag, tw);
  }
  __device__ __forceinline__ void store(int row, float v) const { st_tagged(y + row, v, tag); }
  __device__ __forceinline__ void store_plain(int row, float v) const { st_tagged(y + row, v, tag); }
};
// No global output: the row values stay in the phase's LDS row buffer (obuf)
// for a following phase of the same workgroup.
struct OutNone {
  __device__ __forceinline__ unsigned long long res_issue(int) const { return 0; }
  __device__ __forceinline__ float res_finish(unsigned long long, int) const { return 0.0f; }
  __device__ __forceinline__ void store(int, float) const {}
  __device__ __forceinline__ void store_plain(int, float) const {}
};

// x staging reads exactly the float4 groups a thread owns: group u of thread t
// is elements 4 (t + (u0 + u) BS).., so a thread polls only cells that hold
// data (a padded slot would poll a cell it already read, first before its
// producer had written, costing one more round trip).  Slots past K (only when
// K is not a multiple of 4 BS) repeat element 0.
template <int N, int BS, class IN>
__device__ __forceinline__ void x_groups(const IN &x, int K, int u0, int (&e)[N], float4 (&v)[N]) {
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int i = 4 * ((int)threadIdx.x + (u0 + u) * BS);
    e[u] = i < K ? i : 0;
  }
  x.load4(e, v);
}

template <int N, int BS, class IN>
__device__ __forceinline__ void x_copy_lds(const IN &x, int K, int u0, float *xs) {
  int e[N];
  float4 v[N];
  x_groups<N, BS>(x, K, u0, e, v);
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int i = 4 * ((int)threadIdx.x + (u0 + u) * BS);
    if (i < K) *(float4 *)(xs + i) = v[u];
  }
}

// x and the norm weights wait in registers while the sum of squares is
// reduced.  With up to 2 groups per thread the weights are requested before x
// is polled (a load placed after the poll costs one more round trip); with
// more they are requested after it.  Measured per token: weights first is
// 2.3% faster at 2 groups (Llama-3.2-1B shape) and 9% slower at 4 (Llama-3.1-8B
// shape) than weights after.
template <int N, int BS, class IN>
__device__ __forceinline__ void x_norm_lds(const IN &x, const float *normw, float eps, int K, float *xs, float *red) {
  constexpr bool W_FIRST = N <= 2;
  float ss = 0.0f;
  float4 xv[N], wv[N];
  int e[N];
  if (W_FIRST) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int i = 4 * ((int)threadIdx.x + u * BS);
      wv[u] = *(const float4 *)(normw + (i < K ? i : 0));
    }
  }
  x_groups<N, BS>(x, K, 0, e, xv);
  if (!W_FIRST) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int i = 4 * ((int)threadIdx.x + u * BS);
      wv[u] = *(const float4 *)(normw + (i < K ? i : 0));
    }
  }
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int i = 4 * ((int)threadIdx.x + u * BS);
    if (i < K) {
      ss += xv[u].x * xv[u].x;
      ss += xv[u].y * xv[u].y;
      ss += xv[u].z * xv[u].z;
      ss += xv[u].w * xv[u].w;
    }
  }
  ss = block_sum<BS>(ss, red);
  ss /= (float)K;
  ss += eps;
  ss = (float)(1.0 / sqrt((double)ss));
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int i = 4 * ((int)threadIdx.x + u * BS);
    if (i < K) {
      float4 v = xv[u];
      v.x = wv[u].x * (ss * v.x);
      v.y = wv[u].y * (ss * v.y);
      v.z = wv[u].z * (ss * v.z);
      v.w = wv[u].w * (ss * v.w);
      *(float4 *)(xs + i) = v;
    }
  }
}

template <int BS, class IN>
__device__ inline void load_x_lds(const IN &x, const float *normw, float eps, int K, float *xs, float *red) {
  const int ng = (K + 4 * BS - 1) / (4 * BS);  // float4 groups per thread
  if (!normw) {
    // batches of up to 4 groups per thread, all loads of a batch issued before the first LDS write
    for (int u0 = 0; u0 < ng; u0 += 4) {
      const int r = ng - u0;
      if (r >= 4)
        x_copy_lds<4, BS>(x, K, u0, xs);
      else if (r == 3)
        x_copy_lds<3, BS>(x, K, u0, xs);
      else if (r == 2)
        x_copy_lds<2, BS>(x, K, u0, xs);
      else
        x_copy_lds<1, BS>(x, K, u0, xs);
    }
    __syncthreads();
    return;
  }
  if (ng > 4) {  // wide vectors: weights read after the reduction
    float ss = 0.0f;
    for (int i = 4 * threadIdx.x; i < K; i += 4 * BS) {
      float4 vv[1];
      const int e[1] = {i};
      x.load4(e, vv);
      const float4 v = vv[0];
      *(float4 *)(xs + i) = v;
      ss += v.x * v.x;
      ss += v.y * v.y;
      ss += v.z * v.z;
      ss += v.w * v.w;
    }
    ss = block_sum<BS>(ss, red);
    ss /= (float)K;
    ss += eps;
    ss = (float)(1.0 / sqrt((double)ss));
    for (int i = threadIdx.x; i < K; i += BS) xs[i] = normw[i] * (ss * xs[i]);
    __syncthreads();
    return;
  }
  if (ng == 4)
    x_norm_lds<4, BS>(x, normw, eps, K, xs, red);
  else if (ng == 3)
    x_norm_lds<3, BS>(x, normw, eps, K, xs, red);
  else if (ng == 2)
    x_norm_lds<2, BS>(x, normw, eps, K, xs, red);
  else
    x_norm_lds<1, BS>(x, normw, eps, K, xs, red);
  __syncthreads();
}

__device__ __forceinline__ float silu_ref(float v) { return v / (float)(1.0 + exp((double)(-v))); }

// ------------------------------------------------------------------ GEMV
// Weight tiles stream from HBM straight into LDS (buffer_load_dwordx4 ... lds:
// no registers are held while a load is in flight) through a ring of DEPTH
// slots per wave.  A slot holds SC 16-byte chunks per lane plus, for Q8_0, the
// fp16 block scales of those chunks packed per (row, gate/up) pair.
//
// The wait before a slot is read is explicit: s_waitcnt vmcnt(N) with N the
// number of loads issued after the slot's own (loads complete in issue order).
// Inside the slot loop a wave issues no other vector-memory operation (the
// results go to LDS and are written out after the loop), so N is exact.
typedef __attribute__((address_space(3))) void lds_void_t;

template <int S, int N>
__device__ __forceinline__ u32x4 *ring_w() {
  __shared__ __attribute__((aligned(16))) u32x4 a[N];
  return a;
}
template <int S, int N>
__device__ __forceinline__ unsigned *ring_s() {
  __shared__ __attribute__((aligned(16))) unsigned a[N];
  return a;
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N < 63 ? N : 63) : "memory");
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Buffer descriptor of a weight / cache region: base, stride 0, 2^31-1 bytes.
typedef int dma_rsrc_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ dma_rsrc_t rsrc(const void *p) {
  const unsigned long long b = (unsigned long long)p;
  dma_rsrc_t r;
  r.x = (int)(unsigned)b;
  r.y = (int)((unsigned)(b >> 32) & 0xffffu);
  r.z = 0x7fffffff;
  r.w = 0x00020000;
  return r;
}

// 16 (4) bytes per lane from rsrc + voff + soff into LDS at lds + 16 (4) * lane,
// nontemporal (weights and KV are read once per token).  Written as inline
// assembly on purpose: the compiler does not see these loads as LDS writes,
// so it adds no waits of its own before LDS accesses; every read of a ring
// slot is preceded by an explicit s_waitcnt on the loads issued for it, and
// every reissue into a slot by s_waitcnt lgkmcnt(0) (its reads completed).
// descriptor, LDS address and soffset are wave-uniform: read them from lane 0 into SGPRs
__device__ __forceinline__ dma_rsrc_t uniform(dma_rsrc_t r) {
  dma_rsrc_t u;
  u.x = __builtin_amdgcn_readfirstlane(r.x);
  u.y = __builtin_amdgcn_readfirstlane(r.y);
  u.z = __builtin_amdgcn_readfirstlane(r.z);
  u.w = __builtin_amdgcn_readfirstlane(r.w);
  return u;
}
__device__ __forceinline__ void dma16(dma_rsrc_t r, void *lds, unsigned voff, unsigned soff) {
  r = uniform(r);
  soff = __builtin_amdgcn_readfirstlane(soff);
  const unsigned m0v = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void_t *)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
               :
               : "s"(m0v), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}
// Same with the agent-scope sc1 bit: for the KV cache, whose rows are written
// by whichever workgroup owns the newest position and may be read by a
// workgroup of another XCD later in the same launch (L2 is per XCD).
__device__ __forceinline__ void dma16_coherent(dma_rsrc_t r, void *lds, unsigned voff, unsigned soff) {
  r = uniform(r);
  soff = __builtin_amdgcn_readfirstlane(soff);
  const unsigned m0v = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void_t *)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen sc1 nt lds"
               :
               : "s"(m0v), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(dma_rsrc_t r, void *lds, unsigned voff, unsigned soff) {
  r = uniform(r);
  soff = __builtin_amdgcn_readfirstlane(soff);
  const unsigned m0v = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void_t *)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen nt lds"
               :
               : "s"(m0v), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}

// Loads a GEMV phase may request for the phase after it once its own last
// slot has arrived (so they do not delay its waits): operator() is called at
// most once, after the wait for the last slot and before that slot's dot
// products; after(u) after the dot products of slot-load u (its ring slot may
// then take other loads).
struct NoTail {
  __device__ __forceinline__ void operator()() {}
  __device__ __forceinline__ void after(int) {}
};

// MAP 0: workgroup blk takes items blk, blk + nblk, ...; MAP 1: the items are
// split into nblk contiguous runs (the host checks that nblk divides them).
// DEPTH 4: the workgroup's slot-loads 0..3 sit in ring slots 0..3 and are all
// issued before run() (in any order, at any time the slots are free); run()
// reads them once its input is staged, which waits for every load issued
// before it.  Further slot-loads (u >= 4) reuse the slots with full waits.
template <int FMT, int KC, int KS, int NR, int MODE, int BS, int SC_ = 0, int DEPTH = 2, int MAP = 0>
struct GemvPhase {
  typedef ChunkTraits<FMT> T;
  static constexpr int EPC = T::EPC;
  static constexpr int WPB = BS / GL3_WAVE;
  static constexpr int RG = WPB / KS;                    // row groups per workgroup
  static constexpr int NP = (MODE == MODE_SWIGLU) ? 2 : 1;
  static constexpr int ROWS_PER_ITEM = RG * NR;          // output rows per work item
  static constexpr int CHUNKS = NR * NP * KC;            // 16-byte chunks per lane per item
  // ring slot size (chunks per lane), a multiple of 4
  static constexpr int SC = SC_ > 0 ? SC_ : ((CHUNKS < 8 ? CHUNKS : 8) + 3) / 4 * 4;
  static constexpr int JP = (KC < SC / (NR * NP)) ? KC : SC / (NR * NP);  // K-chunks per pass
  static constexpr int PASSES = (KC + JP - 1) / JP;      // slot loads per item
  static constexpr int WCH = WPB * SC * GL3_WAVE;        // u32x4 per slot
  static constexpr int SDW = WPB * SC * 16;              // scale dwords per slot
  static constexpr int SEG = JP * 64;                    // scale bytes per (row, pair) and pass
  static constexpr int NSI = FMT == FMT_Q8 ? (NR * NP * SEG + 255) / 256 : 0;  // scale loads per slot
  static constexpr int JMIN = KC - (PASSES - 1) * JP;    // K-chunks of the last pass
  static constexpr int NI_MIN = NR * NP * JMIN + NSI;    // fewest loads a slot takes
  static_assert(WPB % KS == 0, "K-split must divide the waves of a workgroup");
  static_assert(SC % 4 == 0 && NR * NP <= SC && JP >= 1, "ring slot too small for the rows of a wave");
  static_assert(DEPTH >= 2 && DEPTH <= 4, "ring depth");
  // x of the lane lives in registers when an item is one slot load and the
  // slice is at most 128 floats; when no norm applies and no two waves share a
  // slice, each wave loads its slice itself (no LDS staging).
  static constexpr bool XREG = PASSES == 1 && KC * EPC <= 128;
  static constexpr bool XDIRECT_OK = XREG && RG == 1;

  static __device__ __forceinline__ int elem(int K, int ks, int lane, int j) {
    return ks * (K / KS) + EPC * (lane + GL3_WAVE * j);
  }
  static __host__ __device__ __forceinline__ int items(int out_rows) {
    return (out_rows + ROWS_PER_ITEM - 1) / ROWS_PER_ITEM;
  }
  // items of workgroup blk
  static __host__ __device__ __forceinline__ int local_items(int out_rows, int blk, int nblk) {
    const int n = items(out_rows);
    if (MAP == 1) return n / nblk;
    return blk < n ? (n - 1 - blk) / nblk + 1 : 0;
  }
  // global index of the workgroup's i-th item
  static __device__ __forceinline__ int item_of(int i, int out_rows, int blk, int nblk) {
    return MAP == 1 ? blk * (items(out_rows) / nblk) + i : blk + i * nblk;
  }

  // Ring slot S (0 <= S < DEPTH) chosen at run time: the step loop is one copy
  // of code for all slots (a loop body per slot, unrolled, overflows the
  // instruction cache of the persistent kernel's layer loop).
  static __device__ __forceinline__ u32x4 *slot_w(int S) {
    u32x4 *p = ring_w<0, WCH>();
    if (S == 1) p = ring_w<1, WCH>();
    if (DEPTH >= 3 && S == 2) p = ring_w<(DEPTH >= 3 ? 2 : 0), WCH>();
    if (DEPTH == 4 && S == 3) p = ring_w<(DEPTH == 4 ? 3 : 0), WCH>();
    return p;
  }
  static __device__ __forceinline__ unsigned *slot_s(int S) {
    unsigned *p = ring_s<0, SDW>();
    if (S == 1) p = ring_s<1, SDW>();
    if (DEPTH >= 3 && S == 2) p = ring_s<(DEPTH >= 3 ? 2 : 0), SDW>();
    if (DEPTH == 4 && S == 3) p = ring_s<(DEPTH == 4 ? 3 : 0), SDW>();
    return p;
  }

  // Issues the loads of slot-load u (the workgroup's item u / PASSES, pass u % PASSES) into ring slot S.
  template <int S>
  static __device__ __forceinline__ void issue(const Mat &W, int out_rows, int u, int blk, int nblk) {
    issue_at(ring_w<S, WCH>(), ring_s<S, SDW>(), W, out_rows, u, blk, nblk);
  }
  static __device__ __forceinline__ void issue_at(u32x4 *ring, unsigned *rings, const Mat &W, int out_rows, int u,
                                                  int blk, int nblk) {
    const int wave = wave_id(), lane = lane_id();
    const int ks = wave % KS, rg = wave / KS;
    const int K = W.cols;
    const int item = item_of(u / PASSES, out_rows, blk, nblk), pass = PASSES > 1 ? u % PASSES : 0;
    const int j0 = pass * JP;
    u32x4 *rw = ring + wave * SC * GL3_WAVE;
    const dma_rsrc_t rq = rsrc(W.q);
    wait_lds();  // reads of the slot's previous contents have completed
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      int row = item * ROWS_PER_ITEM + rg * NR + r;
      row = row < out_rows ? row : out_rows - 1;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const unsigned rowoff = (unsigned)((row + p * out_rows) * K + ks * (K / KS) + j0 * GL3_WAVE * EPC) * T::ESZ;
#pragma unroll
        for (int jj = 0; jj < JP; ++jj) {
          if (PASSES > 1 && j0 + jj >= KC) break;
          dma16(rq, rw + ((r * NP + p) * JP + jj) * GL3_WAVE, 16u * lane, rowoff + jj * GL3_WAVE * 16);
        }
      }
    }
    if (FMT == FMT_Q8) {
      // scales: NR*NP segments of SEG bytes (the pass's chunks), 4 bytes per lane per load
      constexpr int TOTAL = NR * NP * SEG;
      const int valid = (PASSES > 1 && KC - j0 < JP) ? (KC - j0) * 64 : SEG;
      unsigned *rs = rings + wave * SC * 16;
      const dma_rsrc_t rsc = rsrc(W.s);
#pragma unroll
      for (int i = 0; i < NSI; ++i) {
        int b = 256 * i + 4 * lane;
        b = b < TOTAL ? b : TOTAL - 4;
        const int rp = b / SEG;
        int off = b % SEG;
        off = off < valid ? off : valid - 4;
        int row = item * ROWS_PER_ITEM + rg * NR + rp / NP;
        row = row < out_rows ? row : out_rows - 1;
        const unsigned voff = (unsigned)(row + (rp % NP) * out_rows) * (unsigned)(K / 16) + (unsigned)off;
        dma4(rsc, rs + i * GL3_WAVE, voff, (unsigned)(ks * (K / KS) / 16 + j0 * 64));
      }
    }
  }

  // Loads of the workgroup's first DEPTH slot-loads, issued ahead (e.g. while
  // the grid barrier before the phase is still open).
  static __device__ __forceinline__ void prefetch(const Mat &W, int out_rows, int blk, int nblk) {
    const int nu = local_items(out_rows, blk, nblk) * PASSES;
    if (nu > 0) issue<0>(W, out_rows, 0, blk, nblk);
    if (nu > 1) issue<1>(W, out_rows, 1, blk, nblk);
    if (DEPTH >= 3 && nu > 2) issue<(DEPTH >= 3 ? 2 : 1)>(W, out_rows, 2, blk, nblk);
    if (DEPTH == 4 && nu > 3) issue<(DEPTH == 4 ? 3 : 1)>(W, out_rows, 3, blk, nblk);
  }

  struct XSlice {
    float r[XREG ? KC : 1][XREG ? EPC : 1];
    const float *lds;
    int e0;
    __device__ __forceinline__ float get(int j, int i) const {
      return XREG ? r[XREG ? j : 0][XREG ? i : 0] : lds[e0 + GL3_WAVE * EPC * j + i];
    }
  };

  // acc[r][p] += the lane's part of the dot products held in ring slot (ring, rings) (pass `pass` of the item)
  static __device__ __forceinline__ void dot_at(const u32x4 *ring, const unsigned *rings, const XSlice &xr, int pass,
                                                float (&acc)[NR][NP]) {
    const int wave = wave_id(), lane = lane_id();
    const u32x4 *rw = ring + wave * SC * GL3_WAVE + lane;
    const uint8_t *rs = (const uint8_t *)(rings + wave * SC * 16);
    const int j0 = pass * JP;
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        float a = acc[r][p];
#pragma unroll
        for (int jj = 0; jj < JP; ++jj) {
          if (PASSES > 1 && j0 + jj >= KC) break;
          const int c = (r * NP + p) * JP + jj;
          const int j = PASSES > 1 ? j0 + jj : jj;
          const u32x4 w = rw[c * GL3_WAVE];
          const unsigned ww[4] = {w.x, w.y, w.z, w.w};
          if (FMT == FMT_Q8) {
            const float sc = h2f(*(const uint16_t *)(rs + (r * NP + p) * SEG + ((lane + GL3_WAVE * jj) & ~1)));
            float cacc = 0.0f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              cacc = fmaf(sbyte<0>(ww[d]), xr.get(j, 4 * d + 0), cacc);
              cacc = fmaf(sbyte<1>(ww[d]), xr.get(j, 4 * d + 1), cacc);
              cacc = fmaf(sbyte<2>(ww[d]), xr.get(j, 4 * d + 2), cacc);
              cacc = fmaf(sbyte<3>(ww[d]), xr.get(j, 4 * d + 3), cacc);
            }
            a = fmaf(sc, cacc, a);
          } else {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              a = fmaf(h2f_lo(ww[d]), xr.get(j, 2 * d + 0), a);
              a = fmaf(h2f_hi(ww[d]), xr.get(j, 2 * d + 1), a);
            }
          }
        }
        acc[r][p] = a;
      }
  }

  // Reduces and combines the K-split partials of the workgroup's i-th item;
  // the row values go to obuf[i * ROWS_PER_ITEM + row in item] (MODE_SWIGLU:
  // the gate there and the up value in ubuf, combined after the last item).
  static __device__ __forceinline__ void finish_item(int i, float (&acc)[NR][NP], float *kpart, float *obuf,
                                                     float *ubuf) {
    const int wave = wave_id(), lane = lane_id();
    const int ks = wave % KS, rg = wave / KS;
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
    if (ks == 0 && lane < NR) {
      float a0 = acc[0][0], a1 = acc[0][NP - 1];
#pragma unroll
      for (int r = 1; r < NR; ++r)
        if (lane == r) {
          a0 = acc[r][0];
          a1 = acc[r][NP - 1];
        }
      obuf[i * ROWS_PER_ITEM + rg * NR + lane] = a0;
      if (MODE == MODE_SWIGLU) ubuf[i * ROWS_PER_ITEM + rg * NR + lane] = a1;
    }
  }

  template <class TAIL>
  static __device__ __forceinline__ void step(const Mat &W, int out_rows, int u, int nu, int blk, int nblk,
                                              const XSlice &xr, float (&acc)[NR][NP], float *kpart, float *obuf,
                                              float *ubuf, TAIL &tail) {
    const int S = u % DEPTH;
    // slot S is complete once at most the loads of the (up to DEPTH-1) later slot-loads are outstanding
    const int later = nu - 1 - u;
    if (DEPTH == 4) {
      // slot-loads 0..3 completed before the input was staged; later ones are waited for in full
      if (u >= DEPTH) wait_vmem<0>();
      if (later == 0) tail();
    } else if (DEPTH == 3 && later >= 2)
      wait_vmem<2 * NI_MIN>();
    else if (later >= 1)
      wait_vmem<NI_MIN>();
    else {
      wait_vmem<0>();
      tail();
    }
    const int pass = PASSES > 1 ? u % PASSES : 0;
    u32x4 *rw = slot_w(S);
    unsigned *rs = slot_s(S);
    dot_at(rw, rs, xr, pass, acc);
    tail.after(u);
    if (u + DEPTH < nu) issue_at(rw, rs, W, out_rows, u + DEPTH, blk, nblk);
    if (PASSES == 1 || pass == PASSES - 1) {
      finish_item(u / PASSES, acc, kpart, obuf, ubuf);
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int p = 0; p < NP; ++p) acc[r][p] = 0.0f;
    }
  }

  // LDS layout of a phase: [x (K floats, when staged)] [red 32] [kpart] [obuf] [best keys | SwiGLU up values]
  static __host__ __device__ constexpr int kpart_floats() { return RG * NR * NP * KS; }
  // float offset of obuf (the workgroup's row values, in local item order) in the phase's LDS
  static __host__ __device__ __forceinline__ int obuf_offset(int K, bool has_norm) {
    return (staged(has_norm) ? K : 0) + 32 + kpart_floats();
  }
  static __host__ __device__ __forceinline__ bool staged(bool has_norm) { return !(XDIRECT_OK && !has_norm); }
  static __host__ __device__ __forceinline__ size_t lds_bytes(int K, int out_rows, int nblk, bool has_norm) {
    const int lr = local_items(out_rows, 0, nblk) * ROWS_PER_ITEM;
    return (size_t)((staged(has_norm) ? K : 0) + 32 + kpart_floats() + (MODE == MODE_SWIGLU ? 2 : 1) * lr + 2 * WPB +
                    4) * sizeof(float);
  }

  // Runs the phase.  x: input vector (K floats, coherent); normw: RMSNorm
  // weights or nullptr; y: output (MODE_RESIDUAL: y += W n(x)); for
  // MODE_LOGITS, y gets the rows and best_out[blk] the argmax key of the rows
  // this workgroup produced.  prefetched: prefetch() was already called with
  // the same W, out_rows, blk and nblk.  tail: requests for a following phase,
  // made once, when the last weight slot has arrived (see NoTail).
  template <class IN, class OUT, class TAIL = NoTail>
  static __device__ void run(const Mat &W, int out_rows, const IN &x, const float *normw, float eps, const OUT &y,
                             unsigned long long *best_out, int blk, int nblk, float *lds, bool prefetched = false,
                             TAIL tail = TAIL{}) {
    const int K = W.cols;
    const bool stg = staged(normw != nullptr);
    float *xs = lds;                          // K floats when staged
    float *red = lds + (stg ? K : 0);         // reduction scratch (32 floats)
    float *kpart = red + 32;                  // cross-wave partials
    float *obuf = kpart + kpart_floats();     // row values of the workgroup's items
    const int nli = local_items(out_rows, blk, nblk);
    float *ubuf = obuf + nli * ROWS_PER_ITEM;  // MODE_SWIGLU: up values of the same rows
    const int nu = nli * PASSES;
    if (!prefetched) prefetch(W, out_rows, blk, nblk);

    const int wave = wave_id(), lane = lane_id();
    const int ks = wave % KS;
    // residual input of the first BS local rows, read while the phase runs
    const int nlr = nli * ROWS_PER_ITEM;
    const int row0 = item_of((int)threadIdx.x / ROWS_PER_ITEM, out_rows, blk, nblk) * ROWS_PER_ITEM +
                     (int)threadIdx.x % ROWS_PER_ITEM;
    unsigned long long res0 = 0;
    if (MODE == MODE_RESIDUAL && (int)threadIdx.x < nlr && row0 < out_rows) res0 = y.res_issue(row0);
    XSlice xr;
    xr.lds = xs;
    xr.e0 = elem(K, ks, lane, 0);
    if (!stg) {
      if (XDIRECT_OK) {
        constexpr int NV = XDIRECT_OK ? KC * EPC / 4 : 1;
        int e[NV];
        float4 v[NV];
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
          for (int i = 0; i < EPC; i += 4) e[XDIRECT_OK ? j * (EPC / 4) + i / 4 : 0] = elem(K, ks, lane, j) + i;
        x.load4(e, v);
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
          for (int i = 0; i < EPC; i += 4) {
            const float4 w = v[XDIRECT_OK ? j * (EPC / 4) + i / 4 : 0];
            xr.r[j][i] = w.x;
            xr.r[j][i + 1] = w.y;
            xr.r[j][i + 2] = w.z;
            xr.r[j][i + 3] = w.w;
          }
      }
    } else {
      load_x_lds<BS>(x, normw, eps, K, xs, red);
      if (XREG) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
          const int e = elem(K, ks, lane, j);
#pragma unroll
          for (int i = 0; i < EPC; i += 4) {
            float4 v = *(const float4 *)(xs + e + i);
            xr.r[j][i] = v.x;
            xr.r[j][i + 1] = v.y;
            xr.r[j][i + 2] = v.z;
            xr.r[j][i + 3] = v.w;
          }
        }
      }
    }

    // DEPTH 4: the preloaded slots were issued before the input reads, so this wait is already met
    if (DEPTH == 4) wait_vmem<0>();
    float acc[NR][NP];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int p = 0; p < NP; ++p) acc[r][p] = 0.0f;
#pragma unroll 1
    for (int u = 0; u < nu; ++u) step(W, out_rows, u, nu, blk, nblk, xr, acc, kpart, obuf, ubuf, tail);
    if (MODE == MODE_SWIGLU && ks == 0) {
      // silu(gate) * up for the rows this wave finished, one lane per row: the
      // double-precision exp runs once per wave, not once per item (a lone wave
      // per SIMD waits out its whole latency each time)
      const int rg = wave / KS;
      for (int q = lane; q < nli * NR; q += GL3_WAVE) {
        const int o = (q / NR) * ROWS_PER_ITEM + rg * NR + q % NR;
        obuf[o] = silu_ref(obuf[o]) * ubuf[o];
      }
    }
    __syncthreads();

    // write the rows out (coalesced over the workgroup's items)
    unsigned long long best = 0;
    for (int lr = threadIdx.x; lr < nlr; lr += BS) {
      const int row = item_of(lr / ROWS_PER_ITEM, out_rows, blk, nblk) * ROWS_PER_ITEM + lr % ROWS_PER_ITEM;
      if (row < out_rows) {
        const float v = obuf[lr];
        if (MODE == MODE_RESIDUAL) {
          const unsigned long long r = lr == (int)threadIdx.x ? res0 : y.res_issue(row);
          y.store(row, y.res_finish(r, row) + v);
        } else if (MODE == MODE_LOGITS) {
          y.store_plain(row, v);
          const unsigned long long k = argmax_key(v, row);
          best = k > best ? k : best;
        } else {
          y.store(row, v);
        }
      }
    }
    if (MODE == MODE_LOGITS) {
      unsigned long long *bred = (unsigned long long *)(obuf + nli * ROWS_PER_ITEM + 1);
      bred = (unsigned long long *)(((uintptr_t)bred + 7) & ~(uintptr_t)7);
      for (int o = 32; o >= 1; o >>= 1) {
        unsigned long long other = __shfl_xor(best, o);
        best = other > best ? other : best;
      }
      if (lane == 0) bred[wave] = best;
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned long long b = 0;
        for (int w = 0; w < WPB; ++w) b = bred[w] > b ? bred[w] : b;
        __hip_atomic_store(best_out + blk, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();  // LDS is reused by the next phase
  }
};

// Quiet wait of a workgroup that reaches a phase long before its input: wave 0
// polls one cell per producer (cells base[i * stride + last], i < count <= 256:
// each producer's last store), with long sleeps between rounds, until all
// carry the tag; the phase's staging then reads the whole input as usual (and
// still checks every cell).  Keeps waiting workgroups from polling the whole
// vector for microseconds while the fabric carries other traffic: measured
// +2.8% tokens/s on the Llama-3.2-1B Q8_0 shape for the workgroups without an
// attention item.  Only for waits off the critical path: before the reduce of
// the fused FFN (every workgroup waits there for the slowest) it cost 5%.
__device__ __forceinline__ void quiet_wait(const uint2 *base, int stride, int last, int count, unsigned tag,
                                           const TagWait &tw) {
  if (threadIdx.x < GL3_WAVE) {
    const int lane = threadIdx.x;
    int e[4];
    bool act[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = lane + j * GL3_WAVE;
      act[j] = i < count;
      e[j] = (act[j] ? i : 0) * stride + last;
    }
    unsigned spins = 0;
    for (;;) {
      bool ok = true;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (act[j]) {
          const unsigned long long w = ld_coherent_u64((const unsigned long long *)(base + e[j]));
          if ((unsigned)(w >> 32) == tag) act[j] = false;
          else ok = false;
        }
      if (__all(ok)) break;
      ++spins;
      if (spins > tw.spin_limit || ld_coherent_u32(tw.err) != 0u) break;  // the staging wait reports it
      __builtin_amdgcn_s_sleep(8);
    }
  }
  __syncthreads();
}

// ------------------------------------------------- fused FFN (down slices)
// When every workgroup owns 32 consecutive SwiGLU rows (one Q8_0 block of the
// down projection's K), it multiplies them by its 32-column slice of Wdown
// right away: 2048-row partial sums, no SwiGLU vector exchanged between
// workgroups.  The slice is stored contiguously ([slice][row][32] quants,
// [slice][row] scales), streamed through the ring as 1024-row slot-loads
// (8 KB of quants and 512 B of scales per wave).  A reduce phase then sums
// the partials of each row in a fixed order.
template <int BS, int DEPTH>
struct DownSliceQ8 {
  static constexpr int WPB = BS / GL3_WAVE;
  static constexpr int RPU = WPB * 256;             // rows per slot-load (256 per wave)
  static constexpr int WCH = WPB * 8 * GL3_WAVE;    // u32x4 per ring slot (same ring as the GEMV phases)
  static constexpr int SDW = WPB * 8 * 16;          // scale dwords per ring slot
  static constexpr int NI = 8 + 2;                  // loads per wave per slot-load
  static_assert(WPB == 4, "four waves");

  static __device__ __forceinline__ int units(int rows) { return rows / RPU; }

  // slot-load u (rows [u RPU, (u + 1) RPU)) of slice `slice` into ring slot S
  template <int S>
  static __device__ __forceinline__ void issue(const Mat &W, int rows, int slice, int u) {
    const int wave = wave_id(), lane = lane_id();
    const int r0 = u * RPU + wave * 256;
    u32x4 *rw = ring_w<S, WCH>() + wave * 8 * GL3_WAVE;
    unsigned *rs = ring_s<S, SDW>() + wave * 8 * 16;
    const dma_rsrc_t rq = rsrc(W.q), rsc = rsrc(W.s);
    wait_lds();
    const unsigned qoff = (unsigned)(((size_t)slice * rows + r0) * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) dma16(rq, rw + i * GL3_WAVE, 16u * lane, qoff + i * 1024u);
    const unsigned soff = (unsigned)(((size_t)slice * rows + r0) * 2);
#pragma unroll
    for (int i = 0; i < 2; ++i) dma4(rsc, rs + i * GL3_WAVE, 4u * lane, soff + i * 256u);
  }

  // Partial sums of the wave's 256 rows of the slot-load held in slot S: lane l
  // takes half l % 2 of rows 32 c + l / 2 (hv = its 16 SwiGLU values); pv[c]
  // gets row 32 c + l / 2 in both lanes of the pair.
  template <int S>
  static __device__ __forceinline__ void compute(const float (&hv)[16], float (&pv)[8]) {
    const int wave = wave_id(), lane = lane_id();
    const u32x4 *rw = ring_w<S, WCH>() + wave * 8 * GL3_WAVE + lane;
    const uint16_t *rs = (const uint16_t *)(ring_s<S, SDW>() + wave * 8 * 16);
    u32x4 w[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) w[c] = rw[c * GL3_WAVE];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const unsigned ww[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
      float a = 0.0f;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        a = fmaf(sbyte<0>(ww[d]), hv[4 * d + 0], a);
        a = fmaf(sbyte<1>(ww[d]), hv[4 * d + 1], a);
        a = fmaf(sbyte<2>(ww[d]), hv[4 * d + 2], a);
        a = fmaf(sbyte<3>(ww[d]), hv[4 * d + 3], a);
      }
      // the two halves of the row: lanes l and l ^ 1 (low half first)
      const float o = __shfl_xor(a, 1);
      const float blk = (lane & 1) ? o + a : a + o;
      pv[c] = h2f(rs[c * 32 + lane / 2]) * blk;
    }
  }

  // The whole phase for dim = 2 RPU: slot-loads 0 and 1 were issued by prefetch.
  static __device__ __forceinline__ void prefetch(const Mat &W, int rows, int slice) {
    issue<0>(W, rows, slice, 0);
    issue<1>(W, rows, slice, 1);
  }
  // SA, SB: the ring slots holding the first and the second slot-load
  template <int SA = 0, int SB = 1>
  static __device__ __forceinline__ void run(int rows, const float *hb_lds, uint2 *dst, unsigned tag) {
    const int lane = lane_id();
    float hv[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 v = *(const float4 *)(hb_lds + 16 * (lane & 1) + i);
      hv[i] = v.x;
      hv[i + 1] = v.y;
      hv[i + 2] = v.z;
      hv[i + 3] = v.w;
    }
    static_assert(DEPTH == 2, "two ring slots");
    const int wave = wave_id();
    // two slot-loads (dim 2048); stores only after both, so the waits count loads alone
    float p0[8], p1[8];
    wait_vmem<NI>();
    compute<SA>(hv, p0);
    wait_vmem<0>();
    compute<SB>(hv, p1);
    if ((lane & 1) == 0) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        st_tagged(dst + wave * 256 + c * 32 + lane / 2, p0[c], tag);
        st_tagged(dst + RPU + wave * 256 + c * 32 + lane / 2, p1[c], tag);
      }
    }
  }
};

// Reduce of the down partials: workgroup v owns rows [v R, (v + 1) R) with
// R = dim / nblk (<= 8): out[row] = res[row] + sum_w part[w][row], the sum over
// w = 0 .. nblk-1 in a fixed order (per-lane partial sums of 8 rows, then a
// wave tree, then the 4 waves in order).
template <int BS>
__device__ __forceinline__ void phase_reduce(const uint2 *part, int dim, const uint2 *res, unsigned rtag, uint2 *out,
                                             unsigned tag, unsigned ptag, const TagWait &tw, int blk, int nblk,
                                             float *lds) {
  constexpr int WPB = BS / GL3_WAVE;
  const int R = dim / nblk;
  const int row0 = blk * R;
  const int wave = wave_id(), lane = lane_id();
  // residual input of the workgroup's rows, requested before the partials are
  // polled (it was written a phase earlier and is normally ready)
  const unsigned long long res_w =
      (int)threadIdx.x < R ? ld_coherent_u64((const unsigned long long *)(res + row0 + threadIdx.x)) : 0ull;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int w = threadIdx.x; w < nblk; w += BS) {
    // R consecutive cells of workgroup w's partials (R <= 8, row0 a multiple of R)
    const uint2 *src = part + (size_t)w * dim + row0;
    if (R == 8) {
      const int e[2] = {w * dim + row0, w * dim + row0 + 4};  // uniform base, per-lane offsets
      float4 v[2];
      ld_tagged4(part, e, ptag, tw, v);
      acc[0] += v[0].x;
      acc[1] += v[0].y;
      acc[2] += v[0].z;
      acc[3] += v[0].w;
      acc[4] += v[1].x;
      acc[5] += v[1].y;
      acc[6] += v[1].z;
      acc[7] += v[1].w;
    } else {
      for (int i = 0; i < R; ++i) acc[i] += ld_tagged1(src, i, ptag, tw);
    }
  }
  float *red = lds;  // [WPB][8]
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = wave_sum(acc[i]);
    if (lane == 0) red[wave * 8 + i] = t;
  }
  __syncthreads();
  if ((int)threadIdx.x < R) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < WPB; ++w) t += red[w * 8 + threadIdx.x];
    const int row = row0 + threadIdx.x;
    const float r = (unsigned)(res_w >> 32) == rtag ? __uint_as_float((unsigned)res_w) : ld_tagged1(res, row, rtag, tw);
    st_tagged(out + row, r + t, tag);
  }
  __syncthreads();
}

// -------------------------------------------------------------- attention
// Flash-decode over the fp16 KV cache on the matrix cores.  Work item = (kv
// head, split of positions); the workgroup serves the GQ query heads of the kv
// head's GQA group, so each K/V element is read from HBM once per group.
//
// The split is cut into tiles of 16 positions; wave w takes tiles w, w+4, ...
// A tile's K rows ([16][hd], contiguous in the cache) and V columns (the V
// cache is stored in 16-position blocks, each transposed to [hd][16], so a
// tile's V is one contiguous 2*16*hd-byte block) stream into the per-wave LDS
// ring of the GEMV phases by DMA, DEPTH tiles ahead.  Per tile:
//   S[16 pos][16 heads] = K[16][hd] . Q^T    v_mfma_f32_16x16x32_f16
//   online softmax over the tile (scores / sqrt(hd), InferenceCore.java:114-121)
//   O[16 heads][hd]    += P[16][16] . V     v_mfma_f32_16x16x16_f16
// q and p are fp32: each is split into fp16 hi + lo parts (hi = fp16(x),
// lo = fp16(x - hi)) and both products are accumulated, so the scores and
// outputs carry ~22 significant bits of q and p (K and V are exactly fp16).
// Heads beyond GQ are zero columns.  The four waves merge through LDS, the
// splits of a kv head by log-sum-exp in the workgroup that finishes last.
//
// q (and, in the split holding `pos`, the new k and v) are read straight into
// registers together with their RoPE partners and table entries (one round
// trip); Qwen3's per-head RMSNorm is a sum over the 4 lanes holding a head
// (InferenceCore.java:341-347), RoPE follows InferenceCore.java:82-100 / :472-491.

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define ATT_DEPTH 3  // K/V ring slots per wave (2 or 3; a shape may choose 2 to free LDS)
#define ATT_RING_U4 (4 * 8 * GL3_WAVE)  // default ring slot (4 waves x 8 KB), in u32x4

__device__ __forceinline__ void rope_pair(float &v0, float &v1, float c, float s) {
  float a = v0 * c - v1 * s;
  float b = v0 * s + v1 * c;
  v0 = a;
  v1 = b;
}

// Positions per split: a multiple of 64 (16-position tiles x 4 waves).
__host__ __device__ __forceinline__ int att_split_len(int n, int max_split, int step) {
  int s = (n + max_split - 1) / max_split;
  s = (s + step - 1) / step * step;
  return s < step ? step : s;
}

// LDS floats of the attention phase: per-wave o [wpb][G][hd], (m, l) [wpb][G][2], a flag
// (16 floats), the staged q [G][hd], new k [hd] and new v [hd] twice (as read and
// normed; prepared) and their per-group sums of squares.
__host__ __device__ __forceinline__ int att_lds_floats(int hd, int G, int wpb, int max_split) {
  (void)max_split;
  return wpb * G * (hd + 2) + 16 + 2 * (G + 2) * hd + (G + 2) * hd / 4;
}

__device__ __forceinline__ void f4_to(float *dst, float4 v) {
  dst[0] = v.x;
  dst[1] = v.y;
  dst[2] = v.z;
  dst[3] = v.w;
}

// Rotation of the K tile's 16-byte chunks inside a row, chosen so that the 16
// rows read by one MFMA operand load fall in distinct LDS bank groups.
template <int NQ>
__device__ __forceinline__ int kswz(int pos) {
  return NQ == 16 ? pos : (NQ == 8 ? (pos >> 1) : (pos >> 2));
}

__device__ __forceinline__ float inv_rms(float ss, int hd, float eps) {
  ss /= (float)hd;
  ss += eps;
  return (float)(1.0 / sqrt((double)ss));
}

// One wave's share of a (kv head, split) item: tile DMA and tile compute.  The
// ring slot is a template parameter so that each slot is its own LDS object and
// the compiler's own wait counts do not serialize the slots.
// RU4: ring slot size in u32x4 (the GEMV phases' slot in the persistent
// kernel, so both use one ring); a wave's tile needs 4 hd of them.
template <int HD, int GQ, int RU4, int AD = ATT_DEPTH>
struct AttTile {
  static_assert(RU4 >= 16 * HD, "ring slot too small for a K/V tile per wave");
  static constexpr int NQ = HD / 8, NC = HD / 32, NB = HD / 16, NKI = HD / 32, NVI = HD / 32, NI = NKI + NVI;
  static constexpr int KT_U4 = 16 * NQ;
  const ModelDev *m;
  dma_rsrc_t rk, rv;
  int t0, t1, pos, wave, lane;

  template <int S>
  __device__ __forceinline__ u32x4 *slot() const {
    return ring_w<S, RU4>() + wave * (RU4 / 4);
  }

  // DMA of this wave's u-th tile (positions t0 + 16 (wave + 4u) ..) into ring slot S.
  // FIRST: the slot has no reads pending (the start of an item, after a
  // workgroup barrier), so no LDS wait, which would also wait for scalar loads.
  template <int S, bool FIRST = false>
  __device__ __forceinline__ void issue(int u) const {
    const int t = t0 + 16 * (wave + 4 * u);
    u32x4 *sl = slot<S>();
    if (!FIRST) wait_lds();
#pragma unroll
    for (int i = 0; i < NKI; ++i) {
      const int ci = GL3_WAVE * i + lane, p = ci / NQ;
      int q = ci % NQ - kswz<NQ>(p);
      q = q < 0 ? q + NQ : q;
      dma16_coherent(rk, sl + GL3_WAVE * i, (unsigned)(((t + p) * HD + 8 * q) * 2), 0u);
    }
#pragma unroll
    for (int i = 0; i < NVI; ++i) {
      const int d = 32 * i + lane / 2;
      dma16_coherent(rv, sl + KT_U4 + GL3_WAVE * i, (unsigned)((t * HD + 16 * d + 8 * (lane % 2)) * 2), 0u);
    }
  }

  template <int S>
  __device__ __forceinline__ void step(int u, int ntw, const half8 (&qh)[NC], const half8 (&ql)[NC],
                                       const unsigned (&knb)[4], const unsigned (&vnb)[4], f32x4 (&O)[NB],
                                       float &mrun, float &lrun) const {
    if (u >= ntw) return;
    // slot S is complete once at most the loads of the later issued tiles are
    // outstanding: min(later, AD - 1) tiles
    const int later = ntw - 1 - u;
    if (AD >= 3 && later >= 2)
      wait_vmem<2 * NI>();
    else if (later >= 1)
      wait_vmem<NI>();
    else
      wait_vmem<0>();
    tile<S>(u, qh, ql, knb, vnb, O, mrun, lrun);
    if (u + AD < ntw) issue<S>(u + AD);
  }

  template <int S>
  __device__ __forceinline__ void tile(int u, const half8 (&qh)[NC], const half8 (&ql)[NC], const unsigned (&knb)[4],
                                       const unsigned (&vnb)[4], f32x4 (&O)[NB], float &mrun, float &lrun) const {
    u32x4 *sl = slot<S>();
    const int hh = lane % 16, kb = lane / 16;
    const int t = t0 + 16 * (wave + 4 * u);
    const int nvalid = min(16, t1 - t);
    // all LDS reads of the tile first: K chunks (MFMA A operand: row hh, dims
    // 32c + 8kb..) and V^T rows 16b + hh, positions 4kb..4kb+3 (B operand)
    u32x4 kw[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int q = 4 * c + kb;
      kw[c] = sl[hh * NQ + (q + kswz<NQ>(hh)) % NQ];
    }
    const uint2 *vt2 = (const uint2 *)(sl + KT_U4);
    uint2 vw[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) vw[b] = vt2[(16 * b + hh) * 4 + kb];
    // The row of the new position is stale in the tile (the DMA may have read
    // the cache before the append): its K chunks and V entries are replaced in
    // registers from the lanes holding the new k, v (lane i: dims 8i..8i+7).
    // The tile is only read, never written, so the slots stay independent.
    if (__builtin_expect(pos >= t && pos < t + 16, 0)) {
      const int pl = pos - t;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int q = 4 * c + kb;
        const u32x4 kn = u32x4{(unsigned)__shfl((int)knb[0], q), (unsigned)__shfl((int)knb[1], q),
                               (unsigned)__shfl((int)knb[2], q), (unsigned)__shfl((int)knb[3], q)};
        if (hh == pl) kw[c] = kn;
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int d = 16 * b + hh, src = d / 8;  // the new v of dim d: lane d/8, element d%8
        const unsigned w0 = (unsigned)__shfl((int)vnb[0], src), w1 = (unsigned)__shfl((int)vnb[1], src);
        const unsigned w2 = (unsigned)__shfl((int)vnb[2], src), w3 = (unsigned)__shfl((int)vnb[3], src);
        const int e = d % 8;
        const unsigned word = e < 2 ? w0 : (e < 4 ? w1 : (e < 6 ? w2 : w3));
        const unsigned h16 = (word >> (16 * (e % 2))) & 0xffffu;
        if (pl / 4 == kb) {
          const int j = pl % 4;
          if (j == 0) vw[b].x = (vw[b].x & 0xffff0000u) | h16;
          if (j == 1) vw[b].x = (vw[b].x & 0x0000ffffu) | (h16 << 16);
          if (j == 2) vw[b].y = (vw[b].y & 0xffff0000u) | h16;
          if (j == 3) vw[b].y = (vw[b].y & 0x0000ffffu) | (h16 << 16);
        }
      }
    }
    // scores S[pos][head] = K . Q^T
    f32x4 sacc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const half8 a = __builtin_bit_cast(half8, kw[c]);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[c], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[c], sacc, 0, 0, 0);
    }
    // lane: head hh, positions 4*kb + v
    float sv[4];
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const bool ok = hh < GQ && 4 * kb + v < nvalid;
      sv[v] = ok ? sacc[v] / m->sqrt_hd : -INFINITY;
      mx = fmaxf(mx, sv[v]);
    }
    mx = xrow_max(mx);
    const float mn = fmaxf(mrun, mx);
    const float cf = (mrun == -INFINITY) ? 0.0f : __expf(mrun - mn);
    float p4[4], ls = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      p4[v] = (sv[v] == -INFINITY) ? 0.0f : __expf(sv[v] - mn);
      ls += p4[v];
    }
    ls = xrow_sum(ls);
    if (mn != -INFINITY) {
      lrun = lrun * cf + ls;
      mrun = mn;
    }
    // O rows are heads 4*kb + v (kb < 2 for GQ <= 8): their rescale factors
    // live in lanes 4*kb + v; rows of heads >= GQ hold zeros
    float cr[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float cv = readlane_f(cf, v), mv = readlane_f(mn, v);
      if (GQ > 4 && kb == 1) {
        cv = readlane_f(cf, 4 + v);
        mv = readlane_f(mn, 4 + v);
      }
      cr[v] = (mv == -INFINITY) ? 1.0f : cv;
    }
    half4 ph, plo;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const _Float16 h16 = (_Float16)p4[v];
      ph[v] = h16;
      plo[v] = (_Float16)(p4[v] - (float)h16);
    }
    // positions >= nvalid of a partial tile read zeros (p is 0 there too)
    const unsigned keep0 = (4 * kb + 0 < nvalid ? 0x0000ffffu : 0u) | (4 * kb + 1 < nvalid ? 0xffff0000u : 0u);
    const unsigned keep1 = (4 * kb + 2 < nvalid ? 0x0000ffffu : 0u) | (4 * kb + 3 < nvalid ? 0xffff0000u : 0u);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int v = 0; v < 4; ++v) O[b][v] *= cr[v];
      uint2 w = vw[b];
      w.x &= keep0;
      w.y &= keep1;
      const half4 vb = __builtin_bit_cast(half4, w);
      O[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vb, O[b], 0, 0, 0);
      O[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo, vb, O[b], 0, 0, 0);
    }
  }
};

// q, k, v come from m.qkv (plain) or from the tagged cells m.tqkv (TAG, cells
// written with tag_in); the output goes to m.att or, with tag_out, to m.tatt.
// Splits per kv head of the attention phase inside the persistent kernel (n
// positions): at most one item per workgroup and 64 splits per head.  With the
// fused FFN, whose workgroups without an item request gate/up's weights during
// attention, at most half the workgroups hold an item once a split would pass
// 48 positions (Llama-3.2-1B Q8_0: -1.3% / -2.5% time per token at positions
// 1728 / 2016; halving at every length costs +1.3% at 1152).
__device__ __forceinline__ int att_tag_splits(const ModelDev &m, int n, int nblk, bool fused) {
  int ms = max(1, min(min(m.max_split, 64), nblk / m.n_kv));
  if (fused && n > 48 * ms) ms = max(1, ms / 2);
  return ms;
}

template <int HD, int GQ, int BS, bool TAG, int RU4 = ATT_RING_U4, int AD = ATT_DEPTH, class PM = NoTail>
__device__ void phase_attention(const ModelDev &m, int layer, int pos, int blk, int nblk, float *lds,
                                unsigned tag_in = 0, unsigned tag_out = 0, TagWait tw = TagWait{nullptr, 0},
                                int tk = -1, PM pm = PM{}, int msplit_tag = 0) {
  constexpr int WPB = BS / GL3_WAVE;
  constexpr int NQ = HD / 8;           // 16-byte chunks of a K row
  constexpr int NC = HD / 32;          // 32-dim chunks (score MFMAs per tile and hi/lo)
  constexpr int NB = HD / 16;          // 16-dim blocks of the output
  static_assert(WPB == 4 && HD % 32 == 0 && HD <= 128 && GQ <= 8, "attention tile shape");
  const int hd = HD, half = HD / 2;
  const int n = pos + 1;
  // tagged merge: at most one item per workgroup (the caller's split count)
  const int msplit = TAG ? (msplit_tag > 0 ? msplit_tag : att_tag_splits(m, n, nblk, false)) : m.max_split;
  const int S = att_split_len(n, msplit, 16 * WPB);
  const int nsplit = (n + S - 1) / S;
  const int items = m.n_kv * nsplit;
  const int hpart = hd + 4;
  float *opart = lds;                     // per-wave o [WPB][GQ][hd]
  float *mlp = opart + WPB * GQ * hd;     // per-wave (m, l) [WPB][GQ][2]
  int *flag = (int *)(mlp + WPB * GQ * 2);
  float *qst = mlp + WPB * GQ * 2 + 16;   // staged q [GQ][hd], new k [hd], new v [hd] (normed, before RoPE)
  float *qrot = qst + (GQ + 2) * HD;      // the same, prepared (normed and rotated)
  float *ssb = qrot + (GQ + 2) * HD;      // per-group sums of squares [(GQ + 2) * hd / 4]
  const LayerDev L = ld_layer(m.layers, layer);
  const int wave = wave_id(), lane = lane_id();
  const int hh = lane % 16, kb = lane / 16;  // MFMA column (head) and k-block of this lane
  const bool neox = m.family != FAM_LLAMA, qwen = m.family == FAM_QWEN3;

  // phase trace (tk >= 0): stamps tk when q/k/v have been read and tk + 1 when
  // the tiles are done (a workgroup without an item stamps both on its way out)
  if (tk >= 0 && blk >= items) {
    trace(m, tk);
    trace(m, tk + 1);
  }
  for (int item = blk; item < items; item += nblk) {
    const int kvh = item / nsplit, sp = item % nsplit;
    const int t0 = sp * S, t1 = min(n, t0 + S);
    const bool owns_pos = (pos >= t0 && pos < t1);
    const int ntile = (t1 - t0 + 15) / 16;
    const int ntw = wave < ntile ? (ntile - 1 - wave) / WPB + 1 : 0;  // tiles of this wave
    uint16_t *kbase = m.kc + ((size_t)layer * m.n_kv + kvh) * m.ctxp * HD;
    uint16_t *vbase = m.vc + ((size_t)layer * m.n_kv + kvh) * HD * m.ctxp;
    const dma_rsrc_t rk = rsrc(kbase), rv = rsrc(vbase);

    AttTile<HD, GQ, RU4, AD> at;
    at.m = &m;
    at.rk = rk;
    at.rv = rv;
    at.t0 = t0;
    at.t1 = t1;
    at.pos = pos;
    at.wave = wave;
    at.lane = lane;
    // only the first tile goes out before q is polled: reads return in issue
    // order per CU, so every tile requested ahead of the poll delays q (and the
    // ring, full, cannot take more); the next tiles follow once q is in
    if (ntw > 0) at.template issue<0, true>(0);

    // ---- q of the GQ heads and, in the split holding pos, the new k and v:
    // read once per workgroup (one float4 of tagged cells per staging thread,
    // all reads in one round trip) and prepared there, once: Qwen3's per-head
    // RMSNorm (InferenceCore.java:341-347), then RoPE (:82-100, interleaved
    // pairs, Llama; :472-491, NeoX halves, Qwen3 / Phi-3).  A staging thread
    // requests its RoPE entries and norm weights before it polls.  The waves
    // then take q (and the wave whose tile holds pos the new k and v) from LDS.
    const int wpos = owns_pos ? ((pos - t0) / 16) % WPB : -1;  // wave whose tile holds pos
    const bool kvw = wave == wpos;                               // uniform over the wave
    const bool qok = hh < GQ;
    {
      constexpr int H4 = HD / 4;  // float4 groups per head
      // staging threads hold group t (and t + BS when the group's q/k/v take more
      // float4 groups than the workgroup has threads: head_dim 128 with 8 heads)
      constexpr int NG = ((GQ + 2) * H4 + BS - 1) / BS;
      const int nq4 = GQ * H4, nst4 = nq4 + (owns_pos ? 2 * H4 : 0);
      bool act[NG], rot[NG], is_q[NG];
      int tg[NG], gi[NG], d[NG];
      float c4[NG][4], s4[NG][4], w4[NG][4];
      float4 v[NG];
#pragma unroll
      for (int r = 0; r < NG; ++r) {
        const int t = (int)threadIdx.x + r * BS;
        tg[r] = t;
        act[r] = t < nst4;
        is_q[r] = t < nq4;
        const bool is_k = !is_q[r] && t < nq4 + H4;
        // q and k are normed (Qwen3) and rotated; v is stored as read.  Without RoPE
        // tables (the op-level entry points) q and k are taken as given.
        rot[r] = act[r] && (is_q[r] || is_k) && m.rope_cos != nullptr;
        gi[r] = is_q[r] ? t : (is_k ? t - nq4 : t - nq4 - H4);  // group index within q / k / v
        d[r] = 4 * (gi[r] % H4);                                  // first dim of the group in its head
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          c4[r][i] = 1.0f;
          s4[r][i] = 0.0f;
          w4[r][i] = 1.0f;
        }
        if (rot[r]) {
          // RoPE entries of the group: NeoX dims d.. use entries (d mod half)..;
          // Llama pairs (d, d+1), (d+2, d+3) use entries d/2, d/2 + 1
          if (neox) {
            const int te = d[r] < half ? d[r] : d[r] - half;
            const float4 c = *(const float4 *)(m.rope_cos + (size_t)pos * half + te);
            const float4 sv = *(const float4 *)(m.rope_sin + (size_t)pos * half + te);
            c4[r][0] = c.x; c4[r][1] = c.y; c4[r][2] = c.z; c4[r][3] = c.w;
            s4[r][0] = sv.x; s4[r][1] = sv.y; s4[r][2] = sv.z; s4[r][3] = sv.w;
          } else {
            const float2 c = *(const float2 *)(m.rope_cos + (size_t)pos * half + d[r] / 2);
            const float2 sv = *(const float2 *)(m.rope_sin + (size_t)pos * half + d[r] / 2);
            c4[r][0] = c.x; c4[r][1] = c.y;
            s4[r][0] = sv.x; s4[r][1] = sv.y;
          }
          if (qwen) {
            const float4 w = *(const float4 *)((is_q[r] ? L.q_norm : L.k_norm) + d[r]);
            w4[r][0] = w.x; w4[r][1] = w.y; w4[r][2] = w.z; w4[r][3] = w.w;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < NG; ++r) {
        v[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (act[r]) {
          const int t = tg[r];
          const int e = is_q[r] ? kvh * GQ * HD + 4 * t
                                : (t < nq4 + H4 ? m.q_dim + kvh * HD + d[r] : m.q_dim + m.kv_dim + kvh * HD + d[r]);
          const int e1[1] = {e};
          float4 v1[1];
          if (TAG)
            ld_tagged4(m.tqkv, e1, tag_in, tw, v1);
          else
            InPlain{m.qkv}.load4(e1, v1);
          v[r] = v1[0];
        }
      }
      // head_dim 64 / 128: a head's groups are H4 consecutive lanes of one wave
      // (heads start at multiples of H4), so the per-head sum and the NeoX
      // partners move by lane shuffles; head_dim 96 goes through LDS
      constexpr bool SHFL = (H4 & (H4 - 1)) == 0 && H4 <= GL3_WAVE;
      if (qwen) {
        float ssh[NG];
        if constexpr (SHFL) {
          // butterfly over the head's lanes: every lane ends with the same sum
#pragma unroll
          for (int r = 0; r < NG; ++r) {
            float ss = act[r] ? ((v[r].x * v[r].x + v[r].y * v[r].y) + v[r].z * v[r].z) + v[r].w * v[r].w : 0.0f;
#pragma unroll
            for (int o = H4 / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
            ssh[r] = ss;
          }
        } else {
          // the group partials in dim order
#pragma unroll
          for (int r = 0; r < NG; ++r)
            if (act[r]) ssb[tg[r]] = ((v[r].x * v[r].x + v[r].y * v[r].y) + v[r].z * v[r].z) + v[r].w * v[r].w;
          __syncthreads();
#pragma unroll
          for (int r = 0; r < NG; ++r) {
            ssh[r] = 0.0f;
            if (rot[r]) {
              const int h0 = tg[r] - gi[r] % H4;
              for (int i = 0; i < H4; ++i) ssh[r] += ssb[h0 + i];
            }
          }
        }
#pragma unroll
        for (int r = 0; r < NG; ++r)
          if (rot[r]) {
            const float si = inv_rms(ssh[r], HD, m.eps);
            v[r].x = w4[r][0] * (si * v[r].x);
            v[r].y = w4[r][1] * (si * v[r].y);
            v[r].z = w4[r][2] * (si * v[r].z);
            v[r].w = w4[r][3] * (si * v[r].w);
          }
      }
      if (neox) {
        // the partner of dim d is d +- half, in group gi +- H4/2 of the same head
        float4 pvs[NG];
        if constexpr (SHFL) {
#pragma unroll
          for (int r = 0; r < NG; ++r)
            pvs[r] = make_float4(__shfl_xor(v[r].x, H4 / 2), __shfl_xor(v[r].y, H4 / 2), __shfl_xor(v[r].z, H4 / 2),
                                 __shfl_xor(v[r].w, H4 / 2));
        } else {
#pragma unroll
          for (int r = 0; r < NG; ++r)
            if (act[r]) *(float4 *)(qst + 4 * tg[r]) = v[r];
          __syncthreads();
#pragma unroll
          for (int r = 0; r < NG; ++r) {
            const bool low = d[r] < half;
            pvs[r] = rot[r] ? *(const float4 *)(qst + 4 * (low ? tg[r] + H4 / 2 : tg[r] - H4 / 2))
                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          }
        }
#pragma unroll
        for (int r = 0; r < NG; ++r)
          if (rot[r]) {
            const bool low = d[r] < half;
            const float4 pv = pvs[r];
            float vv[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
            const float pp[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float v0 = low ? vv[i] : pp[i], v1 = low ? pp[i] : vv[i];
              rope_pair(v0, v1, c4[r][i], s4[r][i]);
              vv[i] = low ? v0 : v1;
            }
            v[r] = make_float4(vv[0], vv[1], vv[2], vv[3]);
          }
      } else {
#pragma unroll
        for (int r = 0; r < NG; ++r)
          if (rot[r]) {
            rope_pair(v[r].x, v[r].y, c4[r][0], s4[r][0]);
            rope_pair(v[r].z, v[r].w, c4[r][1], s4[r][1]);
          }
      }
#pragma unroll
      for (int r = 0; r < NG; ++r)
        if (act[r]) *(float4 *)(qrot + 4 * tg[r]) = v[r];
      __syncthreads();
      if (ntw > 1) at.template issue<1, true>(1);
      if (AD >= 3 && ntw > 2) at.template issue<(AD >= 3 ? 2 : 1), true>(2);
    }
    if (tk >= 0 && item == blk) trace(m, tk);
    // q of head hh (columns >= GQ take head 0 and keep zeros) as fp16 hi + lo
    half8 qh[NC], ql[NC];
    {
      const float *qh0 = qrot + (qok ? hh : 0) * HD;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float qv[8];
        f4_to(&qv[0], *(const float4 *)(qh0 + 32 * c + 8 * kb));
        f4_to(&qv[4], *(const float4 *)(qh0 + 32 * c + 8 * kb + 4));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float x = qok ? qv[i] : 0.0f;
          const _Float16 h16 = (_Float16)x;
          qh[c][i] = h16;
          ql[c][i] = (_Float16)(x - (float)h16);
        }
      }
    }
    // new k, v (fp16 bits) of the 8 dims 8*lane.. held by lanes < NQ of the wave whose tile holds pos
    unsigned knb[4] = {0u, 0u, 0u, 0u}, vnb[4] = {0u, 0u, 0u, 0u};
    if (kvw) {
      const int d0k = 8 * (lane < NQ ? lane : 0);
      float kv[8], vv[8];
      f4_to(&kv[0], *(const float4 *)(qrot + GQ * HD + d0k));
      f4_to(&kv[4], *(const float4 *)(qrot + GQ * HD + d0k + 4));
      f4_to(&vv[0], *(const float4 *)(qrot + (GQ + 1) * HD + d0k));
      f4_to(&vv[4], *(const float4 *)(qrot + (GQ + 1) * HD + d0k + 4));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        knb[i] = (unsigned)f2h(kv[2 * i]) | ((unsigned)f2h(kv[2 * i + 1]) << 16);
        vnb[i] = (unsigned)f2h(vv[2 * i]) | ((unsigned)f2h(vv[2 * i + 1]) << 16);
      }
    }

    // ---- tiles
    f32x4 O[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) O[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float mrun = -INFINITY, lrun = 0.0f;
    for (int u = 0; u < ntw; u += AD) {
      at.template step<0>(u, ntw, qh, ql, knb, vnb, O, mrun, lrun);
      at.template step<1>(u + 1, ntw, qh, ql, knb, vnb, O, mrun, lrun);
      if (AD >= 3) at.template step<(AD >= 3 ? 2 : 1)>(u + 2, ntw, qh, ql, knb, vnb, O, mrun, lrun);
    }
    if (wave == wpos && lane < NQ) {
      // append the new row to the cache, after the tiles: the stores count in
      // vmcnt, so issued earlier they would hold up the tile waits.  Agent-scope
      // (sc1) stores: later steps of the same launch may read the row from
      // another XCD.
      const int d0 = 8 * lane;
      const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(kbase, 0, 0x7fffffff, 0x00020000);
      const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(vbase, 0, 0x7fffffff, 0x00020000);
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{knb[0], knb[1], knb[2], knb[3]}, kr,
                                             (unsigned)((pos * HD + d0) * 2), 0, 16 /* sc1 */);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)(vnb[i / 2] >> (16 * (i % 2))), vr,
                                              (unsigned)((((pos / 16) * HD + d0 + i) * 16 + pos % 16) * 2), 0,
                                              16 /* sc1 */);
    }
    // ---- wave partials to LDS: O rows (heads) 4*kb + v, columns (dims) 16b + hh
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int g = 4 * kb + v;
        if (g < GQ) opart[(wave * GQ + g) * hd + 16 * b + hh] = O[b][v];
      }
    if (kb == 0 && hh < GQ) {
      mlp[(wave * GQ + hh) * 2] = mrun;
      mlp[(wave * GQ + hh) * 2 + 1] = lrun;
    }
    __syncthreads();
    if (tk >= 0 && item == blk) trace(m, tk + 1);
    constexpr int PAIRS = (GQ * HD + BS - 1) / BS;  // per-thread (g, d) slots
    float Ofin[PAIRS], Mfin[PAIRS], Lfin[PAIRS];
#pragma unroll
    for (int k = 0; k < PAIRS; ++k) {
      Ofin[k] = 0.0f;
      Mfin[k] = -INFINITY;
      Lfin[k] = 0.0f;
      const int idx = threadIdx.x + k * BS;
      if (idx < GQ * hd) {
        const int g = idx / hd, d = idx % hd;
        float mv[WPB], lv[WPB], ov[WPB];
#pragma unroll
        for (int w = 0; w < WPB; ++w) {
          mv[w] = mlp[(w * GQ + g) * 2];
          lv[w] = mlp[(w * GQ + g) * 2 + 1];
          ov[w] = opart[(w * GQ + g) * hd + d];
        }
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WPB; ++w) M = fmaxf(M, mv[w]);
        float Ls = 0.0f, Ov = 0.0f;
#pragma unroll
        for (int w = 0; w < WPB; ++w) {
          const float wt = (mv[w] == -INFINITY) ? 0.0f : __expf(mv[w] - M);
          Ls = fmaf(lv[w], wt, Ls);
          Ov = fmaf(ov[w], wt, Ov);
        }
        Mfin[k] = M;
        Lfin[k] = Ls;
        Ofin[k] = Ov;
      }
    }
    if (nsplit == 1) {
      pm();
#pragma unroll
      for (int k = 0; k < PAIRS; ++k) {
        const int idx = threadIdx.x + k * BS;
        if (idx < GQ * hd) {
          const int g = idx / hd, d = idx % hd;
          const size_t o = (size_t)(kvh * GQ + g) * hd + d;
          if (TAG)
            st_tagged(m.tatt + o, Ofin[k] / Lfin[k], tag_out);
          else
            st_coherent(m.att + o, Ofin[k] / Lfin[k]);
        }
      }
      __syncthreads();
      continue;
    }
#pragma unroll
    for (int k = 0; k < PAIRS; ++k) {
      const int idx = threadIdx.x + k * BS;
      if (idx < GQ * hd) {
        const int g = idx / hd, d = idx % hd;
        const size_t po = ((size_t)(kvh * GQ + g) * m.max_split + sp) * hpart;
        if (TAG) {
          uint2 *pt = m.tpart + po;
          st_tagged(pt + d, Ofin[k], tag_out);
          if (d == 0) {
            st_tagged(pt + hd, Mfin[k], tag_out);
            st_tagged(pt + hd + 1, Lfin[k], tag_out);
          }
        } else {
          float *pp = m.part + po;
          st_coherent(pp + d, Ofin[k]);
          if (d == 0) {
            st_coherent(pp + hd, Mfin[k]);
            st_coherent(pp + hd + 1, Lfin[k]);
          }
        }
      }
    }
    bool merge;
    // the item's outputs are out: the workgroup's own loads (e.g. the next
    // phase's weights) may go out ahead of the merge's reads
    pm();
    if (TAG) {
      // Every split's workgroup merges a slice of the kv head's GQ x hd
      // outputs: float4 groups [sp * gpw, (sp + 1) * gpw), one thread per
      // (group, split) reading that split's (m, l) and 4 dims as tagged cells,
      // then a log-sum-exp butterfly over the spl lanes of the group.  The
      // splits of a head wait for one another; with at most one item per
      // workgroup (the split count is capped so) every wait ends.
      constexpr int G4 = GQ * HD / 4;
      const int gpw = (G4 + nsplit - 1) / nsplit;
      int spl = 1;
      while (spl < nsplit) spl *= 2;  // <= 64: the lanes of a group lie in one wave
      const int gpp = BS / spl;
      for (int g0 = 0; g0 < gpw; g0 += gpp) {
        const int gl = g0 + (int)threadIdx.x / spl, sl = (int)threadIdx.x % spl;
        const int gi = sp * gpw + gl;
        const bool act = gl < gpw && gi < G4;  // uniform over the lanes of a group
        const int gc = act ? gi : 0;
        const int gg = (4 * gc) / HD, dd = (4 * gc) % HD;
        const bool real = sl < nsplit;
        // uniform base (m.tpart), per-lane cell offsets
        const unsigned pc = (unsigned)(((kvh * GQ + gg) * m.max_split + (real ? sl : 0)) * hpart);
        const uint2 *pt = m.tpart;
        u32x4 rh = ld_coherent_x4(pt, (pc + (unsigned)hd) * 8u);
        u32x4 ra = ld_coherent_x4(pt, (pc + (unsigned)dd) * 8u), rb = ld_coherent_x4(pt, (pc + (unsigned)dd) * 8u + 16u);
        if (act && real) {
          unsigned spins = 0;
          while (!(rh.y == tag_out && rh.w == tag_out && ra.y == tag_out && ra.w == tag_out && rb.y == tag_out &&
                   rb.w == tag_out)) {
            if (!tag_retry(tw, spins)) break;
            rh = ld_coherent_x4(pt, (pc + (unsigned)hd) * 8u);
            ra = ld_coherent_x4(pt, (pc + (unsigned)dd) * 8u);
            rb = ld_coherent_x4(pt, (pc + (unsigned)dd) * 8u + 16u);
          }
        }
        float M = real ? __uint_as_float(rh.x) : -INFINITY, Ls = real ? __uint_as_float(rh.z) : 0.0f;
        float4 O = real ? make_float4(__uint_as_float(ra.x), __uint_as_float(ra.z), __uint_as_float(rb.x),
                                      __uint_as_float(rb.z))
                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int msk = 1; msk < spl; msk <<= 1) {
          const float M2 = __shfl_xor(M, msk), L2 = __shfl_xor(Ls, msk);
          const float o2x = __shfl_xor(O.x, msk), o2y = __shfl_xor(O.y, msk), o2z = __shfl_xor(O.z, msk),
                      o2w = __shfl_xor(O.w, msk);
          const float mn = fmaxf(M, M2);
          const float c1 = (mn == -INFINITY) ? 0.0f : __expf(M - mn);
          const float c2 = (mn == -INFINITY) ? 0.0f : __expf(M2 - mn);
          Ls = Ls * c1 + L2 * c2;
          O.x = O.x * c1 + o2x * c2;
          O.y = O.y * c1 + o2y * c2;
          O.z = O.z * c1 + o2z * c2;
          O.w = O.w * c1 + o2w * c2;
          M = mn;
        }
        if (act && sl == 0) {
          uint2 *dst = m.tatt + (size_t)(kvh * GQ + gg) * hd + dd;
          st_tagged(dst + 0, O.x / Ls, tag_out);
          st_tagged(dst + 1, O.y / Ls, tag_out);
          st_tagged(dst + 2, O.z / Ls, tag_out);
          st_tagged(dst + 3, O.w / Ls, tag_out);
        }
      }
      merge = false;
    } else {
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
      merge = flag[0] != 0;
    }
    if (merge) {
      // log-sum-exp merge of the splits: out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s.
      // NT threads per 4 output dims, each folding splits s = q, q + NT, ... with all
      // loads of a batch issued before any is used; then the NT partial states merge.
      const int npos = GQ * hd / 4;  // <= BS (GQ * hd <= 4 * BS)
      int nt = 1;                    // threads per output float4, a power of two <= 8
      while (nt < 8 && 2 * nt * npos <= BS) nt *= 2;
      const int pidx = threadIdx.x / nt, q = threadIdx.x % nt;
      if (pidx < npos) {
        const int gg = (4 * pidx) / hd, dd = (4 * pidx) % hd;
        const size_t hb0 = (size_t)(kvh * GQ + gg) * m.max_split * hpart;
        float M = -INFINITY, Ls = 0.0f;
        float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int s0 = q; s0 < nsplit; s0 += 8 * nt) {
          float4 hv[8], ov[8];
          {
            int e[16];  // (m, l) cells then the 4 output dims of 8 splits, all loads in flight together
#pragma unroll
            for (int b = 0; b < 8; ++b) {
              const int s = s0 + b * nt;
              const int sc = s < nsplit ? s : 0;
              e[b] = (int)hb0 + sc * hpart + hd;  // uniform base (m.part), per-lane offsets
              e[8 + b] = (int)hb0 + sc * hpart + dd;
            }
            float4 v[16];
            InPlain{m.part}.load4(e, v);
#pragma unroll
            for (int b = 0; b < 8; ++b) {
              hv[b] = v[b];
              ov[b] = v[8 + b];
            }
          }
#pragma unroll
          for (int b = 0; b < 8; ++b) {
            const int s = s0 + b * nt;
            if (s < nsplit && hv[b].x != -INFINITY) {
              const float mn = fmaxf(M, hv[b].x);
              const float c1 = __expf(M - mn), c2 = __expf(hv[b].x - mn);
              Ls = Ls * c1 + hv[b].y * c2;
              O.x = O.x * c1 + ov[b].x * c2;
              O.y = O.y * c1 + ov[b].y * c2;
              O.z = O.z * c1 + ov[b].z * c2;
              O.w = O.w * c1 + ov[b].w * c2;
              M = mn;
            }
          }
        }
        // merge the nt lanes of this output (adjacent lanes)
        for (int msk = 1; msk < nt; msk <<= 1) {
          const float M2 = __shfl_xor(M, msk), L2 = __shfl_xor(Ls, msk);
          const float o2x = __shfl_xor(O.x, msk), o2y = __shfl_xor(O.y, msk), o2z = __shfl_xor(O.z, msk),
                      o2w = __shfl_xor(O.w, msk);
          const float mn = fmaxf(M, M2);
          const float c1 = (mn == -INFINITY) ? 0.0f : __expf(M - mn);
          const float c2 = (mn == -INFINITY) ? 0.0f : __expf(M2 - mn);
          Ls = Ls * c1 + L2 * c2;
          O.x = O.x * c1 + o2x * c2;
          O.y = O.y * c1 + o2y * c2;
          O.z = O.z * c1 + o2z * c2;
          O.w = O.w * c1 + o2w * c2;
          M = mn;
        }
        if (q == 0) {
          float *dst = m.att + (size_t)(kvh * GQ + gg) * hd + dd;
          st_coherent(dst + 0, O.x / Ls);
          st_coherent(dst + 1, O.y / Ls);
          st_coherent(dst + 2, O.z / Ls);
          st_coherent(dst + 3, O.w / Ls);
        }
      }
    }
    __syncthreads();
  }
}

}  // namespace gl3
