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
  float *part;              // attention partials [n_heads][max_split][hd + 4]: o[hd], m, l, pad
  unsigned *att_ctr;        // split-merge counters [L][n_kv]
  unsigned long long *best; // argmax keys [2][nbest]
  DecodeState *st;
  int *tokens_out;          // device copy of generated tokens
  unsigned long long *tstamp;  // optional phase trace: s_memrealtime at each phase boundary (workgroup 0)
};

// Phase trace of the persistent kernel: workgroup 0 stamps the 100 MHz real-time
// counter when it leaves a phase (before the grid barrier) and when it enters
// the next one (after the barrier).
__device__ __forceinline__ void trace(const ModelDev &m, int idx) {
  if (m.tstamp && threadIdx.x == 0) m.tstamp[(size_t)idx * gridDim.x + blockIdx.x] = __builtin_amdgcn_s_memrealtime();
}

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
template <int BS>
__device__ inline void load_x_lds(const float *x, const float *normw, float eps, int K, float *xs, float *red) {
  if (!normw) {
#pragma unroll 4
    for (int i = 4 * threadIdx.x; i < K; i += 4 * BS) *(float4 *)(xs + i) = ld_coherent_f4(x, i);
    __syncthreads();
    return;
  }
  if (K > 16 * BS) {  // wide vectors: weights read after the reduction
    float ss = 0.0f;
    for (int i = 4 * threadIdx.x; i < K; i += 4 * BS) {
      float4 v = ld_coherent_f4(x, i);
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
  // x and the norm weights are fetched together; the weights wait in registers
  // (up to 4 float4 per thread) while the sum of squares is reduced.
  float ss = 0.0f;
  float4 wv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = 4 * (threadIdx.x + u * BS);
    if (i < K) {
      float4 v = ld_coherent_f4(x, i);
      wv[u] = *(const float4 *)(normw + i);
      *(float4 *)(xs + i) = v;
      ss += v.x * v.x;
      ss += v.y * v.y;
      ss += v.z * v.z;
      ss += v.w * v.w;
    }
  }
  ss = block_sum<BS>(ss, red);
  ss /= (float)K;
  ss += eps;
  ss = (float)(1.0 / sqrt((double)ss));
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = 4 * (threadIdx.x + u * BS);
    if (i < K) {
      float4 v = *(float4 *)(xs + i);
      v.x = wv[u].x * (ss * v.x);
      v.y = wv[u].y * (ss * v.y);
      v.z = wv[u].z * (ss * v.z);
      v.w = wv[u].w * (ss * v.w);
      *(float4 *)(xs + i) = v;
    }
  }
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

// 16 (4) bytes per lane from rsrc + voff + soff into LDS at lds + 16 (4) * lane.
#define GL3_DMA_NT 2  // cache policy: nontemporal (weights are read once per token)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void *lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)lds, 16, voff, soff, 0, GL3_DMA_NT);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, void *lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)lds, 4, voff, soff, 0, GL3_DMA_NT);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, 0x7fffffff, 0x00020000);
}

template <int FMT, int KC, int KS, int NR, int MODE, int BS, int SC_ = 0, int DEPTH = 2>
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
  static_assert(DEPTH == 2 || DEPTH == 3, "ring depth");
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
    return blk < n ? (n - 1 - blk) / nblk + 1 : 0;
  }

  // Issues the loads of slot-load u (the workgroup's item u / PASSES, pass u % PASSES) into ring slot S.
  template <int S>
  static __device__ __forceinline__ void issue(const Mat &W, int out_rows, int u, int blk, int nblk) {
    const int wave = wave_id(), lane = lane_id();
    const int ks = wave % KS, rg = wave / KS;
    const int K = W.cols;
    const int item = blk + (u / PASSES) * nblk, pass = PASSES > 1 ? u % PASSES : 0;
    const int j0 = pass * JP;
    u32x4 *rw = ring_w<S, WCH>() + wave * SC * GL3_WAVE;
    const __amdgpu_buffer_rsrc_t rq = rsrc(W.q);
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
      unsigned *rs = ring_s<S, SDW>() + wave * SC * 16;
      const __amdgpu_buffer_rsrc_t rsc = rsrc(W.s);
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
    if (DEPTH == 3 && nu > 2) issue<(DEPTH == 3 ? 2 : 1)>(W, out_rows, 2, blk, nblk);
  }

  struct XSlice {
    float r[XREG ? KC : 1][XREG ? EPC : 1];
    const float *lds;
    int e0;
    __device__ __forceinline__ float get(int j, int i) const {
      return XREG ? r[XREG ? j : 0][XREG ? i : 0] : lds[e0 + GL3_WAVE * EPC * j + i];
    }
  };

  // acc[r][p] += the lane's part of the dot products held in slot S (pass `pass` of the item)
  template <int S>
  static __device__ __forceinline__ void dot_slot(const XSlice &xr, int pass, float (&acc)[NR][NP]) {
    const int wave = wave_id(), lane = lane_id();
    const u32x4 *rw = ring_w<S, WCH>() + wave * SC * GL3_WAVE + lane;
    const uint8_t *rs = (const uint8_t *)(ring_s<S, SDW>() + wave * SC * 16);
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
  // the row values go to obuf[i * ROWS_PER_ITEM + row in item].
  static __device__ __forceinline__ void finish_item(int i, float (&acc)[NR][NP], float *kpart, float *obuf) {
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
      obuf[i * ROWS_PER_ITEM + rg * NR + lane] = (MODE == MODE_SWIGLU) ? silu_ref(a0) * a1 : a0;
    }
  }

  template <int S>
  static __device__ __forceinline__ void step(const Mat &W, int out_rows, int u, int nu, int blk, int nblk,
                                              const XSlice &xr, float (&acc)[NR][NP], float *kpart, float *obuf) {
    if (u < nu) {
      // slot S is complete once at most the loads of the (up to DEPTH-1) later slot-loads are outstanding
      const int later = nu - 1 - u;
      if (DEPTH == 3 && later >= 2)
        wait_vmem<2 * NI_MIN>();
      else if (later >= 1)
        wait_vmem<NI_MIN>();
      else
        wait_vmem<0>();
      const int pass = PASSES > 1 ? u % PASSES : 0;
      dot_slot<S>(xr, pass, acc);
      if (u + DEPTH < nu) issue<S>(W, out_rows, u + DEPTH, blk, nblk);
      if (PASSES == 1 || pass == PASSES - 1) {
        finish_item(u / PASSES, acc, kpart, obuf);
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
          for (int p = 0; p < NP; ++p) acc[r][p] = 0.0f;
      }
    }
  }

  // LDS layout of a phase: [x (K floats, when staged)] [red 32] [kpart] [obuf] [best keys]
  static __host__ __device__ constexpr int kpart_floats() { return RG * NR * NP * KS; }
  static __host__ __device__ __forceinline__ bool staged(bool has_norm) { return !(XDIRECT_OK && !has_norm); }
  static __host__ __device__ __forceinline__ size_t lds_bytes(int K, int out_rows, int nblk, bool has_norm) {
    const int lr = local_items(out_rows, 0, nblk) * ROWS_PER_ITEM;
    return (size_t)((staged(has_norm) ? K : 0) + 32 + kpart_floats() + lr + 2 * WPB + 4) * sizeof(float);
  }

  // Runs the phase.  x: input vector (K floats, coherent); normw: RMSNorm
  // weights or nullptr; y: output (MODE_RESIDUAL: y += W n(x)); for
  // MODE_LOGITS, y gets the rows and best_out[blk] the argmax key of the rows
  // this workgroup produced.  prefetched: prefetch() was already called with
  // the same W, out_rows, blk and nblk.
  static __device__ void run(const Mat &W, int out_rows, const float *x, const float *normw, float eps, float *y,
                             unsigned long long *best_out, int blk, int nblk, float *lds, bool prefetched = false) {
    const int K = W.cols;
    const bool stg = staged(normw != nullptr);
    float *xs = lds;                          // K floats when staged
    float *red = lds + (stg ? K : 0);         // reduction scratch (32 floats)
    float *kpart = red + 32;                  // cross-wave partials
    float *obuf = kpart + kpart_floats();     // row values of the workgroup's items
    const int nli = local_items(out_rows, blk, nblk);
    const int nu = nli * PASSES;
    if (!prefetched) prefetch(W, out_rows, blk, nblk);

    const int wave = wave_id(), lane = lane_id();
    const int ks = wave % KS;
    XSlice xr;
    xr.lds = xs;
    xr.e0 = elem(K, ks, lane, 0);
    if (!stg) {
      if (XDIRECT_OK) {
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
          for (int i = 0; i < EPC; i += 4) {
            const float4 v = ld_coherent_f4(x, (unsigned)(elem(K, ks, lane, j) + i));
            xr.r[j][i] = v.x;
            xr.r[j][i + 1] = v.y;
            xr.r[j][i + 2] = v.z;
            xr.r[j][i + 3] = v.w;
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

    float acc[NR][NP];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int p = 0; p < NP; ++p) acc[r][p] = 0.0f;
    for (int u = 0; u < nu; u += DEPTH) {
      step<0>(W, out_rows, u, nu, blk, nblk, xr, acc, kpart, obuf);
      step<1>(W, out_rows, u + 1, nu, blk, nblk, xr, acc, kpart, obuf);
      if (DEPTH == 3) step<(DEPTH == 3 ? 2 : 1)>(W, out_rows, u + 2, nu, blk, nblk, xr, acc, kpart, obuf);
    }
    __syncthreads();

    // write the rows out (coalesced over the workgroup's items)
    unsigned long long best = 0;
    for (int lr = threadIdx.x; lr < nli * ROWS_PER_ITEM; lr += BS) {
      const int row = (blk + (lr / ROWS_PER_ITEM) * nblk) * ROWS_PER_ITEM + lr % ROWS_PER_ITEM;
      if (row < out_rows) {
        const float v = obuf[lr];
        if (MODE == MODE_RESIDUAL) {
          st_coherent(y + row, ld_coherent(y + row) + v);
        } else if (MODE == MODE_LOGITS) {
          y[row] = v;
          const unsigned long long k = argmax_key(v, row);
          best = k > best ? k : best;
        } else {
          st_coherent(y + row, v);
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

// -------------------------------------------------------------- attention
// Flash-decode over the fp16 KV cache [L][n_kv][ctx][hd].  Work item = (kv
// head, split of positions); the workgroup serves the GQ query heads of the kv
// head's GQA group, so each K/V row is read from HBM once per group.
//
// Every wavefront owns positions in steps of PPW = 64/LP: LP lanes hold 8
// dimensions each of one position's K and V row (16-byte loads), q of all GQ
// heads in registers, reduce the GQ scores over the LP lanes with DPP and keep
// an online softmax state (max, sum, o) per lane group in registers.  K/V
// loads run ATT_DEPTH steps ahead in a register ring.  The lane groups of a
// wave are merged with shuffles, the waves through LDS, and the splits of a kv
// head by log-sum-exp in the workgroup that finishes last.
//
// q (and, in the split holding `pos`, the new k and v) are read straight into
// registers together with the RoPE table entries and the first K/V rows, so
// the preparation costs one memory round trip: the Qwen3 per-head RMSNorm is a
// lane-group sum, RoPE rotates pairs inside a lane (Llama, interleaved) or
// across lanes half a head apart (NeoX).  Scores are (q . k) / sqrt(hd)
// (InferenceCore.java:114-121); norm and RoPE follow InferenceCore.java:82-100,
// :341-372, :472-491.

#define ATT_DEPTH 4

__device__ __forceinline__ void rope_pair(float &v0, float &v1, float c, float s) {
  float a = v0 * c - v1 * s;
  float b = v0 * s + v1 * c;
  v0 = a;
  v1 = b;
}

// Positions per split: a multiple of the workgroup's positions per step.
__host__ __device__ __forceinline__ int att_split_len(int n, int max_split, int step) {
  int s = (n + max_split - 1) / max_split;
  s = (s + step - 1) / step * step;
  return s < step ? step : s;
}

// LDS floats of the attention phase: lane-group states o [PPB][G][hd], (m, l)
// [PPB][G][2] and a flag, with PPB = 64 / LP lane groups per wave x wpb waves.
__host__ __device__ __forceinline__ int att_lds_floats(int hd, int G, int wpb, int max_split) {
  (void)max_split;
  const int ppb = (GL3_WAVE / (hd <= 64 ? 8 : 16)) * wpb;
  return ppb * G * (hd + 2) + 16;
}

__device__ __forceinline__ void f4_to(float *dst, float4 v) {
  dst[0] = v.x;
  dst[1] = v.y;
  dst[2] = v.z;
  dst[3] = v.w;
}

// Qwen3 per-head RMSNorm of the 8 dims a lane holds (lane group = one head):
// v = w * (ss * v), ss = 1/sqrt(mean(v^2) + eps)  (InferenceCore.java:341-347)
template <int LP>
__device__ __forceinline__ void head_norm(float (&v)[8], const float (&w)[8], int hd, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
  ss = group_sum<LP>(ss);
  ss /= (float)hd;
  ss += eps;
  ss = (float)(1.0 / sqrt((double)ss));
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = w[i] * (ss * v[i]);
}

// RoPE of the 8 dims d0..d0+7 a lane holds.  Llama: pairs (2i, 2i+1) with
// table entry i (c, s hold entries d0/2 .. d0/2+3).  NeoX: pairs (i, i+hd/2)
// with entry i; the partner dims live in lane `partner` (c, s hold entries
// (d0 mod hd/2) .. +7).  Inactive lanes (d0 >= hd) take part in the shuffle only.
__device__ __forceinline__ void rope_lane(float (&v)[8], const float (&c)[8], const float (&s)[8], bool neox,
                                          bool low, int partner) {
  if (!neox) {
#pragma unroll
    for (int i = 0; i < 4; ++i) rope_pair(v[2 * i], v[2 * i + 1], c[i], s[i]);
  } else {
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = __shfl(v[i], partner);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v0 = low ? v[i] : o[i], v1 = low ? o[i] : v[i];
      rope_pair(v0, v1, c[i], s[i]);
      v[i] = low ? v0 : v1;
    }
  }
}

template <int LP, int GQ, int BS>
__device__ void phase_attention(const ModelDev &m, int layer, int pos, int blk, int nblk, float *lds) {
  constexpr int WPB = BS / GL3_WAVE, PPW = GL3_WAVE / LP, PPB = PPW * WPB;
  const int hd = m.hd, half = hd / 2;
  const int n = pos + 1;
  const int S = att_split_len(n, m.max_split, PPB);
  const int nsplit = (n + S - 1) / S;
  const int items = m.n_kv * nsplit;
  const int hpart = hd + 4;
  static_assert(LP == 8 || LP == 16, "lane group");
  float *opart = lds;                     // lane-group o [PPB][GQ][hd]
  float *mlp = opart + PPB * GQ * hd;     // lane-group (m, l) [PPB][GQ][2]
  int *flag = (int *)(mlp + PPB * GQ * 2);
  const LayerDev L = ld_layer(m.layers, layer);
  const size_t head_stride = (size_t)m.ctx * hd;
  uint16_t *kc_l = m.kc + (size_t)layer * m.n_kv * head_stride;
  uint16_t *vc_l = m.vc + (size_t)layer * m.n_kv * head_stride;
  const int wave = wave_id(), lane = lane_id();
  const int grp = lane / LP, sub = lane % LP, d0 = 8 * sub;
  const bool act = d0 < hd;
  const bool neox = m.family != FAM_LLAMA;
  const bool low = d0 < half;
  const int partner = (lane - sub) + (low ? sub + half / 8 : sub - half / 8);
  const bool qwen = m.family == FAM_QWEN3;
  const int te = neox ? (low ? d0 : d0 - half) : d0 / 2;  // first RoPE table entry of the lane

  for (int item = blk; item < items; item += nblk) {
    const int kvh = item / nsplit, sp = item % nsplit;
    const int t0 = sp * S, t1 = min(n, t0 + S);
    const bool owns_pos = (pos >= t0 && pos < t1);
    uint16_t *kh = kc_l + kvh * head_stride;
    uint16_t *vh = vc_l + kvh * head_stride;
    const int tb0 = t0 + wave * PPW + grp;

    // ---- one round trip: q, new k/v, RoPE entries, norm weights, first K/V rows
    float qr[GQ][8], kn[8], vn[8], rc[8], rs[8], qw[8], kw8[8];
    if (act) {
#pragma unroll
      for (int g = 0; g < GQ; ++g) {
        const unsigned qo = (unsigned)((kvh * GQ + g) * hd + d0);
        f4_to(&qr[g][0], ld_coherent_f4(m.qkv, qo));
        f4_to(&qr[g][4], ld_coherent_f4(m.qkv, qo + 4));
      }
      if (owns_pos) {
        const unsigned ko = (unsigned)(m.q_dim + kvh * hd + d0), vo = ko + (unsigned)m.kv_dim;
        f4_to(&kn[0], ld_coherent_f4(m.qkv, ko));
        f4_to(&kn[4], ld_coherent_f4(m.qkv, ko + 4));
        f4_to(&vn[0], ld_coherent_f4(m.qkv, vo));
        f4_to(&vn[4], ld_coherent_f4(m.qkv, vo + 4));
      }
      const float *cr = m.rope_cos + (size_t)pos * half + te, *ci = m.rope_sin + (size_t)pos * half + te;
      f4_to(&rc[0], *(const float4 *)cr);
      f4_to(&rs[0], *(const float4 *)ci);
      if (neox) {
        f4_to(&rc[4], *(const float4 *)(cr + 4));
        f4_to(&rs[4], *(const float4 *)(ci + 4));
      }
      if (qwen) {
        f4_to(&qw[0], *(const float4 *)(L.q_norm + d0));
        f4_to(&qw[4], *(const float4 *)(L.q_norm + d0 + 4));
        f4_to(&kw8[0], *(const float4 *)(L.k_norm + d0));
        f4_to(&kw8[4], *(const float4 *)(L.k_norm + d0 + 4));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int g = 0; g < GQ; ++g) qr[g][i] = 0.0f;
        kn[i] = vn[i] = rc[i] = rs[i] = qw[i] = kw8[i] = 0.0f;
      }
    }
    u32x4 kr[ATT_DEPTH], vr[ATT_DEPTH];
#pragma unroll
    for (int u = 0; u < ATT_DEPTH; ++u) {
      const int t = tb0 + u * PPB;
      if (act && t < t1 && t != pos) {
        kr[u] = ld_stream(kh + (size_t)t * hd + d0);
        vr[u] = ld_stream(vh + (size_t)t * hd + d0);
      } else {
        kr[u] = u32x4{0u, 0u, 0u, 0u};
        vr[u] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    // ---- q (and new k): per-head norm (Qwen3), RoPE at pos
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      if (qwen) head_norm<LP>(qr[g], qw, hd, m.eps);
      rope_lane(qr[g], rc, rs, neox, low, partner);
    }
    if (owns_pos) {
      if (qwen) head_norm<LP>(kn, kw8, hd, m.eps);
      rope_lane(kn, rc, rs, neox, low, partner);
      // fp16 cache entries at pos; the values used below are the rounded ones
      unsigned kb[4], vb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t k0 = f2h(kn[2 * i]), k1 = f2h(kn[2 * i + 1]);
        const uint16_t v0 = f2h(vn[2 * i]), v1 = f2h(vn[2 * i + 1]);
        kb[i] = (unsigned)k0 | ((unsigned)k1 << 16);
        vb[i] = (unsigned)v0 | ((unsigned)v1 << 16);
        kn[2 * i] = h2f(k0);
        kn[2 * i + 1] = h2f(k1);
        vn[2 * i] = h2f(v0);
        vn[2 * i + 1] = h2f(v1);
      }
      if (wave == 0 && grp == 0 && act) {
        *(u32x4 *)(kh + (size_t)pos * hd + d0) = u32x4{kb[0], kb[1], kb[2], kb[3]};
        *(u32x4 *)(vh + (size_t)pos * hd + d0) = u32x4{vb[0], vb[1], vb[2], vb[3]};
      }
    }

    float mr[GQ], lr[GQ], o[GQ][8];
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      mr[g] = -INFINITY;
      lr[g] = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[g][i] = 0.0f;
    }
    // ---- scores and softmax, ATT_DEPTH steps per batch: all scores of the
    //      batch first, one rescale of the running state, then the V terms.
    //      Slot u of the register ring is reloaded ATT_DEPTH steps ahead right
    //      after use; steps past the split's end are skipped by the wave.
    const int wb = __builtin_amdgcn_readfirstlane(t0 + wave * PPW);  // the wave's first position
    for (int it = 0; wb + it * ATT_DEPTH * PPB < t1; ++it) {
      const int tb = tb0 + it * ATT_DEPTH * PPB, wt = wb + it * ATT_DEPTH * PPB;
      float sc[ATT_DEPTH][GQ], bm[GQ];
#pragma unroll
      for (int g = 0; g < GQ; ++g) bm[g] = -INFINITY;
#pragma unroll
      for (int u = 0; u < ATT_DEPTH; ++u) {
#pragma unroll
        for (int g = 0; g < GQ; ++g) sc[u][g] = -INFINITY;
        if (wt + u * PPB < t1) {
          const int t = tb + u * PPB;
          float kf[8];
          if (t == pos) {
#pragma unroll
            for (int i = 0; i < 8; ++i) kf[i] = kn[i];
          } else {
            const unsigned ka[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              kf[2 * i] = h2f_lo(ka[i]);
              kf[2 * i + 1] = h2f_hi(ka[i]);
            }
          }
          const int tn = t + ATT_DEPTH * PPB;
          if (act && tn < t1 && tn != pos) kr[u] = ld_stream(kh + (size_t)tn * hd + d0);
#pragma unroll
          for (int g = 0; g < GQ; ++g) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) a = fmaf(qr[g][i], kf[i], a);
            const float sv = group_sum<LP>(a) / m.sqrt_hd;
            if (t < t1) {
              sc[u][g] = sv;
              bm[g] = fmaxf(bm[g], sv);
            }
          }
        }
      }
#pragma unroll
      for (int g = 0; g < GQ; ++g) {
        const float mn = fmaxf(mr[g], bm[g]);
        if (mn != -INFINITY) {
          const float c = __expf(mr[g] - mn);
          lr[g] *= c;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[g][i] *= c;
          mr[g] = mn;
        }
      }
#pragma unroll
      for (int u = 0; u < ATT_DEPTH; ++u) {
        if (wt + u * PPB < t1) {
          const int t = tb + u * PPB;
          float vf[8];
          if (t == pos) {
#pragma unroll
            for (int i = 0; i < 8; ++i) vf[i] = vn[i];
          } else {
            const unsigned va[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              vf[2 * i] = h2f_lo(va[i]);
              vf[2 * i + 1] = h2f_hi(va[i]);
            }
          }
          const int tn = t + ATT_DEPTH * PPB;
          if (act && tn < t1 && tn != pos) vr[u] = ld_stream(vh + (size_t)tn * hd + d0);
#pragma unroll
          for (int g = 0; g < GQ; ++g) {
            if (sc[u][g] != -INFINITY) {
              const float p = __expf(sc[u][g] - mr[g]);
              lr[g] += p;
#pragma unroll
              for (int i = 0; i < 8; ++i) o[g][i] = fmaf(p, vf[i], o[g][i]);
            }
          }
        }
      }
    }
    // ---- the PPB lane-group states of the workgroup go to LDS; thread (g, d)
    //      pairs merge them
    {
      const int pi = wave * PPW + grp;
      if (act) {
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
          float *dst = opart + (pi * GQ + g) * hd + d0;
          *(float4 *)dst = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
          *(float4 *)(dst + 4) = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
        }
      }
      if (sub == 0) {
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
          mlp[(pi * GQ + g) * 2] = mr[g];
          mlp[(pi * GQ + g) * 2 + 1] = lr[g];
        }
      }
    }
    __syncthreads();
    constexpr int PAIRS = (GQ * LP * 8 + BS - 1) / BS;  // per-thread (g, d) slots (hd <= 8 * LP)
    constexpr int CB = 8;                                 // partials read per batch
    static_assert(PPB % CB == 0, "lane-group partials per batch");
    float Ofin[PAIRS], Mfin[PAIRS], Lfin[PAIRS];
#pragma unroll
    for (int k = 0; k < PAIRS; ++k) {
      Ofin[k] = 0.0f;
      Mfin[k] = -INFINITY;
      Lfin[k] = 0.0f;
      const int idx = threadIdx.x + k * BS;
      if (idx < GQ * hd) {
        const int g = idx / hd, d = idx % hd;
        // LDS reads are issued CB at a time before their first use (one wave per
        // SIMD: nothing else hides their latency)
        float M = -INFINITY;
        for (int p0 = 0; p0 < PPB; p0 += CB) {
          float mv[CB];
#pragma unroll
          for (int c = 0; c < CB; ++c) mv[c] = mlp[((p0 + c) * GQ + g) * 2];
#pragma unroll
          for (int c = 0; c < CB; ++c) M = fmaxf(M, mv[c]);
        }
        float Ls = 0.0f, O = 0.0f;
        for (int p0 = 0; p0 < PPB; p0 += CB) {
          float mv[CB], lv[CB], ov[CB];
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            mv[c] = mlp[((p0 + c) * GQ + g) * 2];
            lv[c] = mlp[((p0 + c) * GQ + g) * 2 + 1];
            ov[c] = opart[((p0 + c) * GQ + g) * hd + d];
          }
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            const float w = (mv[c] == -INFINITY) ? 0.0f : __expf(mv[c] - M);
            Ls = fmaf(lv[c], w, Ls);
            O = fmaf(ov[c], w, O);
          }
        }
        Mfin[k] = M;
        Lfin[k] = Ls;
        Ofin[k] = O;
      }
    }
    if (nsplit == 1) {
#pragma unroll
      for (int k = 0; k < PAIRS; ++k) {
        const int idx = threadIdx.x + k * BS;
        if (idx < GQ * hd) {
          const int g = idx / hd, d = idx % hd;
          st_coherent(m.att + (size_t)(kvh * GQ + g) * hd + d, Ofin[k] / Lfin[k]);
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
        float *pp = m.part + ((size_t)(kvh * GQ + g) * m.max_split + sp) * hpart;
        st_coherent(pp + d, Ofin[k]);
        if (d == 0) {
          st_coherent(pp + hd, Mfin[k]);
          st_coherent(pp + hd + 1, Lfin[k]);
        }
      }
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
      // log-sum-exp merge of the splits: out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s.
      // NT threads per 4 output dims, each folding splits s = q, q + NT, ... with all
      // loads of a batch issued before any is used; then the NT partial states merge.
      const int npos = GQ * hd / 4;  // <= BS (GQ * hd <= 4 * BS)
      int nt = 1;                    // threads per output float4, a power of two <= 8
      while (nt < 8 && 2 * nt * npos <= BS) nt *= 2;
      const int pidx = threadIdx.x / nt, q = threadIdx.x % nt;
      if (pidx < npos) {
        const int gg = (4 * pidx) / hd, dd = (4 * pidx) % hd;
        const float *base = m.part + (size_t)(kvh * GQ + gg) * m.max_split * hpart;
        float M = -INFINITY, Ls = 0.0f;
        float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int s0 = q; s0 < nsplit; s0 += 8 * nt) {
          float4 hv[8], ov[8];
#pragma unroll
          for (int b = 0; b < 8; ++b) {
            const int s = s0 + b * nt;
            if (s < nsplit) {
              hv[b] = ld_coherent_f4(base, (unsigned)(s * hpart + hd));
              ov[b] = ld_coherent_f4(base, (unsigned)(s * hpart + dd));
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
