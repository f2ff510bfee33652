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
#include <algorithm>

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

typedef _Float16 ph2 __attribute__((ext_vector_type(2)));

// 4 int8 quants (one dword) as 4 exact fp16 values: each byte, biased to
// unsigned, becomes the low mantissa byte of fp16 0x64xx (= 1024 + u), and
// 1152 = 1024 + 128 is subtracted (v_perm_b32 + packed fp16 subtraction).
__device__ __forceinline__ void i8x4_to_h4(unsigned w, ph2 &lo, ph2 &hi) {
  const unsigned u = w ^ 0x80808080u;
  const unsigned a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const unsigned b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const ph2 bias = ph2{(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(ph2, a) - bias;
  hi = __builtin_bit_cast(ph2, b) - bias;
}

__device__ __forceinline__ ph8 q8_to_h8(unsigned w0, unsigned w1) {
  ph2 a, b, c, d;
  i8x4_to_h4(w0, a, b);
  i8x4_to_h4(w1, c, d);
  return ph8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

constexpr int GBT = 64;        // rows of X per workgroup tile
constexpr int GBN = 128;       // rows of W per workgroup tile (SwiGLU: 64 gate + the 64 matching up rows)
constexpr int GBK = 64;        // columns per stage (two Q8_0 blocks)
constexpr int XSTR = GBK + 8;  // X tile row stride in LDS, halves (144 B: conflict-free 16-B reads by 16 rows)

struct GemmArgs {
  const uint8_t *wq;
  const uint16_t *ws;
  int N, K;                  // output columns (SwiGLU: hidden), reduction length
  const _Float16 *xh, *xl;   // activations [T][K] as hi / lo planes
  int T;
  float *y;                  // MODE_STORE / MODE_RESIDUAL output [T][N]
  _Float16 *yh, *yl;         // MODE_SWIGLU output planes [T][N]
  float *part;               // split-K partials [ksplit][T][NW] (NW = N, SwiGLU 2N: gate then up)
  int ksplit;
};

// Output element (t, n) of the matrix product, applied per mode.
template <int MODE>
__device__ __forceinline__ void gemm_store(const GemmArgs &g, int t, int n, float a, float up) {
  const size_t i = (size_t)t * g.N + n;
  if (MODE == MODE_STORE)
    g.y[i] = a;
  else if (MODE == MODE_RESIDUAL)
    g.y[i] += a;
  else
    put_split(g.yh, g.yl, i, silu_ref(a) * up);  // InferenceCore.java:162-166
}

}  // namespace

// Y[T][N] = X[T][K] . W[N][K]^T on the matrix cores.  A workgroup computes a
// 64 (rows of X) x 128 (rows of W) tile over its share of K, in stages of 64
// columns: both operands go through LDS (global -> registers -> LDS, the next
// stage's loads in flight during the current stage's products, two LDS
// buffers, one barrier per stage).  Wave w owns W tile rows 32w .. 32w + 31
// (SwiGLU: gate rows 16w .. 16w + 15 and the matching up rows, so that one lane
// holds both values of an output) against all 64 rows of X: 2 x 4 MFMA tiles of
// 16 x 16.  MFMA operands: lane (hh, kb) holds row hh of the A tile (a row of
// X) and column hh of the B tile (a row of W), elements 8 kb .. 8 kb + 7 of the
// 32-column block; the result lane holds rows 4 kb .. 4 kb + 3 of column hh.
// With ksplit > 1, blockIdx.z takes K / ksplit columns and writes fp32
// partials; gemm_reduce_kernel adds them in split order and applies the mode.
template <int FMT, int MODE>
__global__ __launch_bounds__(PBS) void gemm_kernel(GemmArgs g) {
  constexpr bool SW = MODE == MODE_SWIGLU;
  constexpr int WSB = FMT == FMT_Q8 ? 80 : 144;    // W tile row stride in LDS, bytes (conflict-free reads)
  constexpr int WLD = FMT == FMT_Q8 ? 2 : 4;       // 16-byte W loads per thread per stage
  __shared__ __align__(16) _Float16 xs[2][2][GBT * XSTR];  // [buffer][hi / lo][row * XSTR + column]
  __shared__ __align__(16) uint8_t wsm[2][GBN * WSB];      // [buffer][row * WSB + byte]
  __shared__ unsigned ssm[2][GBN];                         // Q8_0: the row's two block scales of the stage

  const int tid = threadIdx.x, wave = tid / GL3_WAVE, lane = tid % GL3_WAVE;
  const int hh = lane % 16, kb = lane / 16;
  const int n0 = blockIdx.x * (SW ? GBN / 2 : GBN);
  const int t0 = blockIdx.y * GBT;
  const int kper = g.K / g.ksplit, kbeg = blockIdx.z * kper, nst = kper / GBK;

  // global W row of LDS tile row r (rows past the matrix repeat its last row; their results are dropped)
  auto wrow = [&](int r) -> size_t {
    if (SW) return r < GBN / 2 ? (size_t)min(n0 + r, g.N - 1) : (size_t)g.N + min(n0 + r - GBN / 2, g.N - 1);
    return (size_t)min(n0 + r, g.N - 1);
  };
  // loaders: X rows tid / 8 and tid / 8 + 32, 16-byte chunk tid % 8, both planes;
  // W (Q8_0: 64 bytes per row, 4 threads a row; F16: 128 bytes, 8 threads a row)
  const int xr = tid / 8, xc = 8 * (tid % 8);
  const size_t xo0 = (size_t)min(t0 + xr, g.T - 1) * g.K + xc, xo1 = (size_t)min(t0 + xr + 32, g.T - 1) * g.K + xc;
  constexpr int TPR = FMT == FMT_Q8 ? 4 : 8;  // threads per W row
  constexpr int RPL = PBS / TPR;              // W rows per load round
  size_t wo[WLD];
#pragma unroll
  for (int i = 0; i < WLD; ++i)
    wo[i] = wrow(tid / TPR + RPL * i) * (size_t)g.K * (FMT == FMT_Q8 ? 1 : 2) + 16 * (tid % TPR);
  const size_t so = FMT == FMT_Q8 && tid < GBN ? wrow(tid) * (size_t)(g.K / 32) : 0;

  u32x4 rx[4], rw[WLD];
  unsigned rs = 0;
  auto gload = [&](int k0) {
    rx[0] = *(const u32x4 *)(g.xh + xo0 + k0);
    rx[1] = *(const u32x4 *)(g.xl + xo0 + k0);
    rx[2] = *(const u32x4 *)(g.xh + xo1 + k0);
    rx[3] = *(const u32x4 *)(g.xl + xo1 + k0);
#pragma unroll
    for (int i = 0; i < WLD; ++i) rw[i] = *(const u32x4 *)(g.wq + wo[i] + (size_t)k0 * (FMT == FMT_Q8 ? 1 : 2));
    if (FMT == FMT_Q8 && tid < GBN) rs = *(const unsigned *)(g.ws + so + k0 / 32);
  };
  auto lstore = [&](int buf) {
    *(u32x4 *)&xs[buf][0][xr * XSTR + xc] = rx[0];
    *(u32x4 *)&xs[buf][1][xr * XSTR + xc] = rx[1];
    *(u32x4 *)&xs[buf][0][(xr + 32) * XSTR + xc] = rx[2];
    *(u32x4 *)&xs[buf][1][(xr + 32) * XSTR + xc] = rx[3];
#pragma unroll
    for (int i = 0; i < WLD; ++i) *(u32x4 *)&wsm[buf][(tid / TPR + RPL * i) * WSB + 16 * (tid % TPR)] = rw[i];
    if (FMT == FMT_Q8 && tid < GBN) ssm[buf][tid] = rs;
  };

  // this wave's two 16-row groups of the W tile
  const int rj[2] = {SW ? 16 * wave : 32 * wave, SW ? GBN / 2 + 16 * wave : 32 * wave + 16};
  pf4 acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = pf4{0.0f, 0.0f, 0.0f, 0.0f};

  gload(kbeg);
  lstore(0);
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    if (st + 1 < nst) gload(kbeg + (st + 1) * GBK);
#pragma unroll
    for (int b = 0; b < 2; ++b) {  // the stage's two 32-column blocks
      ph8 ah[4], al[4], bw[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ah[i] = *(const ph8 *)&xs[buf][0][(16 * i + hh) * XSTR + 32 * b + 8 * kb];
        al[i] = *(const ph8 *)&xs[buf][1][(16 * i + hh) * XSTR + 32 * b + 8 * kb];
      }
      float sc[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = rj[j] + hh;
        if (FMT == FMT_Q8) {
          const uint2 w = *(const uint2 *)&wsm[buf][r * WSB + 32 * b + 8 * kb];
          bw[j] = q8_to_h8(w.x, w.y);
          sc[j] = h2f((uint16_t)(ssm[buf][r] >> (16 * b)));
        } else {
          bw[j] = *(const ph8 *)&wsm[buf][r * WSB + 2 * (32 * b + 8 * kb)];
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (FMT == FMT_Q8) {
            pf4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bw[j], pf4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bw[j], tmp, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[j][i][v] = fmaf(tmp[v], sc[j], acc[j][i][v]);
          } else {
            acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bw[j], acc[j][i], 0, 0, 0);
            acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bw[j], acc[j][i], 0, 0, 0);
          }
        }
    }
    if (st + 1 < nst) lstore(buf ^ 1);
    __syncthreads();
  }

  const int NW = SW ? 2 * g.N : g.N;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int t = t0 + 16 * i + 4 * kb + v;
      if (t >= g.T) continue;
      if (SW) {
        const int n = n0 + 16 * wave + hh;
        if (n >= g.N) continue;
        if (g.ksplit == 1) {
          gemm_store<MODE>(g, t, n, acc[0][i][v], acc[1][i][v]);
        } else {
          float *pp = g.part + ((size_t)blockIdx.z * g.T + t) * NW;
          pp[n] = acc[0][i][v];
          pp[g.N + n] = acc[1][i][v];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + 32 * wave + 16 * j + hh;
          if (n >= g.N) continue;
          if (g.ksplit == 1)
            gemm_store<MODE>(g, t, n, acc[j][i][v], 0.0f);
          else
            g.part[((size_t)blockIdx.z * g.T + t) * NW + n] = acc[j][i][v];
        }
      }
    }
}

// Sum of the split-K partials in split order, then the mode's output.
template <int MODE>
__global__ __launch_bounds__(PBS) void gemm_reduce_kernel(GemmArgs g) {
  const size_t i = (size_t)blockIdx.x * PBS + threadIdx.x;
  if (i >= (size_t)g.T * g.N) return;
  const int t = (int)(i / g.N), n = (int)(i % g.N);
  const int NW = MODE == MODE_SWIGLU ? 2 * g.N : g.N;
  float a = 0.0f, u = 0.0f;
  for (int s = 0; s < g.ksplit; ++s) {
    const float *pp = g.part + ((size_t)s * g.T + t) * NW;
    a += pp[n];
    if (MODE == MODE_SWIGLU) u += pp[g.N + n];
  }
  gemm_store<MODE>(g, t, n, a, u);
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

// Causal attention of the block's rows on the matrix cores (InferenceCore.java:105-144:
// scores q.k / sqrt(head_dim), softmax over positions 0 .. pos, weighted sum of
// v), flash style: one wave per (16 query rows, query head), over 16-position
// tiles of the cache up to the block's last row.  Per tile:
//   S^T[16 pos][16 rows] = K[16][hd] . Q^T    v_mfma_f32_16x16x32_f16 (q as hi + lo fp16)
//   online softmax per row (a column of S^T: the four lanes l, l^16, l^32, l^48)
//   O[16 rows][hd]     += P[16][16] . V        v_mfma_f32_16x16x16_f16 (p as hi + lo fp16)
// S^T puts the positions on the rows so that P comes out of the first product
// already in the A-operand layout of the second.  The next tile's K and V are
// loaded while the current one is computed.  Positions past a row's own are
// masked (and V past the block's last row zeroed: cache rows there may hold
// anything).  Output as hi / lo planes.
template <int HD>
__global__ __launch_bounds__(PBS) void attn_rows_kernel(ModelDev m, int layer, const float *QKV, int p0, int T,
                                                        _Float16 *Oh, _Float16 *Ol) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  constexpr int NC = HD / 32, NB = HD / 16;
  const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
  const int hh = lane % 16, kb = lane / 16;
  const int G = m.n_heads / m.n_kv;
  const int item = blockIdx.x * (PBS / GL3_WAVE) + wave;  // ((row block * n_kv) + kv head) * G + group member
  const int g = item % G, kvh = (item / G) % m.n_kv, rb = item / (G * m.n_kv);
  if (rb * 16 >= T) return;  // the whole wave leaves; nothing below synchronizes the workgroup
  const int h = kvh * G + g, t0 = rb * 16;
  const int last = p0 + min(t0 + 15, T - 1);        // last position any row of the block attends
  const int qpos = min(p0 + t0 + hh, last);          // position of this lane's query row (column hh)
  const int stride = m.q_dim + 2 * m.kv_dim;
  // q of row t0 + hh as the B operand (column hh), dims 32c + 8kb .. + 7, hi and lo parts
  ph8 qh[NC], ql[NC];
  {
    const float *qr = QKV + (size_t)min(t0 + hh, T - 1) * stride + h * HD;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 a = *(const float4 *)(qr + 32 * c + 8 * kb), b = *(const float4 *)(qr + 32 * c + 8 * kb + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const _Float16 hv = (_Float16)x[i];
        qh[c][i] = hv;
        ql[c][i] = (_Float16)(x[i] - (float)hv);
      }
    }
  }
  const uint16_t *kc = m.kc + ((size_t)layer * m.n_kv + kvh) * m.ctxp * HD;
  const uint2 *vt = (const uint2 *)(m.vc + ((size_t)layer * m.n_kv + kvh) * HD * m.ctxp);
  pf4 O[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) O[b] = pf4{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun = -INFINITY, lrun = 0.0f;
  // tile operands: K rows ts + hh (A: row hh, dims 32c + 8kb ..), V dims 16b + hh at positions 4kb .. 4kb + 3 (B)
  ph8 kw[NC];
  uint2 vw[NB];
  auto load = [&](int ts, ph8 (&k)[NC], uint2 (&v)[NB]) {
    const uint16_t *kr = kc + (size_t)(ts + hh) * HD;
#pragma unroll
    for (int c = 0; c < NC; ++c) k[c] = *(const ph8 *)(kr + 32 * c + 8 * kb);
    const uint2 *vb = vt + (size_t)(ts / 16) * HD * 4;
#pragma unroll
    for (int b = 0; b < NB; ++b) v[b] = vb[(16 * b + hh) * 4 + kb];
  };
  load(0, kw, vw);
  for (int ts = 0; ts <= last; ts += 16) {
    ph8 kn[NC];
    uint2 vn[NB];
    if (ts + 16 <= last) load(ts + 16, kn, vn);  // the next tile in flight during this one
    pf4 sacc = pf4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kw[c], qh[c], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kw[c], ql[c], sacc, 0, 0, 0);
    }
    // lane: positions ts + 4kb + v, query row hh
    float sv[4], mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sv[v] = ts + 4 * kb + v <= qpos ? sacc[v] / m.sqrt_hd : -INFINITY;
      mx = fmaxf(mx, sv[v]);
    }
    mx = xrow_max(mx);
    const float mn = fmaxf(mrun, mx);  // finite: position 0 is in every row's first tile
    const float cf = mrun == -INFINITY ? 0.0f : __expf(mrun - mn);
    float p4[4], ls = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      p4[v] = sv[v] == -INFINITY ? 0.0f : __expf(sv[v] - mn);
      ls += p4[v];
    }
    ls = xrow_sum(ls);
    lrun = lrun * cf + ls;
    mrun = mn;
    // O rows are query rows 4kb + v: their factors live in column 4kb + v (lane 4kb + v holds it)
    float cr[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) cr[v] = __shfl(cf, 4 * kb + v);
    h4 ph, plo;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const _Float16 hv = (_Float16)p4[v];
      ph[v] = hv;
      plo[v] = (_Float16)(p4[v] - (float)hv);
    }
    // V rows past the block's last position are zeroed (p is 0 there, but 0 * inf is not)
    const int nvalid = min(16, last + 1 - ts);
    const unsigned keep0 = (4 * kb + 0 < nvalid ? 0x0000ffffu : 0u) | (4 * kb + 1 < nvalid ? 0xffff0000u : 0u);
    const unsigned keep1 = (4 * kb + 2 < nvalid ? 0x0000ffffu : 0u) | (4 * kb + 3 < nvalid ? 0xffff0000u : 0u);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int v = 0; v < 4; ++v) O[b][v] *= cr[v];
      const uint2 w = make_uint2(vw[b].x & keep0, vw[b].y & keep1);
      const h4 vb = __builtin_bit_cast(h4, w);
      O[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vb, O[b], 0, 0, 0);
      O[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo, vb, O[b], 0, 0, 0);
    }
    if (ts + 16 <= last) {
#pragma unroll
      for (int c = 0; c < NC; ++c) kw[c] = kn[c];
#pragma unroll
      for (int b = 0; b < NB; ++b) vw[b] = vn[b];
    }
  }
  // O[b][v]: query row t0 + 4kb + v, dim 16b + hh; divided by that row's l (column 4kb + v)
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float l = __shfl(lrun, 4 * kb + v);
    const int t = t0 + 4 * kb + v;
    if (t >= T) continue;
    const size_t ob = (size_t)t * m.q_dim + (size_t)h * HD;
#pragma unroll
    for (int b = 0; b < NB; ++b) put_split(Oh, Ol, ob + 16 * b + hh, O[b][v] / l);
  }
}

bool prefill_supported(const ModelDev &m) {
  return (m.hd == 64 || m.hd == 96 || m.hd == 128) && m.dim % GBK == 0 && m.q_dim % GBK == 0 &&
         m.hidden % GBK == 0 && m.rope_cos != nullptr;
}

// K splits of a product with `base` output tiles: enough for ~512 workgroups
// when the tiles alone leave CUs without one; for long reductions (K >= 4096)
// also enough for ~768 when they leave CUs with a single one (two fit a CU, and
// a lone workgroup per CU leaves the loads of its one stage in flight
// uncovered: measured 9% faster Llama-3.1-8B prefill, while on short
// reductions the partials' reduce costs more than it saves: 9% slower
// Qwen3-0.6B).  Each split is at least 4 stages long and the split count
// divides the K / 64 stages.  The partials then take at most (target + base) *
// 64 * 128 < 1280 * 64 * 128 floats (GL3_PREFILL_PART_FLOATS).
static int gemm_ksplit(int base, int K) {
  const int target = base < 256 ? 512 : (K >= 4096 && base < 512 ? 768 : 0);
  if (target == 0) return 1;
  int s = std::min((target + base - 1) / base, K / (4 * GBK));
  while (s > 1 && (K / GBK) % s) --s;
  return std::max(s, 1);
}

hipError_t launch_prefill_gemm(int fmt, int mode, const Mat &W, int N, const _Float16 *Xh, const _Float16 *Xl, int T,
                               float *Y, _Float16 *Yh, _Float16 *Yl, float *part, hipStream_t s) {
  if (W.cols % GBK != 0 || T <= 0 || N <= 0) return hipErrorInvalidValue;
  GemmArgs g{W.q, W.s, N, W.cols, Xh, Xl, T, Y, Yh, Yl, part, 1};
  const int nt = mode == MODE_SWIGLU ? (N + GBN / 2 - 1) / (GBN / 2) : (N + GBN - 1) / GBN, tt = (T + GBT - 1) / GBT;
  g.ksplit = gemm_ksplit(nt * tt, g.K);
  const dim3 grid(nt, tt, g.ksplit);
  const unsigned rgrid = (unsigned)(((size_t)T * N + PBS - 1) / PBS);
#define GL3_GEMM(F, M)                                                                   \
  if (fmt == F && mode == M) {                                                           \
    hipLaunchKernelGGL((gemm_kernel<F, M>), grid, dim3(PBS), 0, s, g);                   \
    if (g.ksplit > 1) hipLaunchKernelGGL((gemm_reduce_kernel<M>), dim3(rgrid), dim3(PBS), 0, s, g); \
    return hipGetLastError();                                                            \
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
  const int waves = (T + 15) / 16 * m.n_heads;  // one wave per (16 rows, query head)
  const int grid = (waves + PBS / GL3_WAVE - 1) / (PBS / GL3_WAVE);
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
