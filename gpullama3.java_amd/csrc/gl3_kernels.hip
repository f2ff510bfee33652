// Kernels of the decode path and their launch helpers.
//
//  * per-phase kernels: embed, GEMV (store / residual / SwiGLU / logits),
//    attention, step advance — one launch each, captured once per plan in a
//    hipGraph and replayed per token;
//  * decode_step_kernel<Shape>: up to 256 tokens in one cooperative launch,
//    one workgroup per CU; phases hand their outputs on as tagged cells (each
//    read waits for its producer), one grid barrier between tokens;
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

// Rows per wave for the per-phase kernels: small tiles, many resident waves.
template <int KC, int NP>
struct DefaultNR {
  static constexpr int v = (4 / (KC * NP)) > 0 ? (4 / (KC * NP)) : 1;
};

template <class P>
__global__ __launch_bounds__(GL3_BLOCK) void gemv_kernel(Mat W, int out_rows, const float *x, const float *normw,
                                                         float eps, float *y, unsigned long long *best) {
  extern __shared__ float lds[];
  P::run(W, out_rows, InPlain{x}, normw, eps, OutPlain{y}, best, blockIdx.x, gridDim.x, lds);
}

// Workgroups of a GEMV kernel that fit on the device at once (occupancy with
// the phase's LDS, times the CU count).  A workgroup stages (and normalizes)
// the input vector once and then strides over its items, so a grid of one
// resident round amortizes the staging over all the items it holds.
template <class P>
static int resident_gemv_grid(size_t lds) {
  int dev = 0, n_cu = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess)
    return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_kernel<P>, GL3_BLOCK, lds) != hipSuccess)
    return 0;
  return per_cu * n_cu;
}

template <class P>
static hipError_t launch_gemv_t(const Mat &W, int out_rows, const float *x, const float *normw, float eps, float *y,
                                unsigned long long *best, int grid, hipStream_t s) {
  const int items = P::items(out_rows);
  if (grid <= 0) {
    // the LDS of the phase grows by a few floats per item a workgroup holds: size the occupancy query for 4 KB more
    const int res = resident_gemv_grid<P>(P::lds_bytes(W.cols, out_rows, items, normw != nullptr) + 4096);
    grid = res > 0 && res < items ? res : items;
    if (grid > 8192) grid = 8192;
  }
  size_t lds = P::lds_bytes(W.cols, out_rows, grid, normw != nullptr);
  hipLaunchKernelGGL(gemv_kernel<P>, dim3(grid), dim3(GL3_BLOCK), lds, s, W, out_rows, x, normw, eps, y, best);
  return hipGetLastError();
}

int gemv_n(int fmt, int K) {
  const int per = (fmt == FMT_Q8 ? 16 : 8) * GL3_WAVE;
  return (K % per == 0) ? K / per : -1;
}

bool gemv_fast(int fmt, int K) {
  const int n = gemv_n(fmt, K);
#define GL3_SUP(F, N, KC, KS) if (fmt == F && n == N) return true;
  GL3_GEMV_LIST(GL3_SUP)
#undef GL3_SUP
  return false;
}

bool gemv_supported(int fmt, int K) { return gemv_fast(fmt, K) || gemv_any_supported(fmt, K); }

hipError_t launch_gemv(int fmt, int mode, const Mat &W, int out_rows, const float *x, const float *normw, float eps,
                       float *y, unsigned long long *best, int grid, hipStream_t s) {
  const int n = gemv_n(fmt, W.cols);
#define GL3_DISPATCH(F, N, KC, KS)                                                                                 \
  if (fmt == F && n == N) {                                                                                         \
    switch (mode) {                                                                                                 \
      case MODE_STORE:                                                                                              \
        return launch_gemv_t<GemvPhase<F, KC, KS, DefaultNR<KC, 1>::v, MODE_STORE, GL3_BLOCK>>(W, out_rows, x, normw, eps, y,  \
                                                                                    best, grid, s);                 \
      case MODE_RESIDUAL:                                                                                           \
        return launch_gemv_t<GemvPhase<F, KC, KS, DefaultNR<KC, 1>::v, MODE_RESIDUAL, GL3_BLOCK>>(W, out_rows, x, normw, eps, \
                                                                                       y, best, grid, s);           \
      case MODE_SWIGLU:                                                                                             \
        return launch_gemv_t<GemvPhase<F, KC, KS, DefaultNR<KC, 2>::v, MODE_SWIGLU, GL3_BLOCK>>(W, out_rows, x, normw, eps, y, \
                                                                                     best, grid, s);                \
      default:                                                                                                      \
        return launch_gemv_t<GemvPhase<F, KC, KS, DefaultNR<KC, 1>::v, MODE_LOGITS, GL3_BLOCK>>(W, out_rows, x, normw, eps, y, \
                                                                                     best, grid, s);                \
    }                                                                                                               \
  }
  GL3_GEMV_LIST(GL3_DISPATCH)
#undef GL3_DISPATCH
  // a width outside the compiled tiles
  return launch_gemv_any(fmt, mode, W, out_rows, x, normw, eps, y, best, grid, s);
}

template <class P>
__global__ __launch_bounds__(GL3_BLOCK) void logits_kernel(ModelDev m) {
  extern __shared__ float lds[];
  const int parity = ld_coherent_i32(&m.st->parity);
  const int nbest = ld_coherent_i32(&m.st->nbest);
  P::run(m.cls, m.vocab, InPlain{m.x}, m.out_norm, m.eps, OutPlain{m.logits}, m.best + (size_t)parity * nbest,
         blockIdx.x, gridDim.x, lds);
}

hipError_t launch_logits(const ModelDev &m, int grid, hipStream_t s) {
  const int n = gemv_n(m.cls_fmt, m.dim);
#define GL3_LOGITS(F, N, KC, KS)                                                                     \
  if (m.cls_fmt == F && n == N) {                                                                    \
    typedef GemvPhase<F, KC, KS, DefaultNR<KC, 1>::v, MODE_LOGITS, GL3_BLOCK> P;                                \
    hipLaunchKernelGGL(logits_kernel<P>, dim3(grid), dim3(GL3_BLOCK), P::lds_bytes(m.dim, m.vocab, grid, true), s, m); \
    return hipGetLastError();                                                                        \
  }
  GL3_GEMV_LIST(GL3_LOGITS)
#undef GL3_LOGITS
  return launch_logits_any(m, grid, s);  // a width outside the compiled tiles
}

// ------------------------------------------------------ per-phase kernels

__global__ __launch_bounds__(GL3_BLOCK) void embed_kernel(ModelDev m) {
  __shared__ int si_lds[8];
  StepInfo si = read_step(m, si_lds);
  phase_embed<false>(m, si.token, blockIdx.x, gridDim.x);
}

template <int HD, int GQ>
__global__ __launch_bounds__(GL3_STEP_BLOCK) void attention_kernel(ModelDev m, int layer) {
  extern __shared__ float lds[];
  __shared__ int si_lds[8];
  StepInfo si = read_step(m, si_lds);
  phase_attention<HD, GQ, GL3_STEP_BLOCK, false>(m, layer, si.pos, blockIdx.x, gridDim.x, lds);
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

size_t attention_lds_bytes(int hd, int G, int max_split) {
  return (size_t)att_lds_floats(hd, G, GL3_STEP_BLOCK / GL3_WAVE, max_split) * sizeof(float);
}


hipError_t launch_embed(const ModelDev &m, hipStream_t s) {
  int grid = (m.dim + GL3_BLOCK - 1) / GL3_BLOCK;
  hipLaunchKernelGGL(embed_kernel, dim3(grid), dim3(GL3_BLOCK), 0, s, m);
  return hipGetLastError();
}
hipError_t launch_attention(const ModelDev &m, int layer, hipStream_t s) {
  const int grid = m.n_kv * m.max_split;
  const int G = m.n_heads / m.n_kv;
  const size_t lds = attention_lds_bytes(m.hd, G, m.max_split);
#define GL3_ATT(HD_, G_)                                                                                        \
  if (m.hd == HD_ && G == G_) {                                                                                 \
    hipLaunchKernelGGL((attention_kernel<HD_, G_>), dim3(grid), dim3(GL3_STEP_BLOCK), lds, s, m, layer);        \
    return hipGetLastError();                                                                                   \
  }
  GL3_ATT(64, 1) GL3_ATT(64, 2) GL3_ATT(64, 3) GL3_ATT(64, 4) GL3_ATT(64, 8)
  GL3_ATT(96, 1) GL3_ATT(96, 2) GL3_ATT(96, 3) GL3_ATT(96, 4) GL3_ATT(96, 8)
  GL3_ATT(128, 1) GL3_ATT(128, 2) GL3_ATT(128, 3) GL3_ATT(128, 4) GL3_ATT(128, 8)
#undef GL3_ATT
  return hipErrorInvalidValue;
}
bool attention_supported(int hd, int G) {
  return (hd == 64 || hd == 96 || hd == 128) && (G == 1 || G == 2 || G == 3 || G == 4 || G == 8);
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

// Compile-time shapes of the models the persistent kernel is built for.  Each
// GEMV phase lists its tile (KC chunks per lane, KS waves splitting K, NR rows
// per wave) for 4-wave workgroups, chosen so that a wave's tile fills one ring
// slot of SC chunks and the work items of every phase spread evenly over the
// CUs.  DEPTH ring slots per wave are in flight.  Qwen3-4B FP16 (K = 2560: five
// 512-element rounds per row) takes 12-chunk slots so that a gate/up row pair
// is one slot-load, two of them in flight, and two K/V tiles in flight in the
// attention phase, which keeps the ring within LDS.
template <int KC_, int KS_, int NR_>
struct Tile {
  static constexpr int KC = KC_, KS = KS_, NR = NR_;
};
// FFN 1: fused FFN (gate/up rows in contiguous runs of 32 per workgroup, each
// multiplied by its 32-column slice of Wdown, partials reduced by row);
// needs Q8_0, a two-slot ring, hidden = 32 x grid, dim = R x grid, R <= 8, and
// gate/up tiles such that a workgroup's 32 rows are four slot-loads (held in
// ring slots 0..3 at once).
template <int FMT_, int DIM, int QD, int KVD, int HID, int HD, int G, int SC, int DEPTH, class TQKV, class TWO,
          class TGU, class TDN, class TCLS, int FFN = 0, int ATTD = ATT_DEPTH>
struct Shape {
  static constexpr int fmt = FMT_, dim = DIM, q_dim = QD, kv_dim = KVD, hidden = HID, hd = HD, gqa = G;
  static constexpr int ffn = FFN;
  static constexpr int att_depth = ATTD;  // K/V tiles in flight per wave in the attention phase
  static constexpr int BS = GL3_STEP_BLOCK;
  typedef GemvPhase<FMT_, TQKV::KC, TQKV::KS, TQKV::NR, MODE_STORE, BS, SC, DEPTH> QKV;
  typedef GemvPhase<FMT_, TWO::KC, TWO::KS, TWO::NR, MODE_RESIDUAL, BS, SC, DEPTH> WO;
  // fused FFN: the four gate/up slot-loads of a workgroup are all requested ahead (ring slots 0..3)
  typedef GemvPhase<FMT_, TGU::KC, TGU::KS, TGU::NR, MODE_SWIGLU, BS, SC, FFN == 1 ? 4 : DEPTH, FFN> GU;
  typedef DownSliceQ8<BS, DEPTH> DS;
  typedef GemvPhase<FMT_, TDN::KC, TDN::KS, TDN::NR, MODE_RESIDUAL, BS, SC, DEPTH> DOWN;
  typedef GemvPhase<FMT_, TCLS::KC, TCLS::KS, TCLS::NR, MODE_LOGITS, BS, SC, DEPTH> CLS;
};

//                  fmt     dim   q_dim kv_dim hidden hd  G SC D  QKV           WO            GU            DOWN          CLS
typedef Shape<FMT_Q8,  2048, 2048,  512,  8192,  64, 4, 8, 2, Tile<2, 1, 3>, Tile<2, 1, 2>, Tile<2, 1, 2>, Tile<2, 4, 4>, Tile<2, 1, 4>, 1> ShapeLlama1BQ8;
typedef Shape<FMT_F16, 2048, 2048,  512,  8192,  64, 4, 8, 3, Tile<4, 1, 3>, Tile<4, 1, 2>, Tile<4, 1, 1>, Tile<4, 4, 2>, Tile<4, 1, 2>> ShapeLlama1BF16;
typedef Shape<FMT_Q8,  1024, 2048, 1024,  3072, 128, 2, 8, 3, Tile<1, 1, 4>, Tile<1, 2, 2>, Tile<1, 1, 3>, Tile<3, 1, 1>, Tile<1, 1, 8>> ShapeQwen3_06BQ8;
typedef Shape<FMT_F16, 3072, 3072, 3072,  8192,  96, 1, 8, 3, Tile<6, 1, 1>, Tile<6, 1, 1>, Tile<3, 2, 1>, Tile<4, 4, 2>, Tile<6, 1, 1>> ShapePhi3MiniF16;
typedef Shape<FMT_Q8,  4096, 4096, 1024, 14336, 128, 4, 8, 2, Tile<4, 1, 2>, Tile<4, 1, 2>, Tile<4, 1, 1>, Tile<7, 2, 1>, Tile<4, 1, 2>> ShapeLlama8BQ8;
typedef Shape<FMT_Q8,  3072, 3072, 1024,  8192, 128, 3, 8, 2, Tile<3, 1, 2>, Tile<3, 1, 2>, Tile<3, 1, 1>, Tile<4, 2, 1>, Tile<3, 1, 2>> ShapeLlama3BQ8;
typedef Shape<FMT_Q8,  3072, 3072, 3072,  8192,  96, 1, 8, 2, Tile<3, 1, 1>, Tile<3, 1, 1>, Tile<3, 1, 1>, Tile<4, 2, 1>, Tile<3, 1, 2>> ShapePhi3MiniQ8;
typedef Shape<FMT_F16, 4096, 4096, 1024, 14336, 128, 4, 8, 3, Tile<8, 1, 1>, Tile<8, 1, 1>, Tile<4, 2, 1>, Tile<7, 4, 1>, Tile<8, 1, 1>> ShapeMistral7BF16;
typedef Shape<FMT_F16, 2560, 4096, 1024,  9728, 128, 4, 12, 2, Tile<5, 1, 2>, Tile<2, 4, 5>, Tile<5, 1, 1>, Tile<19, 1, 1>, Tile<5, 1, 2>, 0, 2> ShapeQwen3_4BF16;

// The fused FFN's Wdown slice (two slot-loads), requested into ring slots 0
// and 1 as soon as gate/up's dot products are done with them, so it streams
// while gate/up finishes.
template <class DS>
struct DownSliceAfterGateUp {
  Mat W;
  int rows, slice;
  __device__ __forceinline__ void operator()() {}
  __device__ __forceinline__ void after(int u) {
    if (u == 0) DS::template issue<0>(W, rows, slice, 0);
    if (u == 1) DS::template issue<1>(W, rows, slice, 1);
  }
};

// Fused FFN, a workgroup with an attention item: gate/up's slot-load 1 goes
// into ring slot 1 (free once the item's tiles are done) as soon as the item's
// outputs are stored, ahead of the split merge's reads.  Measured on the
// Llama-3.2-1B Q8_0 shape: +0.8% tokens/s; slot-loads 1-2 there: -0.6%, 1-3: -2%
// (the merge's reads return behind them).
template <class GU>
struct GateUpAfterAttention {
  Mat W;
  int rows, blk, nblk;
  __device__ __forceinline__ void operator()() { GU::template issue<1>(W, rows, 1, blk, nblk); }
};

// n_steps greedy decode steps in one launch: per step embedding, L x (QKV,
// attention, Wo, gate/up, down), classifier.  Inside a step no phase waits at
// a barrier: each reads its input vector as tagged cells and waits only for
// the cells it reads (TagWait).  Every workgroup holds items of every GEMV
// phase (the host sizes the grid so), which makes one buffer per vector (two
// for the residual stream) safe against overwriting: a workgroup that writes
// a vector again has waited, through the cells it read in between, for every
// workgroup to finish reading the previous contents.  A grid barrier between
// steps makes the argmax keys, the advanced control block and the appended
// KV rows visible.  Each GEMV phase requests its first weight tiles before
// it waits for its input (weights do not depend on it).
//
// Tags: tag0 + (1 + 5 L) s for step s's embedding, then 5 per layer (q/k/v,
// attention, Wo output, SwiGLU, down output).
template <class SH>
__global__ __launch_bounds__(GL3_STEP_BLOCK, 1) void decode_step_kernel(ModelDev m, GridBarrier gb, unsigned epoch,
                                                                        unsigned tag, int n_steps) {
  extern __shared__ float lds[];
  __shared__ int si_lds[8];
  const int blk = blockIdx.x, nblk = gridDim.x;
  const int rows_qkv = SH::q_dim + 2 * SH::kv_dim;
  const TagWait tw{gb.err, gb.spin_limit};
  // layer descriptors are loaded where they are used (scalar loads), so only
  // the current phase's matrix occupies registers
  const cLayerDev *layers = (const cLayerDev *)m.layers;
  for (int step = 0; step < n_steps; ++step) {
    int tk = 0;
    trace(m, tk++);
    StepInfo si = read_step(m, si_lds);
    unsigned t_x = tag++;  // tag of the residual stream in txa
    phase_embed<true>(m, si.token, blk, nblk, t_x);
    if (step == 0) SH::QKV::prefetch(ld_mat(&layers[0].qkv), rows_qkv, blk, nblk);  // later steps: at the step boundary
    trace(m, tk++);
    trace(m, tk++);
    for (int l = 0; l < m.n_layers; ++l) {
      const cLayerDev *L = layers + l;
      const unsigned t_qkv = tag, t_att = tag + 1, t_wo = tag + 2, t_hb = tag + 3, t_dn = tag + 4;
      tag += 5;
      SH::QKV::run(ld_mat(&L->qkv), rows_qkv, InTag{m.txa, t_x, tw}, L->attn_norm, m.eps,
                   OutTag{m.tqkv, t_qkv, nullptr, 0u, tw}, nullptr, blk, nblk, lds, true);
      trace(m, tk++);
      // attention streams K/V through the GEMV ring: Wo's tiles are requested after it
      // (two stamps inside: q/k/v read, tiles done)
      const int msplit = att_tag_splits(m, si.pos + 1, nblk, SH::ffn == 1);
      if constexpr (SH::ffn == 1)
        phase_attention<SH::hd, SH::gqa, SH::BS, true, SH::QKV::WCH, SH::att_depth>(
            m, l, si.pos, blk, nblk, lds, t_qkv, t_att, tw, m.tstamp ? tk : -1,
            GateUpAfterAttention<typename SH::GU>{ld_mat(&L->gu), SH::hidden, blk, nblk}, msplit);
      else
        phase_attention<SH::hd, SH::gqa, SH::BS, true, SH::QKV::WCH, SH::att_depth>(
            m, l, si.pos, blk, nblk, lds, t_qkv, t_att, tw, m.tstamp ? tk : -1, NoTail{}, msplit);
      tk += 2;
      trace(m, tk++);
      // workgroups without an attention item wait quietly for the attention output
      const int S = att_split_len(si.pos + 1, msplit, 16 * (SH::BS / GL3_WAVE));
      const bool att_wg = blk < m.n_kv * ((si.pos + S) / S);
      SH::WO::prefetch(ld_mat(&L->wo), SH::dim, blk, nblk);
      if constexpr (SH::ffn == 1) {
        // fused FFN: gate/up's slot-loads 1..3 go into ring slots 1..3 (free
        // during Wo) while the workgroup has nothing else to read: before the
        // wait for the attention output when it holds no attention item, else
        // slot-load 1 after the item's outputs and 2..3 once Wo's output is
        // stored; slot-load 0 follows Wo (slot 0 holds Wo)
        const Mat wgu = ld_mat(&L->gu);
        if (!att_wg) {
          SH::GU::template issue<1>(wgu, SH::hidden, 1, blk, nblk);
          SH::GU::template issue<2>(wgu, SH::hidden, 2, blk, nblk);
          SH::GU::template issue<3>(wgu, SH::hidden, 3, blk, nblk);
          quiet_wait(m.tatt, SH::gqa * SH::hd, SH::gqa * SH::hd - 1, m.n_kv, t_att, tw);
        }
        SH::WO::run(ld_mat(&L->wo), SH::dim, InTag{m.tatt, t_att, tw}, nullptr, m.eps,
                    OutTag{m.txb, t_wo, m.txa, t_x, tw}, nullptr, blk, nblk, lds, true);
        trace(m, tk++);
        if (att_wg) {
          // slot-load 1 went out after the attention item
          SH::GU::template issue<2>(wgu, SH::hidden, 2, blk, nblk);
          SH::GU::template issue<3>(wgu, SH::hidden, 3, blk, nblk);
        }
        SH::GU::template issue<0>(wgu, SH::hidden, 0, blk, nblk);
        trace(m, tk++);
        // this workgroup's 32 SwiGLU rows stay in LDS and meet its 32-column
        // slice of Wdown; t_hb tags the partial sums
        const Mat wds = ld_mat(&L->down_sl);
        SH::GU::run(wgu, SH::hidden, InTag{m.txb, t_wo, tw}, L->ffn_norm, m.eps, OutNone{}, nullptr, blk, nblk, lds,
                    true, DownSliceAfterGateUp<typename SH::DS>{wds, SH::dim, blk});
        trace(m, tk++);
        trace(m, tk++);
        SH::DS::template run<0, 1>(SH::dim, lds + SH::GU::obuf_offset(SH::dim, true), m.tdp + (size_t)blk * SH::dim,
                                   t_hb);
        trace(m, tk++);
        // the reduce polls the partials first: weight requests issued before them
        // would hold up their returns (in issue order per CU), so the next phase's
        // weights are requested after it (measured 0.7-1.0% faster per token)
        phase_reduce<SH::BS>(m.tdp, SH::dim, m.txb, t_wo, m.txa, t_dn, t_hb, tw, blk, nblk, lds);
        if (l + 1 < m.n_layers)
          SH::QKV::prefetch(ld_mat(&layers[l + 1].qkv), rows_qkv, blk, nblk);
        else
          SH::CLS::prefetch(m.cls, m.vocab, blk, nblk);
        trace(m, tk++);
      } else {
        if (!att_wg) quiet_wait(m.tatt, SH::gqa * SH::hd, SH::gqa * SH::hd - 1, m.n_kv, t_att, tw);
        SH::WO::run(ld_mat(&L->wo), SH::dim, InTag{m.tatt, t_att, tw}, nullptr, m.eps,
                    OutTag{m.txb, t_wo, m.txa, t_x, tw}, nullptr, blk, nblk, lds, true);
        trace(m, tk++);
        SH::GU::prefetch(ld_mat(&L->gu), SH::hidden, blk, nblk);
        trace(m, tk++);
        SH::GU::run(ld_mat(&L->gu), SH::hidden, InTag{m.txb, t_wo, tw}, L->ffn_norm, m.eps,
                    OutTag{m.thb, t_hb, nullptr, 0u, tw}, nullptr, blk, nblk, lds, true);
        trace(m, tk++);
        SH::DOWN::prefetch(ld_mat(&L->down), SH::dim, blk, nblk);
        trace(m, tk++);
        SH::DOWN::run(ld_mat(&L->down), SH::dim, InTag{m.thb, t_hb, tw}, nullptr, m.eps,
                      OutTag{m.txa, t_dn, m.txb, t_wo, tw}, nullptr, blk, nblk, lds, true);
        trace(m, tk++);
        if (l + 1 < m.n_layers)
          SH::QKV::prefetch(ld_mat(&layers[l + 1].qkv), rows_qkv, blk, nblk);
        else
          SH::CLS::prefetch(m.cls, m.vocab, blk, nblk);
        trace(m, tk++);
      }
      t_x = t_dn;
    }
    SH::CLS::run(m.cls, m.vocab, InTag{m.txa, t_x, tw}, m.out_norm, m.eps, OutPlain{m.logits},
                 m.best + (size_t)si.parity * si.nbest, blk, nblk, lds, true);
    trace(m, tk++);
    // every workgroup has read the control block: workgroup 0 waited, through
    // the classifier input, for all down-projection rows, which every
    // workgroup wrote after its read_step
    if (blk == 0) advance_step(m, si);
    if (step + 1 < n_steps) {
      // the next step reads every workgroup's argmax key and the advanced state
      grid_arrive(gb);
      SH::QKV::prefetch(ld_mat(&layers[0].qkv), rows_qkv, blk, nblk);
      if (!grid_wait(gb, ++epoch)) return;
    }
  }
}

template <class SH>
static bool shape_matches(const ModelDev &m) {
  return m.fmt == SH::fmt && m.cls_fmt == SH::fmt && m.dim == SH::dim && m.q_dim == SH::q_dim &&
         m.kv_dim == SH::kv_dim && m.hidden == SH::hidden && m.hd == SH::hd && m.n_heads / m.n_kv == SH::gqa;
}

template <class SH>
static size_t step_lds_bytes(const ModelDev &m, int grid) {
  size_t b = attention_lds_bytes(m.hd, m.n_heads / m.n_kv, m.max_split);
  const int rows_qkv = SH::q_dim + 2 * SH::kv_dim;
  size_t g[5] = {SH::QKV::lds_bytes(SH::dim, rows_qkv, grid, true), SH::WO::lds_bytes(SH::q_dim, SH::dim, grid, false),
                 SH::GU::lds_bytes(SH::dim, SH::hidden, grid, true),
                 SH::DOWN::lds_bytes(SH::hidden, SH::dim, grid, false),
                 SH::CLS::lds_bytes(SH::dim, m.vocab, grid, true)};
  for (size_t v : g) b = v > b ? v : b;
  return b;
}

template <class SH>
static StepKernel make_step_kernel(const ModelDev &m, int grid) {
  StepKernel k;
  k.fn = (const void *)decode_step_kernel<SH>;
  k.lds_bytes = step_lds_bytes<SH>(m, grid);
  k.tags_per_step = 1 + 5 * m.n_layers;  // grid barriers: one between consecutive steps of a launch
  const int rows_qkv = SH::q_dim + 2 * SH::kv_dim;
  const int items[5] = {SH::QKV::items(rows_qkv), SH::WO::items(SH::dim), SH::GU::items(SH::hidden),
                        SH::DOWN::items(SH::dim), SH::CLS::items(m.vocab)};
  k.max_grid = items[0];
  for (int v : items) k.max_grid = v < k.max_grid ? v : k.max_grid;
  k.ffn = SH::ffn;
  if (SH::ffn == 1) {
    // one 32-column slice of Wdown per workgroup: the grid is fixed
    k.req_grid = SH::hidden / 32;
    const bool ok = SH::GU::items(SH::hidden) % k.req_grid == 0 && SH::dim % k.req_grid == 0 &&
                    SH::dim / k.req_grid <= 8 && SH::dim % (2 * SH::DS::RPU) == 0 && SH::dim == 2 * SH::DS::RPU &&
                    SH::GU::local_items(SH::hidden, 0, k.req_grid) * SH::GU::PASSES == 4;
    if (!ok || k.req_grid > k.max_grid) k.req_grid = -1;  // this shape cannot run fused
  }
  return k;
}

bool find_step_kernel(const ModelDev &m, int grid, StepKernel *out) {
  if (shape_matches<ShapeLlama1BQ8>(m)) { *out = make_step_kernel<ShapeLlama1BQ8>(m, grid); return true; }
  if (shape_matches<ShapeLlama1BF16>(m)) { *out = make_step_kernel<ShapeLlama1BF16>(m, grid); return true; }
  if (shape_matches<ShapeQwen3_06BQ8>(m)) { *out = make_step_kernel<ShapeQwen3_06BQ8>(m, grid); return true; }
  if (shape_matches<ShapePhi3MiniF16>(m)) { *out = make_step_kernel<ShapePhi3MiniF16>(m, grid); return true; }
  if (shape_matches<ShapeLlama8BQ8>(m)) { *out = make_step_kernel<ShapeLlama8BQ8>(m, grid); return true; }
  if (shape_matches<ShapeLlama3BQ8>(m)) { *out = make_step_kernel<ShapeLlama3BQ8>(m, grid); return true; }
  if (shape_matches<ShapePhi3MiniQ8>(m)) { *out = make_step_kernel<ShapePhi3MiniQ8>(m, grid); return true; }
  if (shape_matches<ShapeMistral7BF16>(m)) { *out = make_step_kernel<ShapeMistral7BF16>(m, grid); return true; }
  if (shape_matches<ShapeQwen3_4BF16>(m)) { *out = make_step_kernel<ShapeQwen3_4BF16>(m, grid); return true; }
  return false;
}

hipError_t launch_step_kernel(const StepKernel &k, const ModelDev &m, const GridBarrier &gb, unsigned epoch,
                              unsigned tag, int grid, int n_steps, hipStream_t s) {
  if (grid > k.max_grid) return hipErrorInvalidValue;  // some workgroup would hold no item of a GEMV phase
  ModelDev mm = m;
  GridBarrier gg = gb;
  unsigned e = epoch, t = tag;
  int n = n_steps;
  void *args[] = {&mm, &gg, &e, &t, &n};
  return hipLaunchCooperativeKernel(k.fn, dim3(grid), dim3(GL3_STEP_BLOCK), args, (unsigned)k.lds_bytes, s);
}

// -------------------------------------------------------------- op kernels

// Q8_0 [rows][cols] (quants, scales [rows][cols/32]) -> 32-column slices:
// q_sl[b][r][j] = q[r][32 b + j], s_sl[b][r] = s[r][b].
__global__ void slice_q8_kernel(const uint8_t *q, const uint16_t *s, int rows, int cols, uint8_t *q_sl,
                                uint16_t *s_sl) {
  const size_t nb = (size_t)cols / 32, n16 = (size_t)rows * nb * 2;  // 16-byte pieces
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x) {
    const size_t b = i / ((size_t)rows * 2), rem = i % ((size_t)rows * 2), r = rem / 2, h = rem % 2;
    *(u32x4 *)(q_sl + (b * rows + r) * 32 + h * 16) = *(const u32x4 *)(q + r * (size_t)cols + b * 32 + h * 16);
    if (h == 0) s_sl[b * rows + r] = s[r * nb + b];
  }
}
hipError_t launch_slice_q8(const uint8_t *q, const uint16_t *s, int rows, int cols, uint8_t *q_sl, uint16_t *s_sl,
                           hipStream_t st) {
  if (cols % 32 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(slice_q8_kernel, dim3(2048), dim3(256), 0, st, q, s, rows, cols, q_sl, s_sl);
  return hipGetLastError();
}

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
// rows x cols values, row stride `stride`; value (r, c) is draw number r * cols + c of `seed`
__global__ void fill_normal_f16_kernel(uint16_t *dst, size_t rows, size_t cols, size_t stride,
                                       unsigned long long seed) {
  const size_t n = rows * cols;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    unsigned long long h = splitmix64(seed ^ splitmix64(i));
    float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    float u2 = (float)((h >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);
    float r = sqrtf(-2.0f * logf(u1));
    dst[(i / cols) * stride + i % cols] = f2h(r * cospif(2.0f * u2));
  }
}

// V cache <-> position-major rows: vt is one kv head's [ctxp/16][hd][16] region,
// rows is [npos][hd] (positions pos0..pos0+npos-1)
__device__ __forceinline__ size_t vt_index(int t, int d, int hd) { return ((size_t)(t / 16) * hd + d) * 16 + t % 16; }
__global__ void vt_copy_kernel(uint16_t *vt, uint16_t *rows, int hd, int pos0, int npos, int to_vt) {
  const size_t n = (size_t)npos * hd;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(i / hd), d = (int)(i % hd);
    uint16_t *v = vt + vt_index(pos0 + t, d, hd);
    if (to_vt)
      *v = rows[i];
    else
      rows[i] = *v;
  }
}
// One layer's K / V cache <-> position-major rows [npos][n_kv * hd] of positions
// pos0 .. pos0 + npos - 1 (the reference's [pos][kvDim] order).
__global__ void kv_rows_kernel(uint16_t *kc, uint16_t *vc, uint16_t *rk, uint16_t *rv, int n_kv, int hd, int ctxp,
                               int pos0, int npos, int to_cache) {
  const size_t kv_dim = (size_t)n_kv * hd, n = (size_t)npos * kv_dim;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(i / kv_dim), c = (int)(i % kv_dim), h = c / hd, d = c % hd;
    uint16_t *k = kc + ((size_t)h * ctxp + pos0 + t) * hd + d;
    uint16_t *v = vc + (size_t)h * hd * ctxp + vt_index(pos0 + t, d, hd);
    if (to_cache) {
      *k = rk[i];
      *v = rv[i];
    } else {
      rk[i] = *k;
      rv[i] = *v;
    }
  }
}
// N(0,1) history for positions 0..npos-1 of one kv head's V region (draw d * npos + t)
__global__ void fill_normal_vt_kernel(uint16_t *vt, int hd, int npos, unsigned long long seed) {
  const size_t n = (size_t)npos * hd;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int d = (int)(i / npos), t = (int)(i % npos);
    unsigned long long h = splitmix64(seed ^ splitmix64(i));
    float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    float u2 = (float)((h >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);
    float r = sqrtf(-2.0f * logf(u1));
    vt[vt_index(t, d, hd)] = f2h(r * cospif(2.0f * u2));
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
hipError_t launch_fill_normal_f16(uint16_t *dst, size_t rows, size_t cols, size_t stride, unsigned long long seed,
                                  hipStream_t st) {
  size_t grid = (rows * cols + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (grid == 0) grid = 1;
  hipLaunchKernelGGL(fill_normal_f16_kernel, dim3((unsigned)grid), dim3(256), 0, st, dst, rows, cols, stride, seed);
  return hipGetLastError();
}
hipError_t launch_vt_copy(uint16_t *vt, uint16_t *rows, int hd, int pos0, int npos, bool to_vt, hipStream_t st) {
  size_t grid = ((size_t)npos * hd + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (grid == 0) grid = 1;
  hipLaunchKernelGGL(vt_copy_kernel, dim3((unsigned)grid), dim3(256), 0, st, vt, rows, hd, pos0, npos, to_vt ? 1 : 0);
  return hipGetLastError();
}
hipError_t launch_kv_rows(uint16_t *kc, uint16_t *vc, uint16_t *rk, uint16_t *rv, int n_kv, int hd, int ctxp, int pos0,
                          int npos, bool to_cache, hipStream_t st) {
  size_t grid = ((size_t)npos * n_kv * hd + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (grid == 0) grid = 1;
  hipLaunchKernelGGL(kv_rows_kernel, dim3((unsigned)grid), dim3(256), 0, st, kc, vc, rk, rv, n_kv, hd, ctxp, pos0, npos,
                     to_cache ? 1 : 0);
  return hipGetLastError();
}
hipError_t launch_fill_normal_vt(uint16_t *vt, int hd, int npos, unsigned long long seed, hipStream_t st) {
  size_t grid = ((size_t)npos * hd + 255) / 256;
  if (grid > 65536) grid = 65536;
  if (grid == 0) grid = 1;
  hipLaunchKernelGGL(fill_normal_vt_kernel, dim3((unsigned)grid), dim3(256), 0, st, vt, hd, npos, seed);
  return hipGetLastError();
}

}  // namespace gl3
