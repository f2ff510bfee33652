// Internal interface between the host plan (gl3_plan.hip) and the kernels
// (gl3_kernels.hip).
#pragma once

#include "gl3_phases.h"

namespace gl3 {

struct StepKernel {
  const void *fn = nullptr;
  size_t lds_bytes = 0;
  int tags_per_step = 0;  // tagged vectors written per step
  int max_grid = 0;       // largest grid in which every workgroup holds items of every GEMV phase
  int ffn = 0;            // 1: fused FFN, needs the sliced down copy, the partials buffer and grid == req_grid
  int req_grid = 0;       // fused FFN: the only grid it runs on (-1: not possible for this shape)
};

int gemv_n(int fmt, int K);
// a GEMV of this row length runs: on the compiled GemvPhase tiles, else on the any-length kernel
bool gemv_supported(int fmt, int K);
bool gemv_fast(int fmt, int K);  // the compiled tiles (and the persistent kernel's shapes) cover it

// GEMV for any row length (gl3_gemv_any.hip): K a multiple of 32 (Q8_0) or 8 (F16), up to this
#define GL3_GEMV_ANY_MAX_K 15872
bool gemv_any_supported(int fmt, int K);
hipError_t launch_gemv_any(int fmt, int mode, const Mat &W, int out_rows, const float *x, const float *normw,
                           float eps, float *y, unsigned long long *best, int grid, hipStream_t s);
hipError_t launch_logits_any(const ModelDev &m, int grid, hipStream_t s);
hipError_t launch_gemv(int fmt, int mode, const Mat &W, int out_rows, const float *x, const float *normw, float eps,
                       float *y, unsigned long long *best, int grid, hipStream_t s);
hipError_t launch_logits(const ModelDev &m, int grid, hipStream_t s);
size_t attention_lds_bytes(int hd, int G, int max_split);
bool attention_supported(int hd, int G);
hipError_t launch_embed(const ModelDev &m, hipStream_t s);
hipError_t launch_attention(const ModelDev &m, int layer, hipStream_t s);
hipError_t launch_advance(const ModelDev &m, hipStream_t s);
hipError_t launch_finish(const ModelDev &m, hipStream_t s);

bool find_step_kernel(const ModelDev &m, int grid, StepKernel *out);
hipError_t launch_slice_q8(const uint8_t *q, const uint16_t *s, int rows, int cols, uint8_t *q_sl, uint16_t *s_sl,
                           hipStream_t st);
hipError_t launch_step_kernel(const StepKernel &k, const ModelDev &m, const GridBarrier &gb, unsigned epoch,
                              unsigned tag, int grid, int n_steps, hipStream_t s);

// probs: scratch of 2 n floats (the probabilities, then the top-p candidates' indices);
// best (nullable, with st): the decode step's argmax keys, which give the maximum logit
hipError_t launch_sample(const float *logits, int n, float temperature, float topp, const float *coins, int coin_index,
                         float *probs, int *token_out, DecodeState *st, int *rec, const unsigned long long *best,
                         hipStream_t s);
hipError_t launch_repack_q8(const uint8_t *blocks, size_t nblocks, uint8_t *q, uint16_t *s, hipStream_t st);
hipError_t launch_dequant_q8(const uint8_t *q, const uint16_t *s, size_t n, float *out, hipStream_t st);
hipError_t launch_f16_to_f32(const uint16_t *in, size_t n, float *out, hipStream_t st);
hipError_t launch_fill_normal_f16(uint16_t *dst, size_t rows, size_t cols, size_t stride, unsigned long long seed,
                                  hipStream_t st);
hipError_t launch_vt_copy(uint16_t *vt, uint16_t *rows, int hd, int pos0, int npos, bool to_vt, hipStream_t st);
hipError_t launch_kv_rows(uint16_t *kc, uint16_t *vc, uint16_t *rk, uint16_t *rv, int n_kv, int hd, int ctxp, int pos0,
                          int npos, bool to_cache, hipStream_t st);
hipError_t launch_fill_normal_vt(uint16_t *vt, int hd, int npos, unsigned long long seed, hipStream_t st);

// batched prefill (gl3_prefill.hip)
bool prefill_supported(const ModelDev &m);
#define GL3_PREFILL_PART_FLOATS ((size_t)1280 * 64 * 128)  // split-K partials of one prefill matrix product
hipError_t launch_prefill_gemm(int fmt, int mode, const Mat &W, int N, const _Float16 *Xh, const _Float16 *Xl, int T,
                               float *Y, _Float16 *Yh, _Float16 *Yl, float *part, hipStream_t s);
hipError_t launch_embed_rows(const ModelDev &m, const int *tokens, int T, float *X, hipStream_t s);
hipError_t launch_rmsnorm_rows(const float *X, const float *w, float eps, int dim, int T, _Float16 *Yh, _Float16 *Yl,
                               hipStream_t s);
hipError_t launch_rope_kv_rows(const ModelDev &m, int layer, float *QKV, int p0, int T, hipStream_t s);
hipError_t launch_attn_rows(const ModelDev &m, int layer, const float *QKV, int p0, int T, _Float16 *Oh, _Float16 *Ol,
                            hipStream_t s);

}  // namespace gl3
