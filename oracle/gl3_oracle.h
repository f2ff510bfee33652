/*
 * CPU oracle for the batch-1 decode forward pass of GPULlama3.java.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a restatement, in C, of the reference's
 * CPU forward (InferenceCore.forwardJava / forwardJavaQwen3 / forwardJavaPhi3)
 * and of the tensor numerics it relies on (FloatTensor, Q8_0FloatTensor,
 * FP16FloatTensor, RoPE.precomputeFreqsCis, FloatTensor.argmax).  Only the
 * tests, the smoke check and the benchmark's CPU-baseline leg may load it; the
 * product path (libgpullama3_hip.so) never calls it.
 *
 * Every function cites the reference file:line it follows.  Paths are relative
 * to src/main/java/org/beehive/gpullama3/ of the reference repository.
 *
 * Tensor memory is borrowed, in the GGUF on-disk encodings the reference reads
 * through its mmap: F32 = float[], F16 = IEEE binary16[], Q8_0 = 34-byte blocks
 * {fp16 scale, int8 q[32]} (GGMLType.java:13).
 *
 * Pins (tests/test_oracle.py): exhaustive fp16 decode and Q8_0 dequant,
 * fp64 brute force and closed forms for GEMV, RMSNorm, RoPE, softmax, argmax
 * and attention, and fp64 golden fixtures of tiny models of every family.
 * Parity unpinned: the exact reduceLanes(ADD) order of the Java Vector API
 * dots (Q8_0FloatTensor.java:119, FP16FloatTensor.java:103; a fixed 8-lane
 * order is used here) and the last-ulp behaviour of Math.exp/cos/sin/pow (C's
 * double versions are used); the reference JVM cannot run here, so these are
 * bounded only by the parity tolerance.
 */
#ifndef GL3_ORACLE_H
#define GL3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* model families (ModelType.java); values match include/gl3.h */
enum { ORC_LLAMA = 0, ORC_MISTRAL = 1, ORC_QWEN3 = 2, ORC_PHI3 = 3 };
/* GGML type ids (GGMLType.java ordinal) */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8 };
/* tensor kinds; values match include/gl3.h */
enum {
  ORC_TOKEN_EMBD = 0, ORC_OUTPUT_NORM = 1, ORC_OUTPUT = 2,
  ORC_ATTN_NORM = 3, ORC_ATTN_Q = 4, ORC_ATTN_K = 5, ORC_ATTN_V = 6, ORC_ATTN_QKV = 7,
  ORC_ATTN_OUTPUT = 8, ORC_ATTN_Q_NORM = 9, ORC_ATTN_K_NORM = 10,
  ORC_FFN_NORM = 11, ORC_FFN_GATE = 12, ORC_FFN_UP = 13, ORC_FFN_DOWN = 14,
  ORC_KIND_COUNT = 15
};

typedef struct {
  int family;
  int dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size, context_length;
  float rms_norm_eps;
  double rope_theta;
  int weight_type;   /* GGML type of the linear weights (F16 or Q8_0) */
  int embd_type;     /* GGML type of token_embd */
  int output_type;   /* GGML type of the classifier (== embd_type when tied) */
  /* test aids (default 0 = the reference's behaviour):
   * kv_fp16   round K and V to binary16 when they are appended to the cache
   * f16_exact decode F16 weights exactly in dot products instead of the
   *           vector path's denormals-are-zero decode */
  int kv_fp16;
  int f16_exact;
  int n_threads;     /* 0 = OpenMP default */
} orc_config;

typedef struct orc_model orc_model;

orc_model *orc_create(const orc_config *cfg);
void orc_destroy(orc_model *m);
/* borrow a tensor (GGUF encoding); layer is ignored for global tensors */
int orc_set_tensor(orc_model *m, int kind, int layer, const void *data, int ggml_type);
/* zero the KV cache (fresh State) */
void orc_reset(orc_model *m);
/* one forward pass; logits_out has vocab_size floats. Returns 0 on success. */
int orc_forward(orc_model *m, int token, int position, float *logits_out);
/* direct access to the fp32 KV cache [layer][ctx][kvDim] (for prefill and checks) */
float *orc_key_cache(orc_model *m, int layer);
float *orc_value_cache(orc_model *m, int layer);
/* rope tables actually used */
const float *orc_rope_real(orc_model *m);
const float *orc_rope_imag(orc_model *m);

/* ---- primitive numerics, exported for unit tests ---- */
float orc_f16_to_f32(uint16_t h);                 /* Float.float16ToFloat */
float orc_f16_to_f32_daz(uint16_t h);             /* FP16FloatTensor.java:76-98 bit trick */
uint16_t orc_f32_to_f16(float f);                 /* round-to-nearest-even */
void orc_dequant_q8_0(const void *blocks, size_t n, float *out);   /* Q8_0FloatTensor.getFloat */
float orc_dot_q8_0(const void *w, size_t elem_offset, const float *x, int size);
float orc_dot_f16(const void *w, size_t elem_offset, const float *x, int size, int exact);
float orc_dot_scalar(const float *a, const float *b, int size);     /* FloatTensor.scalarDot */
void orc_matmul(const void *w, int ggml_type, const float *x, float *out, int rows, int cols, int f16_exact);
void orc_rmsnorm(float *out, const float *x, const float *w, int offset, int size, float eps);
void orc_rope_tables(int ctx, int head_size, double theta, float *cr, float *ci);
void orc_softmax(float *x, int size);
int orc_argmax(const float *x, int size);
/* Sampler.selectSampler + CategoricalSampler / ToppSampler on one logits vector
 * (inference/sampler/Sampler.java:74-122, CategoricalSampler.java:31-42,
 * ToppSampler.java:61-156): returns the token the reference samples for the
 * draw `coin` (rng.nextFloat(1f)).  probs and idx are n-element scratch.
 * info (nullable) also gets the decision in exact arithmetic (the
 * exponentials divided by the float nearest their exact sum, cumulative sums
 * in double, candidates in descending order with ties by index), its distance
 * from the nearest decision boundary, the nucleus size, whether the
 * reference's heap extracted the nucleus out of descending order, and how far
 * the reference's float sums at its decision are from the exact ones. */
typedef struct {
  int token_exact;
  double margin_exact;
  int quirk;
  int nucleus;
  double ref_shift;
} orc_sample_info;
int orc_sample(const float *logits, int n, float temperature, float topp, float coin, float *probs, int *idx,
               orc_sample_info *info);

/* attention for one head: q[hs], cache rows at k/v + t*kv_stride, t in [0,pos] */
void orc_attention_head(const float *q, const float *kcache, const float *vcache, int kv_stride,
                        int head_size, int pos, float *att_scratch, float *out);

#ifdef __cplusplus
}
#endif
#endif
