/*
 * gl3.h — C ABI of libgpullama3_hip.so, the MI355X (gfx950) replacement for the
 * TornadoVM execution plan behind GPULlama3.java's per-token decode forward pass.
 *
 * Reference paths are relative to src/main/java/org/beehive/gpullama3/ in the
 * GPULlama3.java repository.
 *
 * Conventions
 *  - Every function returns a gl3_status (0 = success) except gl3_destroy and
 *    gl3_last_error.  No C++ exception crosses the ABI.  On failure a message is
 *    left in a thread-local buffer read by gl3_last_error().
 *  - Host pointers are borrowed for the duration of the call only.
 *  - A gl3_plan is not thread-safe: one generation thread drives it, as one
 *    thread drives a TornadoVMMasterPlan.  Independent plans may run
 *    concurrently; each owns one HIP stream.
 *  - Status -> Java exception mapping used by the FFM binding:
 *      GL3_ERR_INVALID_ARGUMENT -> IllegalArgumentException
 *      GL3_ERR_UNSUPPORTED      -> UnsupportedOperationException
 *      GL3_ERR_OUT_OF_MEMORY    -> OutOfMemoryError (TornadoOutOfMemoryException's role)
 *      GL3_ERR_DEVICE, GL3_ERR_STATE -> IllegalStateException
 */
#ifndef GL3_H
#define GL3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GL3_ABI_VERSION 1

typedef enum gl3_status {
  GL3_OK = 0,
  GL3_ERR_INVALID_ARGUMENT = 1,
  GL3_ERR_UNSUPPORTED = 2,
  GL3_ERR_OUT_OF_MEMORY = 3,
  GL3_ERR_DEVICE = 4,
  GL3_ERR_STATE = 5
} gl3_status;

/* Model families, in the order of the reference's ModelType (model/ModelType.java:24-80).
 * LLAMA_3 and MISTRAL share the Llama graph; QWEN_3 adds per-head Q/K RMSNorm and
 * NeoX RoPE; PHI_3 has fused QKV and gate-up projections and NeoX RoPE.
 * QWEN_2 / DEEPSEEK_R1_DISTILL_QWEN (QKV bias) are rejected with GL3_ERR_UNSUPPORTED. */
typedef enum gl3_model_type {
  GL3_MODEL_LLAMA_3 = 0,
  GL3_MODEL_MISTRAL = 1,
  GL3_MODEL_QWEN_3 = 2,
  GL3_MODEL_PHI_3 = 3,
  GL3_MODEL_QWEN_2 = 4,
  GL3_MODEL_DEEPSEEK_R1_DISTILL_QWEN = 5
} gl3_model_type;

/* GGML type ids (tensor/GGMLType.java ordinal).  Linear weights may be F16 or
 * Q8_0 (34-byte blocks {fp16 scale, int8 q[32]}); norms are F32. */
typedef enum gl3_ggml_type { GL3_TYPE_F32 = 0, GL3_TYPE_F16 = 1, GL3_TYPE_Q8_0 = 8 } gl3_ggml_type;

/* Tensor kinds, named after the GGUF tensors the reference loaders read
 * (model/loader/LlamaModelLoader.java:77-98, Qwen3ModelLoader.java:95-123,
 * Phi3ModelLoader.java:102-122).  For PHI_3, GL3_FFN_UP is the fused
 * [2*hidden][dim] gate-up matrix (gate rows first) and GL3_ATTN_QKV is the fused
 * [dim + 2*kvDim][dim] projection. */
typedef enum gl3_tensor_kind {
  GL3_TOKEN_EMBD = 0,
  GL3_OUTPUT_NORM = 1,
  GL3_OUTPUT = 2,
  GL3_ATTN_NORM = 3,
  GL3_ATTN_Q = 4,
  GL3_ATTN_K = 5,
  GL3_ATTN_V = 6,
  GL3_ATTN_QKV = 7,
  GL3_ATTN_OUTPUT = 8,
  GL3_ATTN_Q_NORM = 9,
  GL3_ATTN_K_NORM = 10,
  GL3_FFN_NORM = 11,
  GL3_FFN_GATE = 12,
  GL3_FFN_UP = 13,
  GL3_FFN_DOWN = 14
} gl3_tensor_kind;

/* Plan flags */
#define GL3_FLAG_PHASE_KERNELS 1u  /* run one kernel per phase (captured in a hipGraph) instead of
                                      the persistent decode kernel */
#define GL3_FLAG_TIMING 2u         /* record HIP events around every launch (gl3_get_timing) */
#define GL3_FLAG_PHASE_TRACE 4u    /* every workgroup of the persistent kernel stamps every phase boundary */
#define GL3_FLAG_STEPWISE_PROMPT 8u  /* generate calls forward the prompt one decode step per token (as the
                                        reference does) instead of the batched prefill */

/* Shape of the model.  Filled by the Java host from the reference's
 * Configuration (model/Configuration.java) — head_dim is
 * numberOfHeadsKey() for Qwen3 and dim/numberOfHeads otherwise. */
typedef struct gl3_config {
  int32_t abi_version;     /* GL3_ABI_VERSION */
  int32_t model_type;      /* gl3_model_type */
  int32_t weight_type;     /* GGML type of output.weight: the planner key (QuantizationPlannerFactory.java:41-49) */
  int32_t dim;
  int32_t hidden_dim;
  int32_t n_layers;
  int32_t n_heads;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t vocab_size;
  int32_t context_length;
  float rms_norm_eps;
  float rope_theta;
  uint32_t flags;
} gl3_config;

typedef struct gl3_plan gl3_plan;

/* Replaces TornadoVMMasterPlan.initializeTornadoVMPlan (tornadovm/TornadoVMMasterPlan.java:37-79)
 * and the routing of QuantizationPlannerFactory.create (layerplanner/base/QuantizationPlannerFactory.java:41-73):
 * validates the (weight type, model type) pair, allocates device weights, the fp16
 * KV cache and activations on the current HIP device. */
int gl3_create(const gl3_config *cfg, gl3_plan **out);

/* Copies one tensor to the device (the FIRST_EXECUTION weight transfers of the
 * layer graphs, e.g. layers/type/q8_0/LlamaQ8_0FFNLayers.java:62-67, and the
 * Q8_0 AoS->SoA repack of tensor/tornado/Q8_0TornadoTensor.java:74-117).
 * host points at the tensor in its GGUF encoding; bytes must equal its exact size.
 * layer is ignored for TOKEN_EMBD, OUTPUT_NORM and OUTPUT. */
int gl3_upload(gl3_plan *p, int kind, int layer, const void *host, size_t bytes, int ggml_type);

/* Optional: use the host's RoPE.precomputeFreqsCis tables (inference/operation/RoPE.java:6-37),
 * [ctx][half] floats each.  Without this call the plan computes the same tables itself. */
int gl3_set_rope_tables(gl3_plan *p, const float *cos_table, const float *sin_table, int ctx, int half);

/* Replaces forceCopyInReadOnlyDataLayered (TornadoVMMasterPlan.java:180-195): checks
 * that every tensor was uploaded and builds the per-token schedule.  Called
 * implicitly by the first forward. */
int gl3_prepare(gl3_plan *p);

/* One decode step.  Replaces InferenceCore.forwardTornadoVM (inference/InferenceCore.java:582-589)
 * + tornadoVMForwardExecuteLayered (TornadoVMMasterPlan.java:127-153): embedding gather
 * on device, all layers, final norm, classifier.  Writes vocab_size fp32 logits to
 * logits_out (nullable) and the greedy token (first maximum, Sampler.TENSOR_ARGMAX)
 * to argmax_out (nullable).  Requires 0 <= token < vocab_size and
 * 0 <= position < context_length.  Returns after the outputs are host-visible. */
int gl3_forward(gl3_plan *p, int32_t token, int32_t position, float *logits_out, int32_t *argmax_out);

/* Greedy decode of n_steps tokens entirely on the device: step i forwards the
 * previous step's argmax at position + i (step 0 forwards token).  tokens_out
 * receives the n_steps argmax tokens.  No reference counterpart: it is the
 * generation loop of InferenceEngine.generateTokensGPULlama (inference/InferenceEngine.java:309-355)
 * with the sampler fixed to TENSOR_ARGMAX, so the logits never leave the GPU. */
int gl3_generate_greedy(gl3_plan *p, int32_t token, int32_t position, int32_t n_steps, int32_t *tokens_out);

/* The prompt phase of the reference's generation loop (InferenceEngine.java:88-131,
 * :162-187: one forward per prompt token, logits unused), batched: the n tokens
 * go through every layer in blocks of up to 512 rows (matrix products on the
 * matrix cores, causal attention over the cache), leaving their K and V at
 * positions position .. position + n - 1 and no logits.  A gl3_forward of the
 * next token then continues as after n single forwards.  Requires head_dim 64,
 * 96 or 128, every token in [0, vocab_size) and position + n <= context_length.
 * Returns after the cache is written. */
int gl3_prefill(gl3_plan *p, const int32_t *tokens, int32_t n, int32_t position);

/* The reference's generation loop with the TENSOR_ARGMAX sampler, entirely on the
 * device (InferenceEngine.generateTokensGPULlama, inference/InferenceEngine.java:309-355):
 * forwards the n_prompt prompt tokens at positions position.. (their logits are
 * not used, as in the reference's prompt phase), then greedy steps; tokens_out
 * receives the n_gen generated tokens (the argmax after the last prompt token,
 * then after each generated one).  All prompt tokens but the last go through the
 * batched prefill of gl3_prefill (one decode step each with
 * GL3_FLAG_STEPWISE_PROMPT, or when the shape has no prefill); the last prompt
 * token and the generated ones are decode steps in persistent launches, no host
 * round trip between them.  Requires every prompt token in [0, vocab_size) and
 * position + n_prompt + n_gen - 1 <= context_length. */
int gl3_generate_from_prompt(gl3_plan *p, const int32_t *prompt, int32_t n_prompt, int32_t position, int32_t n_gen,
                             int32_t *tokens_out);

/* The reference's generation loop with a sampling Sampler, entirely on the
 * device (InferenceEngine.generateTokensGPULlama, inference/InferenceEngine.java:309-355,
 * with Sampler.selectSampler, inference/sampler/Sampler.java:74-122): the
 * n_prompt prompt tokens are forwarded from `position` (logits unused; the
 * prompt as in gl3_generate_from_prompt), then
 * each of the n_gen tokens is sampled on the device from the last step's
 * logits and forwarded: temperature 0 takes the first maximum (TENSOR_ARGMAX);
 * otherwise the logits are divided by the temperature and turned into
 * probabilities, then sampled by CategoricalSampler (CategoricalSampler.java:31-42)
 * when topp <= 0 or topp >= 1, else by ToppSampler (ToppSampler.java:61-156).
 * coins[k] in [0, 1) is the draw for generated token k (the reference's
 * rng.nextFloat(1f)).  Cumulative sums are exact (fixed point) and the nucleus
 * is visited in descending probability, ties by index.  tokens_out receives
 * the n_gen tokens.  Requires position + n_prompt + n_gen - 1 <= context_length. */
int gl3_generate_sampled(gl3_plan *p, const int32_t *prompt, int32_t n_prompt, int32_t position, int32_t n_gen,
                         float temperature, float topp, const float *coins, int32_t *tokens_out);

/* Zero the KV cache (a fresh State: inference/state/LlamaState.java:61-64). */
int gl3_reset(gl3_plan *p);

/* KV-cache access, fp16 [npos][n_kv_heads*head_dim] (the reference's [pos][kvDim] row
 * order) for positions pos0..pos0+npos-1 of one layer.  Used to pre-fill long
 * contexts and to check cache contents. */
int gl3_write_kv(gl3_plan *p, int layer, int pos0, int npos, const uint16_t *k, const uint16_t *v);
int gl3_read_kv(gl3_plan *p, int layer, int pos0, int npos, uint16_t *k, uint16_t *v);
/* Fill positions [0, npos) of every layer with fp16(N(0,1)) values from a counter-based
 * generator keyed by seed (long-context benchmarks). */
int gl3_fill_kv_normal(gl3_plan *p, uint64_t seed, int npos);

/* Timing of the launches of the last gl3_forward/gl3_generate_greedy call (needs
 * GL3_FLAG_TIMING): total elapsed ms on the plan's stream, summed kernel ms, and
 * the number of kernel launches. */
int gl3_get_timing(gl3_plan *p, double *elapsed_ms, double *kernel_ms, int32_t *launches);

/* Phase trace of the last token of the persistent decode kernel (needs
 * GL3_FLAG_PHASE_TRACE): durations in microseconds, as seen by workgroup 0, of
 * embedding, 0, then per layer {QKV, attention up to q/k/v read, attention
 * tiles, attention split merge, Wo (with the request of its weights), request
 * of the gate/up weights, gate/up, request of the down weights, down (fused
 * FFN: down partials), request of the next phase's weights (fused FFN: and
 * the reduce of the down partials)}, then the classifier (each phase includes
 * its wait for its input; a workgroup without an attention item stamps the
 * first two attention boundaries on its way through).  *n_out gets the number
 * of entries written.
 * No reference counterpart (the reference's TornadoVM profiler times whole task
 * graphs: llama-tornado:131-134). */
int gl3_get_phase_trace(gl3_plan *p, double *us_out, int32_t max_entries, int32_t *n_out);

/* Raw phase-boundary stamps of the last persistent-kernel token for every
 * workgroup: out[i * n_workgroups + w] = s_memrealtime (100 MHz) of workgroup
 * w at boundary i (same boundaries as gl3_get_phase_trace, with the step's
 * start at i = 0).  Needs GL3_FLAG_PHASE_TRACE.  No reference counterpart. */
int gl3_get_phase_stamps(gl3_plan *p, uint64_t *out, int64_t max_entries, int32_t *n_stamps, int32_t *n_workgroups);

/* Measurement aid: runs the per-phase schedule's flash-decode attention kernel
 * for `layer` at `position` n_reps times over the plan's KV cache, each launch
 * bracketed by HIP events on the plan's stream, and returns the average launch
 * duration in ms.  Each launch appends the plan's plain q/k/v vector as the
 * cache row at `position` (the cache row is overwritten).  No reference
 * counterpart (the reference times whole task graphs: llama-tornado:131-134). */
int gl3_time_attention(gl3_plan *p, int layer, int32_t position, int32_t n_reps, double *avg_ms);

/* The configuration of a GGUF model file, as the reference derives it: header
 * and metadata as GGUF.loadGGUFMetadata reads them (tensor/GGUF.java:43-92,
 * versions 2 and 3), the family from general.name as
 * ModelLoader.detectModelType (model/loader/ModelLoader.java:45-67), the shape
 * from the <arch>.* keys as the loaders' createConfiguration
 * (LlamaModelLoader.java:47-62, MistralModelLoader.java:44-66,
 * Qwen3ModelLoader.java:48-73, Phi3ModelLoader.java:45-60), and the planner
 * key from the type of output.weight (token_embd.weight when tied,
 * AbstractModelLoader.java:146-150).  context_length is the reference's
 * -n/--max-tokens: < 0 keeps the model's own for Llama, Mistral and Qwen3
 * (Mistral and Qwen3 take the smaller of the two); Phi-3 needs it > 0, as its
 * loader uses the requested value as is.  Reads the file only: no GPU call. */
int gl3_gguf_config(const char *path, int32_t context_length, uint32_t flags, gl3_config *cfg_out);

/* gl3_gguf_config, gl3_create, one gl3_upload per tensor straight from a
 * read-only mapping of the file (no host copy; rope_freqs.weight and tensors
 * this path does not read are skipped, GGUF.java:120-123), then gl3_prepare:
 * the reference's ModelLoader.loadModel (ModelLoader.java:81-92) followed by
 * the weight copy-in of initializeTornadoVMPlan (TornadoVMMasterPlan.java:37-79),
 * for callers that hand the library a path. */
int gl3_create_from_gguf(const char *path, int32_t context_length, uint32_t flags, gl3_plan **out);

/* Replaces freeTornadoExecutionPlan (TornadoVMMasterPlan.java:200-202). */
void gl3_destroy(gl3_plan *p);

/* Thread-local message of the last failure on this thread ("" if none). */
const char *gl3_last_error(void);

/* Name of the device and arch of the current HIP device, e.g. "AMD Instinct MI355X gfx950". */
int gl3_device_name(char *buf, size_t len);

/* ---- Op-level entry points: each runs one device kernel of the decode path on
 *      host buffers (copied in and out).  For parity tests and diagnostics. ---- */

/* Q8_0 dequantisation, n elements from GGUF blocks (Q8_0FloatTensor.getFloat,
 * tensor/standard/Q8_0FloatTensor.java:55-63); out is exact q*f16(scale). */
int gl3_op_dequant_q8_0(const void *blocks, size_t n, float *out);
/* binary16 -> binary32 on the device, subnormals preserved (Float.float16ToFloat). */
int gl3_op_f16_to_f32(const uint16_t *in, size_t n, float *out);

/* GEMV modes */
#define GL3_GEMV_STORE 0     /* y = W x                         (matrixVectorGeneric) */
#define GL3_GEMV_RESIDUAL 1  /* y += W x                        (matrixVectorGenericWithResidual) */
#define GL3_GEMV_SWIGLU 2    /* y[r] = silu(W[r] x) * W[rows/2 + r] x, rows/2 outputs
                                (fusedFeedForwardWithSiLUAndGLUActivation) */
/* y = W · n(x) where n(x) = rmsnorm(x, norm_w, eps) if norm_w != NULL else x.
 * W is [rows][cols] in GGUF encoding (F16 or Q8_0).  Mirrors
 * kernels/TransformerComputeKernelsLayered.java:650-1057. */
int gl3_op_gemv(int ggml_type, const void *w, int rows, int cols, const float *x, const float *norm_w,
                float eps, int mode, float *y);

/* The device sampler of gl3_generate_sampled on host logits [n] (n >= 2), once
 * per draw: tokens_out[k] is the token sampled with coins[k]
 * (Sampler.selectSampler, inference/sampler/Sampler.java:74-122). */
int gl3_op_sample(const float *logits, int32_t n, float temperature, float topp, const float *coins, int32_t n_draws,
                  int32_t *tokens_out);

/* Decode attention of all heads at position pos over an fp16 cache [pos+1][n_kv][hd]
 * (rows for t <= pos): out[n_heads*hd].  q is [n_heads*hd] fp32, already rotated.
 * Mirrors processHeadsParallel / processHeadsFlashAttention
 * (kernels/TransformerComputeKernelsLayered.java:278-628). */
int gl3_op_attention(const float *q, const uint16_t *kcache, const uint16_t *vcache, int n_heads,
                     int n_kv_heads, int head_dim, int pos, float *out);

/* ---- Allocation-free entry point ---- */

/* Scratch of gl3_op_attention_noalloc: one static device array of this many
 * bytes per GPU, held until the process ends. */
#define GL3_NOALLOC_SCRATCH_BYTES (1280u << 10)

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The computation of gl3_op_attention on device-resident
 * buffers, in the plan's cache layout, appending the new row first:
 *   qkv    device fp32 [n_heads*head_dim + 2*n_kv_heads*head_dim]: q (already
 *          rotated), then the new k and v, which are written to the cache at pos;
 *   kcache device fp16 K [n_kv_heads][ctxp][head_dim], rows < pos valid;
 *   vcache device fp16 V in 16-position blocks [n_kv_heads][ctxp/16][head_dim][16];
 *   out    device fp32 [n_heads*head_dim].
 * ctxp is a multiple of 16 above pos.  The split partials, merge counters and
 * control block live in the GPU's GL3_NOALLOC_SCRATCH_BYTES array (counters
 * cleared by a kernel on every call); n_kv_heads <= 64, and a shape whose
 * partials do not fit is rejected with GL3_ERR_INVALID_ARGUMENT.  Calls no
 * allocating routine.  Enqueues on `stream` (a hipStream_t, NULL = default)
 * and returns without waiting; calls that overlap on one GPU share its array
 * and race. */
int gl3_op_attention_noalloc(const float *qkv, uint16_t *kcache, uint16_t *vcache, int n_heads, int n_kv_heads,
                             int head_dim, int ctxp, int pos, float *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* GL3_H */
