/*
 * CPU oracle: C restatement of GPULlama3.java's CPU decode forward pass.
 *
 * TEST INFRASTRUCTURE ONLY (see gl3_oracle.h).  Built with -ffp-contract=off:
 * Java never contracts a*b+c into an FMA, so every multiply and add below is
 * rounded separately except where the reference calls fma explicitly.
 *
 * Reference paths are relative to src/main/java/org/beehive/gpullama3/.
 */
#include "gl3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define Q8_BLOCK 32
#define Q8_BYTES 34

static int g_use_simd = 1;
void orc_set_simd(int on) { g_use_simd = on; }

/* ------------------------------------------------------------------ fp16 */

/* Float.float16ToFloat: exact IEEE binary16 -> binary32, subnormals kept
 * (tensor/standard/FP16FloatTensor.java:48-51, Q8_0FloatTensor.java:61). */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24, normalise */
      int e = -1;
      do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* The vector path's decode (FP16FloatTensor.java:69-98): sign-extend the
 * short, keep the sign, rebias exponent+mantissa, and zero the result when the
 * exponent field is 0 (denormals-are-zero).  Infinities/NaNs are not handled,
 * exactly as in the reference. */
float orc_f16_to_f32_daz(uint16_t h) {
  int32_t b = (int32_t)(int16_t)h;
  int32_t zero_exp_mask = (-(b & 0x7C00)) >> 31;
  uint32_t bits = ((uint32_t)(b & 0x8000) << 16) | (((uint32_t)((b & 0x7FFF) + 0x1C000) << 13) & (uint32_t)zero_exp_mask);
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* binary32 -> binary16, round to nearest even (used for fixtures and the kv_fp16 test aid). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7FFFFFFFu;
  if (absx >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u : 0u));
  if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* overflow after rounding */
  if (absx < 0x38800000u) { /* result subnormal or zero */
    if (absx < 0x33000000u) return (uint16_t)sign;
    uint32_t e = absx >> 23;
    uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126 - e; /* 14..24 */
    uint32_t r = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = absx - 0x38000000u; /* rebias exponent by -112 */
  uint32_t lsb = (r >> 13) & 1u;
  r += 0xFFFu + lsb;
  return (uint16_t)(sign | (r >> 13));
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Q8_0FloatTensor.getFloat (Q8_0FloatTensor.java:55-63): quant * f16(scale). */
static inline float q8_get(const uint8_t *blocks, size_t index) {
  size_t bi = index / Q8_BLOCK, wi = index % Q8_BLOCK;
  const uint8_t *b = blocks + bi * Q8_BYTES;
  return (float)(int8_t)b[2 + wi] * orc_f16_to_f32(rd16(b));
}

void orc_dequant_q8_0(const void *blocks, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) out[i] = q8_get((const uint8_t *)blocks, i);
}

static inline float tensor_get(const void *t, int type, size_t index) {
  switch (type) {
    case ORC_F32: return ((const float *)t)[index];
    case ORC_F16: return orc_f16_to_f32(((const uint16_t *)t)[index]);
    default: return q8_get((const uint8_t *)t, index);
  }
}

/* FloatTensor.scalarDot (FloatTensor.java:86-92): sequential, no FMA. */
float orc_dot_scalar(const float *a, const float *b, int size) {
  float r = 0.0f;
  for (int j = 0; j < size; ++j) r += a[j] * b[j];
  return r;
}

static float scalar_dot_typed(const void *w, int type, size_t off, const float *x, int size) {
  float r = 0.0f;
  for (int j = 0; j < size; ++j) r += tensor_get(w, type, off + j) * x[j];
  return r;
}

/* Vector API reduceLanes(ADD) has no specified order; the lanes are added in
 * index order (the strict order the JDK 21 C2 compiler uses for this node). */
static inline float reduce8(const float v[8]) {
  float r = v[0];
  for (int k = 1; k < 8; ++k) r += v[k];
  return r;
}

/* ---------------------------------------------------------- Q8_0 dot */

/* Q8_0FloatTensor.vectorDot, 256-bit species (Q8_0FloatTensor.java:77-127):
 * per block, lane k: ((x[k]q[k] + x[8+k]q[8+k]) + x[16+k]q[16+k]) + x[24+k]q[24+k],
 * fused-multiply-added with the block scale into the lane accumulator. */
static float dot_q8_lanes_scalar(const uint8_t *blk, const float *x, int nblocks, float acc[8]) {
  for (int b = 0; b < nblocks; ++b, blk += Q8_BYTES, x += Q8_BLOCK) {
    float scale = orc_f16_to_f32(rd16(blk));
    const int8_t *q = (const int8_t *)(blk + 2);
    for (int k = 0; k < 8; ++k) {
      float s0 = x[k] * (float)q[k];
      float s1 = x[8 + k] * (float)q[8 + k];
      float s2 = x[16 + k] * (float)q[16 + k];
      float s3 = x[24 + k] * (float)q[24 + k];
      acc[k] = fmaf(((s0 + s1) + s2) + s3, scale, acc[k]);
    }
  }
  return 0.0f;
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma,f16c")))
static void dot_q8_lanes_avx2(const uint8_t *blk, const float *x, int nblocks, float acc[8]) {
  __m256 val = _mm256_loadu_ps(acc);
  for (int b = 0; b < nblocks; ++b, blk += Q8_BYTES, x += Q8_BLOCK) {
    __m256 scale = _mm256_set1_ps(orc_f16_to_f32(rd16(blk)));
    __m128i lo = _mm_loadu_si128((const __m128i *)(blk + 2));
    __m128i hi = _mm_loadu_si128((const __m128i *)(blk + 18));
    __m256 q0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(lo));
    __m256 q1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(lo, 8)));
    __m256 q2 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(hi));
    __m256 q3 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(hi, 8)));
    __m256 s0 = _mm256_mul_ps(_mm256_loadu_ps(x), q0);
    __m256 s1 = _mm256_mul_ps(_mm256_loadu_ps(x + 8), q1);
    __m256 s2 = _mm256_mul_ps(_mm256_loadu_ps(x + 16), q2);
    __m256 s3 = _mm256_mul_ps(_mm256_loadu_ps(x + 24), q3);
    __m256 sum = _mm256_add_ps(_mm256_add_ps(_mm256_add_ps(s0, s1), s2), s3);
    val = _mm256_fmadd_ps(sum, scale, val);
  }
  _mm256_storeu_ps(acc, val);
}
static int have_avx2(void) {
  static int cached = -1;
  if (cached < 0) cached = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
  return cached;
}
#endif

float orc_dot_q8_0(const void *w, size_t this_offset, const float *x, int size) {
  const uint8_t *blocks = (const uint8_t *)w;
  float result = 0.0f;
  int j = 0;
  int align = (int)((-(long long)this_offset) & (Q8_BLOCK - 1));
  int alignment_bound = size < align ? size : align;
  if (alignment_bound > 0) {
    result += scalar_dot_typed(w, ORC_Q8_0, this_offset, x, alignment_bound);
    j += alignment_bound;
  }
  int upper = size / Q8_BLOCK * Q8_BLOCK; /* as in the reference: not adjusted for j */
  int nblocks = upper > j ? (upper - j) / Q8_BLOCK : 0;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const uint8_t *blk = blocks + (this_offset + j) / Q8_BLOCK * Q8_BYTES;
#if defined(__x86_64__)
  if (g_use_simd && have_avx2()) dot_q8_lanes_avx2(blk, x + j, nblocks, acc);
  else
#endif
    dot_q8_lanes_scalar(blk, x + j, nblocks, acc);
  j += nblocks * Q8_BLOCK;
  result += reduce8(acc);
  if (j < size) result += scalar_dot_typed(w, ORC_Q8_0, this_offset + j, x + j, size - j);
  return result;
}

/* ----------------------------------------------------------- F16 dot */

/* FP16FloatTensor.vectorDot (FP16FloatTensor.java:62-110): lane k accumulates
 * fma(w[k], x[k], acc[k]) over 8-wide steps with the DAZ decode; the tail uses
 * the scalar dot with the exact decode.  exact=1 swaps in the exact decode. */
static void dot_f16_lanes_scalar(const uint16_t *w, const float *x, int n8, int exact, float acc[8]) {
  for (int i = 0; i < n8; ++i, w += 8, x += 8)
    for (int k = 0; k < 8; ++k) {
      float wf = exact ? orc_f16_to_f32(w[k]) : orc_f16_to_f32_daz(w[k]);
      acc[k] = fmaf(wf, x[k], acc[k]);
    }
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma,f16c")))
static void dot_f16_lanes_avx2(const uint16_t *w, const float *x, int n8, int exact, float acc[8]) {
  __m256 val = _mm256_loadu_ps(acc);
  const __m128i expmask = _mm_set1_epi16(0x7C00);
  const __m256 signmask = _mm256_castsi256_ps(_mm256_set1_epi32((int)0x80000000u));
  for (int i = 0; i < n8; ++i, w += 8, x += 8) {
    __m128i h = _mm_loadu_si128((const __m128i *)w);
    __m256 wf = _mm256_cvtph_ps(h); /* exact, keeps subnormals */
    if (!exact) {
      __m128i zero_exp = _mm_cmpeq_epi16(_mm_and_si128(h, expmask), _mm_setzero_si128());
      __m256 zmask = _mm256_castsi256_ps(_mm256_cvtepi16_epi32(zero_exp));
      wf = _mm256_blendv_ps(wf, _mm256_and_ps(wf, signmask), zmask);
    }
    val = _mm256_fmadd_ps(wf, _mm256_loadu_ps(x), val);
  }
  _mm256_storeu_ps(acc, val);
}
#endif

float orc_dot_f16(const void *w, size_t off, const float *x, int size, int exact) {
  const uint16_t *h = (const uint16_t *)w + off;
  int upper = size - size % 8;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#if defined(__x86_64__)
  if (g_use_simd && have_avx2()) dot_f16_lanes_avx2(h, x, upper / 8, exact, acc);
  else
#endif
    dot_f16_lanes_scalar(h, x, upper / 8, exact, acc);
  float result = reduce8(acc);
  if (upper < size) result += scalar_dot_typed(w, ORC_F16, off + upper, x + upper, size - upper);
  return result;
}

/* FloatTensor.matmul (FloatTensor.java:98-100): out[i] = dot(i*dim1, x, 0, dim1),
 * rows in parallel (Parallel.parallelFor); each row's value does not depend on
 * the thread that computes it. */
void orc_matmul(const void *w, int type, const float *x, float *out, int rows, int cols, int f16_exact) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < rows; ++i) {
    size_t off = (size_t)i * cols;
    float r;
    if (type == ORC_Q8_0) r = orc_dot_q8_0(w, off, x, cols);
    else if (type == ORC_F16) r = orc_dot_f16(w, off, x, cols, f16_exact);
    else r = orc_dot_scalar((const float *)w + off, x, cols);
    out[i] = r;
  }
}

/* InferenceCore.rmsnorm (inference/InferenceCore.java:46-55). */
void orc_rmsnorm(float *out, const float *x, const float *w, int offset, int size, float eps) {
  float ss = 0.0f;
  for (int i = 0; i < size; ++i) ss = ss + x[offset + i] * x[offset + i];
  ss /= (float)size;
  ss += eps;
  ss = (float)(1.0 / sqrt((double)ss));
  for (int i = offset; i < offset + size; ++i) out[i] = w[i % size] * (ss * x[i]);
}

/* RoPE.precomputeFreqsCis without scaling (inference/operation/RoPE.java:6-37). */
void orc_rope_tables(int ctx, int hs, double theta, float *cr, float *ci) {
  size_t n = 0;
  for (int pos = 0; pos < ctx; ++pos)
    for (int i = 0; i < hs; i += 2) {
      float freq = (float)(1.0 / pow(theta, i / (double)hs));
      float val = (float)pos * freq;
      cr[n] = (float)cos((double)val);
      ci[n] = (float)sin((double)val);
      ++n;
    }
}

/* FloatTensor.softmaxInPlace (FloatTensor.java:211-219). */
void orc_softmax(float *x, int size) {
  float maxv = -INFINITY;
  for (int i = 0; i < size; ++i) maxv = x[i] > maxv ? x[i] : maxv;
  for (int i = 0; i < size; ++i) x[i] = (float)exp((double)(x[i] - maxv));
  float sum = 0.0f;
  for (int i = 0; i < size; ++i) sum += x[i];
  for (int i = 0; i < size; ++i) x[i] = x[i] / sum;
}

/* ------------------------------------------------------------- sampling
 * Sampler.selectSampler (inference/sampler/Sampler.java:74-122) applied to one
 * logits vector: temperature 0 -> TENSOR_ARGMAX; otherwise the logits are
 * divided by the temperature (FloatTensor.divideInPlace, FloatTensor.java:203-205),
 * turned into probabilities (softmaxInPlace, :211-219) and handed to
 * CategoricalSampler (CategoricalSampler.java:31-42) when topp <= 0 or topp >= 1,
 * else to ToppSampler (ToppSampler.java:61-156).  `coin` is the value the
 * reference draws with rng.nextFloat(1f). */

/* ToppSampler.siftDown (ToppSampler.java:30-44) with the comparator of
 * sampleFromFloatTensor (:60: comparingDouble(getFloat).reversed()): a node
 * goes below a child with a strictly larger probability. */
static void topp_sift_down(int *a, int from, int n, const float *p) {
  int prev = from, next;
  while ((next = 2 * prev + 1) < n) {
    int r = 2 * prev + 2;
    if (r < n && (double)p[a[r]] > (double)p[a[next]]) next = r;
    if ((double)p[a[next]] > (double)p[a[prev]]) {
      int t = a[prev];
      a[prev] = a[next];
      a[next] = t;
      prev = next;
    } else {
      break;
    }
  }
}

/* probabilities descending, then index ascending */
static const float *g_sort_p;
static int cmp_desc(const void *x, const void *y) {
  int a = *(const int *)x, b = *(const int *)y;
  if (g_sort_p[a] > g_sort_p[b]) return -1;
  if (g_sort_p[a] < g_sort_p[b]) return 1;
  return a < b ? -1 : (a > b);
}

int orc_sample(const float *logits, int n, float temperature, float topp, float coin, float *probs, int *idx,
               orc_sample_info *info) {
  orc_sample_info dummy;
  if (!info) info = &dummy;
  info->token_exact = -1;
  info->margin_exact = 0.0;
  info->quirk = 0;
  info->nucleus = 0;
  info->ref_shift = 0.0;
  if (temperature == 0.0f) {  /* Sampler.java:76-78 */
    int t = orc_argmax(logits, n);
    info->token_exact = t;
    info->margin_exact = 1.0;
    return t;
  }
  for (int i = 0; i < n; ++i) probs[i] = logits[i] / temperature;  /* FloatTensor.java:203-205 */
  /* softmaxInPlace (FloatTensor.java:211-219), keeping the exponentials for the exact path */
  float maxv = -INFINITY;
  for (int i = 0; i < n; ++i) maxv = probs[i] > maxv ? probs[i] : maxv;
  float *pe = (float *)malloc(sizeof(float) * (size_t)n);
  float sum = 0.0f;
  double sum_d = 0.0;
  for (int i = 0; i < n; ++i) {
    probs[i] = (float)exp((double)(probs[i] - maxv));
    pe[i] = probs[i];
    sum += probs[i];
    sum_d += (double)probs[i];
  }
  for (int i = 0; i < n; ++i) probs[i] = probs[i] / sum;
  /* exact normalisation: the exponentials over the float nearest their exact sum */
  const float sum_f = (float)sum_d;
  for (int i = 0; i < n; ++i) pe[i] = pe[i] / sum_f;
  int token;
  if (topp <= 0 || topp >= 1) {
    /* CategoricalSampler.sampleFromFloatTensor (CategoricalSampler.java:31-42) */
    float cdf = 0.0f;
    token = n - 1;
    for (int i = 0; i < n; ++i) {
      cdf += probs[i];
      if (coin < cdf) {
        token = i;
        break;
      }
    }
    /* the walk over the exact probabilities in double: decision and distance from its boundaries */
    double c = 0.0, prev = 0.0;
    int te = n - 1, hit = 0;
    for (int i = 0; i < n; ++i) {
      prev = c;
      c += (double)pe[i];
      if ((double)coin < c) {
        te = i;
        hit = 1;
        break;
      }
    }
    info->token_exact = te;
    if (hit) {
      const double m1 = c - (double)coin, m2 = (double)coin - prev;
      info->margin_exact = m1 < m2 ? m1 : m2;
    }
    double at_ref = 0.0;
    for (int i = 0; i <= token; ++i) at_ref += (double)pe[i];
    info->ref_shift = fabs((double)cdf - at_ref);
    info->nucleus = n;
    free(pe);
    return token;
  }
  /* ToppSampler.sampleFromFloatTensor (ToppSampler.java:58-78): crop candidates below the cutoff */
  int head = 0, tail = n - 1;
  const float cutoff = (1.0f - topp) / (float)(n - 1);
  for (int i = 0; i < n; ++i) {
    if (probs[i] >= cutoff)
      idx[head++] = i;
    else
      idx[tail--] = i;
  }
  const int n0 = head;
  /* processTopP (ToppSampler.java:103-156): heap, extraction until the cumulative mass exceeds topp */
  for (int i = n0 / 2 - 1; i >= 0; --i) topp_sift_down(idx, i, n0, probs);
  float cum = 0.0f;
  double cum_pe = 0.0;
  int last = 0;
  float prev_val = INFINITY;
  for (int i = n0 - 1; i >= 0; i--) {
    int t = idx[0];
    idx[0] = idx[i];
    idx[i] = t;
    const float v = probs[idx[i]];
    if (v > prev_val) info->quirk = 1;  /* extraction not in descending order (the siftDown bound below) */
    prev_val = v;
    cum += v;
    cum_pe += (double)pe[idx[i]];
    if (cum > topp) {
      last = i;
      break;
    }
    topp_sift_down(idx, 0, i - 1, probs);  /* ToppSampler.java:128: the bound is i - 1 */
  }
  const float r = coin * cum;
  float cdf = 0.0f;
  double cdf_pe = 0.0;
  token = idx[last];
  for (int i = n0 - 1; i >= last; i--) {
    cdf += probs[idx[i]];
    cdf_pe += (double)pe[idx[i]];
    if (r < cdf) {
      token = idx[i];
      break;
    }
  }
  {
    const double s1 = fabs((double)cum - cum_pe), s2 = fabs((double)cdf - cdf_pe);
    info->ref_shift = s1 > s2 ? s1 : s2;
  }
  /* exact semantics: the exact probabilities' candidates sorted (descending, ties by index),
   * cumulative mass in double until it exceeds topp, r = coin * mass, walk */
  int *ord = (int *)malloc(sizeof(int) * (size_t)(n > 0 ? n : 1));
  int m = 0;
  for (int i = 0; i < n; ++i)
    if (pe[i] >= cutoff) ord[m++] = i;
  g_sort_p = pe;
  qsort(ord, (size_t)m, sizeof(int), cmp_desc);
  double c = 0.0, before = 0.0;
  int k = m, crossed = 0;
  for (int i = 0; i < m; ++i) {
    before = c;
    c += (double)pe[ord[i]];
    if (c > (double)topp) {
      k = i + 1;
      crossed = 1;
      break;
    }
  }
  double margin = crossed ? c - (double)topp : (double)topp - c;
  if (crossed && k > 1) {  /* a smaller topp would have stopped one token earlier */
    const double d = (double)topp - before;
    margin = margin < d ? margin : d;
  }
  const double rr = (double)coin * c;
  double w = 0.0, wprev = 0.0;
  info->token_exact = m > 0 ? ord[k - 1] : n - 1;
  int found = 0;
  for (int i = 0; i < k; ++i) {
    wprev = w;
    w += (double)pe[ord[i]];
    if (rr < w) {
      info->token_exact = ord[i];
      double d1 = w - rr, d2 = rr - wprev;
      d1 = d1 < d2 ? d1 : d2;
      margin = margin < d1 ? margin : d1;
      found = 1;
      break;
    }
  }
  if (!found) margin = 0.0;  /* only rounding ends the walk without a pick */
  info->margin_exact = margin;
  info->nucleus = k;
  free(ord);
  free(pe);
  return token;
}

/* FloatTensor.argmax (FloatTensor.java:138-151): first maximum wins. */
int orc_argmax(const float *x, int size) {
  int mi = 0;
  float mv = x[0];
  for (int i = 0; i < size; ++i)
    if (x[i] > mv) { mv = x[i]; mi = i; }
  return mi;
}

/* One head of attention (inference/InferenceCore.java:105-144):
 * score_t = (q . K_t) / sqrt(hs) with the scalar dot, softmax over [0,pos],
 * out = sum_t a_t V_t accumulated as out = a*v + out (saxpyInPlace, FloatTensor.java:221-227). */
void orc_attention_head(const float *q, const float *kc, const float *vc, int kv_stride, int hs, int pos,
                        float *att, float *out) {
  float sqrt_hs = (float)sqrt((double)hs);
  for (int t = 0; t <= pos; ++t) {
    float score = orc_dot_scalar(q, kc + (size_t)t * kv_stride, hs);
    score /= sqrt_hs;
    att[t] = score;
  }
  orc_softmax(att, pos + 1);
  for (int i = 0; i < hs; ++i) out[i] = 0.0f;
  for (int t = 0; t <= pos; ++t) {
    const float *v = vc + (size_t)t * kv_stride;
    float a = att[t];
    for (int i = 0; i < hs; ++i) out[i] = a * v[i] + out[i];
  }
}

/* ------------------------------------------------------------- model */

struct orc_model {
  orc_config c;
  int q_dim, kv_dim, kv_mul;
  const void *t[ORC_KIND_COUNT];      /* global tensors */
  const void **lt[ORC_KIND_COUNT];    /* per-layer tensors */
  int ttype[ORC_KIND_COUNT];
  float *key_cache, *value_cache;     /* [L][ctx][kvDim] */
  float *rope_r, *rope_i;
  float *x, *xb, *xb2, *q, *k, *v, *att, *hb, *hb2, *qkv, *logits;
};

static int is_layer_kind(int kind) { return kind >= ORC_ATTN_NORM; }

orc_model *orc_create(const orc_config *cfg) {
  orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
  if (!m) return NULL;
  m->c = *cfg;
  const orc_config *c = &m->c;
  m->q_dim = c->n_heads * c->head_dim;
  m->kv_dim = c->n_kv_heads * c->head_dim;
  m->kv_mul = c->n_heads / c->n_kv_heads;
  for (int k = 0; k < ORC_KIND_COUNT; ++k)
    if (is_layer_kind(k)) m->lt[k] = (const void **)calloc((size_t)c->n_layers, sizeof(void *));
  size_t kv = (size_t)c->n_layers * c->context_length * m->kv_dim;
  m->key_cache = (float *)calloc(kv, sizeof(float));
  m->value_cache = (float *)calloc(kv, sizeof(float));
  size_t rt = (size_t)c->context_length * (c->head_dim / 2);
  m->rope_r = (float *)malloc(rt * sizeof(float));
  m->rope_i = (float *)malloc(rt * sizeof(float));
  orc_rope_tables(c->context_length, c->head_dim, c->rope_theta, m->rope_r, m->rope_i);
  int wide = m->q_dim > c->dim ? m->q_dim : c->dim;
  m->x = (float *)calloc((size_t)c->dim, sizeof(float));
  m->xb = (float *)calloc((size_t)wide, sizeof(float));
  m->xb2 = (float *)calloc((size_t)c->dim, sizeof(float));
  m->q = (float *)calloc((size_t)m->q_dim, sizeof(float));
  m->k = (float *)calloc((size_t)m->kv_dim, sizeof(float));
  m->v = (float *)calloc((size_t)m->kv_dim, sizeof(float));
  m->att = (float *)calloc((size_t)c->n_heads * c->context_length, sizeof(float));
  m->hb = (float *)calloc((size_t)2 * c->hidden_dim, sizeof(float));
  m->hb2 = (float *)calloc((size_t)c->hidden_dim, sizeof(float));
  m->qkv = (float *)calloc((size_t)m->q_dim + 2 * m->kv_dim, sizeof(float));
  m->logits = (float *)calloc((size_t)c->vocab_size, sizeof(float));
  if (!m->key_cache || !m->value_cache || !m->rope_r || !m->rope_i || !m->att || !m->logits) {
    orc_destroy(m);
    return NULL;
  }
  return m;
}

void orc_destroy(orc_model *m) {
  if (!m) return;
  for (int k = 0; k < ORC_KIND_COUNT; ++k) free((void *)m->lt[k]);
  free(m->key_cache); free(m->value_cache); free(m->rope_r); free(m->rope_i);
  free(m->x); free(m->xb); free(m->xb2); free(m->q); free(m->k); free(m->v);
  free(m->att); free(m->hb); free(m->hb2); free(m->qkv); free(m->logits);
  free(m);
}

int orc_set_tensor(orc_model *m, int kind, int layer, const void *data, int type) {
  if (kind < 0 || kind >= ORC_KIND_COUNT) return 1;
  m->ttype[kind] = type;
  if (is_layer_kind(kind)) {
    if (layer < 0 || layer >= m->c.n_layers) return 1;
    m->lt[kind][layer] = data;
  } else {
    m->t[kind] = data;
  }
  return 0;
}

void orc_reset(orc_model *m) {
  size_t kv = (size_t)m->c.n_layers * m->c.context_length * m->kv_dim;
  memset(m->key_cache, 0, kv * sizeof(float));
  memset(m->value_cache, 0, kv * sizeof(float));
}

float *orc_key_cache(orc_model *m, int layer) { return m->key_cache + (size_t)layer * m->c.context_length * m->kv_dim; }
float *orc_value_cache(orc_model *m, int layer) { return m->value_cache + (size_t)layer * m->c.context_length * m->kv_dim; }
const float *orc_rope_real(orc_model *m) { return m->rope_r; }
const float *orc_rope_imag(orc_model *m) { return m->rope_i; }

static inline float round_f16(float f) { return orc_f16_to_f32(orc_f32_to_f16(f)); }

static void kv_append(orc_model *m, int l, int pos) {
  float *kc = orc_key_cache(m, l) + (size_t)pos * m->kv_dim;
  float *vc = orc_value_cache(m, l) + (size_t)pos * m->kv_dim;
  for (int i = 0; i < m->kv_dim; ++i) {
    kc[i] = m->c.kv_fp16 ? round_f16(m->k[i]) : m->k[i];
    vc[i] = m->c.kv_fp16 ? round_f16(m->v[i]) : m->v[i];
  }
}

static void attention_all_heads(orc_model *m, int l, int pos, float *out) {
  const int hs = m->c.head_dim;
  const float *kc = orc_key_cache(m, l), *vc = orc_value_cache(m, l);
#pragma omp parallel for schedule(static)
  for (int h = 0; h < m->c.n_heads; ++h) {
    int kvo = (h / m->kv_mul) * hs;
    orc_attention_head(m->q + h * hs, kc + kvo, vc + kvo, m->kv_dim, hs, pos,
                       m->att + (size_t)h * m->c.context_length, out + h * hs);
  }
}

/* SwiGLU non-linearity: value / (float)(1.0 + Math.exp(-value)) (InferenceCore.java:162). */
static inline float silu(float v) { return v / (float)(1.0 + exp((double)(-v))); }

static void add_in_place(float *a, const float *b, int n) { for (int i = 0; i < n; ++i) a[i] = a[i] + b[i]; }

static int missing_tensors(const orc_model *m) {
  const orc_config *c = &m->c;
  if (!m->t[ORC_TOKEN_EMBD] || !m->t[ORC_OUTPUT_NORM]) return 1;
  for (int l = 0; l < c->n_layers; ++l) {
    int need[8], n = 0;
    need[n++] = ORC_ATTN_NORM; need[n++] = ORC_ATTN_OUTPUT; need[n++] = ORC_FFN_NORM;
    need[n++] = ORC_FFN_UP; need[n++] = ORC_FFN_DOWN;
    if (c->family == ORC_PHI3) need[n++] = ORC_ATTN_QKV;
    else { need[n++] = ORC_ATTN_Q; need[n++] = ORC_FFN_GATE; }
    for (int i = 0; i < n; ++i) if (!m->lt[need[i]][l]) return 1;
    if (c->family != ORC_PHI3 && (!m->lt[ORC_ATTN_K][l] || !m->lt[ORC_ATTN_V][l])) return 1;
    if (c->family == ORC_QWEN3 && (!m->lt[ORC_ATTN_Q_NORM][l] || !m->lt[ORC_ATTN_K_NORM][l])) return 1;
  }
  return 0;
}

int orc_forward(orc_model *m, int token, int pos, float *logits_out) {
  const orc_config *c = &m->c;
  if (token < 0 || token >= c->vocab_size || pos < 0 || pos >= c->context_length) return 1;
  if (missing_tensors(m)) return 2;
#ifdef _OPENMP
  if (c->n_threads > 0) omp_set_num_threads(c->n_threads);
#endif
  const int dim = c->dim, hs = c->head_dim, kv_dim = m->kv_dim, q_dim = m->q_dim, H = c->hidden_dim;
  const int wt = c->weight_type, f16x = c->f16_exact;
  const size_t half = (size_t)hs / 2;
  const float *cr = m->rope_r + (size_t)pos * half, *ci = m->rope_i + (size_t)pos * half;

  /* token_embedding_table.copyTo (InferenceCore.java:68 / :326 / :457) */
  for (int i = 0; i < dim; ++i) m->x[i] = tensor_get(m->t[ORC_TOKEN_EMBD], m->ttype[ORC_TOKEN_EMBD], (size_t)token * dim + i);

  for (int l = 0; l < c->n_layers; ++l) {
    orc_rmsnorm(m->xb, m->x, (const float *)m->lt[ORC_ATTN_NORM][l], 0, dim, c->rms_norm_eps);
    if (c->family == ORC_PHI3) {
      /* forwardJavaPhi3 (InferenceCore.java:465-487): fused QKV, split, NeoX rotation */
      orc_matmul(m->lt[ORC_ATTN_QKV][l], wt, m->xb, m->qkv, q_dim + 2 * kv_dim, dim, f16x);
      memcpy(m->q, m->qkv, (size_t)dim * sizeof(float));
      memcpy(m->k, m->qkv + dim, (size_t)kv_dim * sizeof(float));
      memcpy(m->v, m->qkv + dim + kv_dim, (size_t)kv_dim * sizeof(float));
      int dim_half = hs / 2;
      for (int i = 0; i < dim; i += 2) {
        int head_dim = i % hs, base = i - head_dim, ic = base + head_dim / 2;
        float fcr = cr[head_dim / 2], fci = ci[head_dim / 2];
        int rotn = i < kv_dim ? 2 : 1;
        for (int vv = 0; vv < rotn; ++vv) {
          float *vec = vv == 0 ? m->q : m->k;
          float v0 = vec[ic], v1 = vec[ic + dim_half];
          vec[ic] = v0 * fcr - v1 * fci;
          vec[ic + dim_half] = v0 * fci + v1 * fcr;
        }
      }
    } else {
      orc_matmul(m->lt[ORC_ATTN_Q][l], wt, m->xb, m->q, q_dim, dim, f16x);
      orc_matmul(m->lt[ORC_ATTN_K][l], wt, m->xb, m->k, kv_dim, dim, f16x);
      orc_matmul(m->lt[ORC_ATTN_V][l], wt, m->xb, m->v, kv_dim, dim, f16x);
      if (c->family == ORC_QWEN3) {
        /* forwardJavaQwen3 (InferenceCore.java:341-366): per-head RMSNorm of q and k, NeoX rotation */
        for (int h = 0; h < c->n_heads; ++h)
          orc_rmsnorm(m->q, m->q, (const float *)m->lt[ORC_ATTN_Q_NORM][l], h * hs, hs, c->rms_norm_eps);
        for (int h = 0; h < c->n_kv_heads; ++h)
          orc_rmsnorm(m->k, m->k, (const float *)m->lt[ORC_ATTN_K_NORM][l], h * hs, hs, c->rms_norm_eps);
        for (int h = 0; h < c->n_heads; ++h) {
          int rotn = h < c->n_kv_heads ? 2 : 1, po = h * hs, nc = hs / 2;
          for (int ic = 0; ic < nc; ++ic) {
            float fcr = cr[ic], fci = ci[ic];
            for (int vv = 0; vv < rotn; ++vv) {
              float *vec = vv == 0 ? m->q : m->k;
              float v0 = vec[po + ic], v1 = vec[po + ic + nc];
              vec[po + ic] = v0 * fcr - v1 * fci;
              vec[po + ic + nc] = v0 * fci + v1 * fcr;
            }
          }
        }
      } else {
        /* forwardJava (InferenceCore.java:82-94): interleaved pairs (i, i+1) */
        for (int i = 0; i < dim; i += 2) {
          int head_dim = i % hs;
          float fcr = cr[head_dim / 2], fci = ci[head_dim / 2];
          int rotn = i < kv_dim ? 2 : 1;
          for (int vv = 0; vv < rotn; ++vv) {
            float *vec = vv == 0 ? m->q : m->k;
            float v0 = vec[i], v1 = vec[i + 1];
            vec[i] = v0 * fcr - v1 * fci;
            vec[i + 1] = v0 * fci + v1 * fcr;
          }
        }
      }
    }
    kv_append(m, l, pos);
    attention_all_heads(m, l, pos, m->xb);
    orc_matmul(m->lt[ORC_ATTN_OUTPUT][l], wt, m->xb, m->xb2, dim, q_dim, f16x);
    add_in_place(m->x, m->xb2, dim);
    orc_rmsnorm(m->xb, m->x, (const float *)m->lt[ORC_FFN_NORM][l], 0, dim, c->rms_norm_eps);
    if (c->family == ORC_PHI3) {
      /* InferenceCore.java:527-535: hb = wGateUp.xb; hbG = silu(hb[0:H]); hbU = hb[H:2H] * hbG */
      orc_matmul(m->lt[ORC_FFN_UP][l], wt, m->xb, m->hb, 2 * H, dim, f16x);
      for (int i = 0; i < H; ++i) {
        float g = silu(m->hb[i]);
        m->hb2[i] = m->hb[H + i] * g;
      }
      orc_matmul(m->lt[ORC_FFN_DOWN][l], wt, m->hb2, m->xb, dim, H, f16x);
    } else {
      /* InferenceCore.java:157-168 */
      orc_matmul(m->lt[ORC_FFN_GATE][l], wt, m->xb, m->hb, H, dim, f16x);
      orc_matmul(m->lt[ORC_FFN_UP][l], wt, m->xb, m->hb2, H, dim, f16x);
      for (int i = 0; i < H; ++i) m->hb[i] = silu(m->hb[i]);
      for (int i = 0; i < H; ++i) m->hb[i] = m->hb[i] * m->hb2[i];
      orc_matmul(m->lt[ORC_FFN_DOWN][l], wt, m->hb, m->xb, dim, H, f16x);
    }
    add_in_place(m->x, m->xb, dim);
  }
  orc_rmsnorm(m->x, m->x, (const float *)m->t[ORC_OUTPUT_NORM], 0, dim, c->rms_norm_eps);
  const void *cls = m->t[ORC_OUTPUT] ? m->t[ORC_OUTPUT] : m->t[ORC_TOKEN_EMBD];
  int cls_type = m->t[ORC_OUTPUT] ? m->ttype[ORC_OUTPUT] : m->ttype[ORC_TOKEN_EMBD];
  orc_matmul(cls, cls_type, m->x, m->logits, c->vocab_size, dim, f16x);
  if (logits_out) memcpy(logits_out, m->logits, (size_t)c->vocab_size * sizeof(float));
  return 0;
}
