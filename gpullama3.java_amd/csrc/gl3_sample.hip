// On-device sampling of the next token from the logits of a decode step: the
// reference's Sampler.selectSampler (inference/sampler/Sampler.java:74-122)
// with CategoricalSampler (CategoricalSampler.java:31-42) and ToppSampler
// (ToppSampler.java:61-156), for a draw `coin` the host supplies in place of
// rng.nextFloat(1f).
//
// One workgroup of 1024 threads.  Probabilities follow the reference's float
// arithmetic (logit / temperature, max, exp, divide by the sum) with two
// deviations: exp is the float expf (the reference rounds a double exp to
// float; the two differ by an ulp or two), and the sum of the exponentials is the float nearest
// their exact sum (the reference's float sum in index order drifts by up to
// ~1e-4 relative over a 128k vocabulary); the cumulative sums the samplers
// compare with the draw and with topp are exact: every probability is converted to a 48-bit fixed-point
// integer and summed in 64-bit integers, so the result does not depend on the
// order of the additions (the reference adds floats in index or heap order;
// the two differ by float rounding only).  The top-p nucleus is found without
// sorting: a radix select over the probabilities' bit patterns (exponent byte,
// then 12 + 11 mantissa bits; histograms of counts and fixed-point mass in LDS,
// the exponent's one per wave) finds the smallest
// probability the nucleus contains and how many tokens of that probability it
// takes; a second select finds where the draw falls.  Candidates are visited
// in descending probability, ties in index order.  The top-p candidates
// (p >= the cutoff) are listed in index order as the probabilities are formed,
// so the select passes read that list, not the vocabulary.  After a decode step
// the maximum logit is read from the step's argmax keys instead of a pass.
#include "gl3_internal.h"

namespace gl3 {

namespace {

constexpr int SBS = 1024;                 // threads of the sampling workgroup
constexpr int SW = SBS / GL3_WAVE;        // waves
constexpr int NEXP = 256;                 // first radix pass: the exponent byte, one histogram per wave
constexpr int NBIN = 4096;                // later passes: bits [22:11] (4096 bins) and [10:0] (2048 bins)
constexpr double FX = 281474976710656.0;  // 2^48: fixed-point scale of a probability

typedef unsigned long long u64;

// p (finite, >= 0) as a 48-bit fixed-point integer, truncated: exact from the bits
__device__ __forceinline__ u64 to_fx(float p) {
  const unsigned b = __float_as_uint(p);
  const int e = (int)((b >> 23) & 0xffu);
  const u64 m = e ? (u64)((b & 0x7fffffu) | 0x800000u) : (u64)(b & 0x7fffffu);
  const int sh = (e ? e : 1) - 150 + 48;  // p = m 2^(e - 150); times 2^48
  return sh >= 0 ? (sh < 40 ? m << sh : 0ull) : (sh > -64 ? m >> (-sh) : 0ull);
}

// Block reductions / scans over the 1024 threads; `sh` holds SW + 1 entries.
__device__ __forceinline__ float block_max(float v, float *sh) {
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x / GL3_WAVE, l = threadIdx.x % GL3_WAVE;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  float r = sh[0];
  for (int i = 1; i < SW; ++i) r = fmaxf(r, sh[i]);
  return r;
}

// Sum of the threads' values: per wave a fixed tree, then the waves in order (deterministic).
__device__ __forceinline__ double block_sum_d(double v, double *sh) {
  for (int o = 1; o < GL3_WAVE; o <<= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x / GL3_WAVE, l = threadIdx.x % GL3_WAVE;
  __syncthreads();
  if (l == 0) sh[w] = v;
  __syncthreads();
  double r = 0.0;
  for (int i = 0; i < SW; ++i) r += sh[i];
  return r;
}

__device__ __forceinline__ u64 wave_sum_u64(u64 v) {
  for (int o = 1; o < GL3_WAVE; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

// Exclusive prefix sum over threads (thread order) and the total.
__device__ __forceinline__ u64 block_scan_u64(u64 v, u64 *sh, u64 *total) {
  const int w = threadIdx.x / GL3_WAVE, l = threadIdx.x % GL3_WAVE;
  u64 inc = v;
  for (int o = 1; o < GL3_WAVE; o <<= 1) {
    const u64 t = __shfl_up(inc, o);
    if (l >= o) inc += t;
  }
  __syncthreads();
  if (l == GL3_WAVE - 1) sh[w] = inc;
  __syncthreads();
  u64 before = 0, all = 0;
  for (int i = 0; i < SW; ++i) {
    if (i < w) before += sh[i];
    all += sh[i];
  }
  *total = all;
  return before + inc - v;
}

// The elements are cut into SW contiguous ranges of a multiple of 256, one per
// wave (index order is range order); a wave reads its range as float4 groups,
// 64 lanes at a time (coalesced).
__device__ __forceinline__ int wave_range(int n) { return ((n + SW - 1) / SW + 255) / 256 * 256; }

__device__ __forceinline__ unsigned key_of(float p) { return __float_as_uint(p); }  // p >= 0: bits are monotone

struct SelectState {
  unsigned prefix, mask;  // bits of the selected key fixed so far
  u64 above;              // mass of the candidates whose key is above the selected range
  int found;              // 0: the candidates' mass never exceeds the target
  unsigned cnt;           // candidates with the selected key (after the last pass)
};

// Picks the bin (scanned from the highest) where the mass, added to `above`,
// first exceeds target; updates the state.  nb <= NBIN bins; thread t scans
// bins nb-1-K*t .. nb-K*(t+1), K = max(1, nb / SBS).
__device__ void pick_bin(const unsigned *hcnt, const u64 *hsum, int nb, int sh, unsigned dmask, u64 target, u64 *shu,
                         SelectState *st) {
  const int t = threadIdx.x;
  const int K = nb >= SBS ? nb / SBS : 1;
  const unsigned prefix = st->prefix, mask = st->mask;
  const u64 above0 = st->above;
  u64 loc = 0;
  for (int k = 0; k < K; ++k) {
    const int b = nb - 1 - K * t - k;
    if (b >= 0) loc += hsum[b];
  }
  u64 tot;
  const u64 ex = block_scan_u64(loc, shu, &tot) + above0;
  __syncthreads();
  if (above0 + tot <= target) {  // no candidate pushes the mass past the target
    if (t == 0) st->found = 0;
  } else if (ex <= target && ex + loc > target) {
    u64 acc = ex;
    for (int k = 0; k < K; ++k) {
      const int b = nb - 1 - K * t - k;
      if (acc + hsum[b] > target) {
        st->above = acc;
        st->prefix = prefix | ((unsigned)b << sh);
        st->mask = mask | (dmask << sh);
        st->cnt = hcnt[b];
        break;
      }
      acc += hsum[b];
    }
  }
  __syncthreads();
}

// Radix select over the candidates (p >= cutoff) for the largest key tau such
// that the mass of the candidates with key > tau is <= target < mass with key
// >= tau.  The exponent byte's histogram (hecnt/hesum, all candidates) is given;
// two passes over the candidates with that exponent fix bits [22:11] and [10:0].
// The candidates are the compact list cand: wave w's in cand[w R .. w R + ccnt[w]).
__device__ void radix_select(const float *p, const int *cand, const unsigned *ccnt, int R, u64 target,
                             const unsigned *hecnt, const u64 *hesum, unsigned *hcnt, u64 *hsum, u64 *shu,
                             SelectState *st) {
  const int t = threadIdx.x, wave = t / GL3_WAVE, lane = t % GL3_WAVE;
  if (t == 0) {
    st->prefix = 0u;
    st->mask = 0u;
    st->above = 0ull;
    st->found = 1;
    st->cnt = 0u;
  }
  __syncthreads();
  pick_bin(hecnt, hesum, NEXP, 23, 0xffu, target, shu, st);
  const int shifts[2] = {11, 0};
  const unsigned dmasks[2] = {0xfffu, 0x7ffu};  // bits [22:11], then [10:0]
  for (int pass = 0; pass < 2; ++pass) {
    if (!st->found) return;
    const int sh = shifts[pass];
    const unsigned dmask = dmasks[pass];
    const int nb = (int)dmask + 1;
    for (int b = t; b < nb; b += SBS) {
      hcnt[b] = 0u;
      hsum[b] = 0ull;
    }
    __syncthreads();
    const unsigned prefix = st->prefix, mask = st->mask;
    const int c0 = wave * R, c1 = c0 + (int)ccnt[wave];
    for (int c = c0 + lane; c < c1; c += GL3_WAVE) {
      const float q = p[cand[c]];
      const unsigned k = key_of(q);
      if ((k & mask) == prefix) {
        const unsigned b = (k >> sh) & dmask;
        atomicAdd(&hcnt[b], 1u);
        atomicAdd(&hsum[b], to_fx(q));
      }
    }
    __syncthreads();
    pick_bin(hcnt, hsum, nb, sh, dmask, target, shu, st);
  }
}

// The first element, in index order, at which the running total of w(i) exceeds
// target (integer weights), or -1 when the total does not.  wt[SW]: the waves'
// range totals.  The wave whose range holds the crossing stages it in pieces of
// 16 x 64 weights through LDS and scans lane sub-chunks of 16.
template <class W>
__device__ int first_crossing_in(const W &w, int r0, int r1, u64 target, const u64 *wt, u64 *piece, int *shi) {
  const int t = threadIdx.x, wave = t / GL3_WAVE, lane = t % GL3_WAVE;
  if (t == 0) shi[0] = -1;
  __syncthreads();
  u64 before = 0;
  for (int i = 0; i < wave; ++i) before += wt[i];
  if (before <= target && before + wt[wave] > target) {
    u64 acc = before;
    for (int p0 = r0; p0 < r1; p0 += 16 * GL3_WAVE) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int i = p0 + j * GL3_WAVE + lane;
        piece[j * GL3_WAVE + lane] = i < r1 ? w(i) : 0ull;
      }
      u64 ls = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) ls += piece[16 * lane + j];
      u64 inc = ls;
      for (int o = 1; o < GL3_WAVE; o <<= 1) {
        const u64 v = __shfl_up(inc, o);
        if (lane >= o) inc += v;
      }
      const u64 tot = __shfl(inc, GL3_WAVE - 1);
      if (acc + tot > target) {
        const u64 ex = acc + inc - ls;
        if (ex <= target && ex + ls > target) {
          u64 k = ex;
          for (int j = 0; j < 16; ++j) {
            k += piece[16 * lane + j];
            if (target < k) {
              shi[0] = p0 + 16 * lane + j;
              break;
            }
          }
        }
        break;
      }
      acc += tot;
    }
  }
  __syncthreads();
  return shi[0];
}
// The same over the waves' ranges of the n elements.
template <class W>
__device__ int first_crossing(const W &w, int n, u64 target, const u64 *wt, u64 *piece, int *shi) {
  const int wave = threadIdx.x / GL3_WAVE;
  const int R = wave_range(n), r0 = wave * R, r1 = min(n, r0 + R);
  return first_crossing_in(w, r0, r1, target, wt, piece, shi);
}

struct FxProb {
  const float *p;
  __device__ __forceinline__ u64 operator()(int i) const { return to_fx(p[i]); }
};
// 1 for the candidates (positions in the compact list) whose key is `key`
struct KeyCount {
  const float *p;
  const int *cand;
  unsigned key;
  __device__ __forceinline__ u64 operator()(int c) const { return key_of(p[cand[c]]) == key ? 1ull : 0ull; }
};

}  // namespace

struct SampleArgs {
  const float *logits;  // [n]
  int n;
  float temperature, topp;
  const float *coins;   // draws; this call uses coins[coin_index]
  int coin_index;
  float *probs;         // scratch [2 n]: the probabilities, then (top-p) the candidates' indices
  int *token_out;       // nullable: the sampled token
  DecodeState *st;      // nullable: the next step forwards the sampled token
  int *rec;             // nullable: rec[coin_index] = the sampled token
  // nullable (with st): the decode step's argmax keys (the logits' orderable
  // keys, st->nbest of them at best + (st->parity ^ 1) * st->nbest once the step
  // has advanced the control block), so the maximum logit needs no pass
  const unsigned long long *best;
};

__global__ __launch_bounds__(SBS) void sample_kernel(SampleArgs a) {
  __shared__ unsigned hcnt[NBIN];  // first: per-wave exponent histograms [SW][NEXP]; later: [2048]
  __shared__ u64 hsum[NBIN];
  __shared__ unsigned hecnt[NEXP];
  __shared__ u64 hesum[NEXP];
  __shared__ float shf[SW + 1];
  __shared__ double shd[SW + 1];
  __shared__ u64 shu[SW + 1];
  __shared__ u64 wt[SW];
  __shared__ int shi[4];
  __shared__ unsigned ccnt[SW];  // top-p: candidates per wave in the compact list
  __shared__ SelectState sel;
  const int t = threadIdx.x, n = a.n, wave = t / GL3_WAVE, lane = t % GL3_WAVE;
  int token = 0;
  if (a.temperature == 0.0f) {
    // TENSOR_ARGMAX (Sampler.java:76-78): first maximum of the logits
    unsigned long long best = 0;
    for (int i = t; i < n; i += SBS) {
      const unsigned long long k = argmax_key(a.logits[i], i);
      best = k > best ? k : best;
    }
    for (int o = 32; o >= 1; o >>= 1) {
      const unsigned long long other = __shfl_xor(best, o);
      best = other > best ? other : best;
    }
    if (t % GL3_WAVE == 0) shu[t / GL3_WAVE] = best;
    __syncthreads();
    best = 0;
    for (int i = 0; i < SW; ++i) best = shu[i] > best ? shu[i] : best;
    token = argmax_key_row(best);
  } else {
    // divideInPlace + softmaxInPlace (FloatTensor.java:203-205, 211-219); one
    // workgroup streams the vector, so every pass reads float4 groups, several in flight
    const int n4 = n >> 2;
    const float4 *l4 = (const float4 *)a.logits;
    float4 *p4 = (float4 *)a.probs;
    const float T = a.temperature;
    float mx = -INFINITY;
    if (a.best && a.st) {
      // max_i (l_i / T) = (max_i l_i) / T (division by T > 0 is monotone): the
      // largest of the step's argmax keys holds the largest logit
      const int *sv = (const int *)a.st;
      const int par = ld_coherent_i32(sv + 3), nb = ld_coherent_i32(sv + 5);
      const unsigned long long *keys = a.best + (size_t)(par ^ 1) * nb;
      unsigned long long bk = 0;
      for (int i = t; i < nb; i += SBS) {
        const unsigned long long k = ld_coherent_u64(keys + i);
        bk = k > bk ? k : bk;
      }
      for (int o = 32; o >= 1; o >>= 1) {
        const unsigned long long other = __shfl_xor(bk, o);
        bk = other > bk ? other : bk;
      }
      if (lane == 0) shu[wave] = bk;
      __syncthreads();
      bk = 0;
      for (int i = 0; i < SW; ++i) bk = shu[i] > bk ? shu[i] : bk;
      __syncthreads();
      const unsigned kb = (unsigned)(bk >> 32);
      mx = __uint_as_float((kb & 0x80000000u) ? (kb & 0x7fffffffu) : ~kb) / T;
    } else {
#pragma unroll 4
      for (int i = t; i < n4; i += SBS) {
        const float4 v = l4[i];
        mx = fmaxf(fmaxf(fmaxf(mx, v.x / T), v.y / T), fmaxf(v.z / T, v.w / T));
      }
      for (int i = 4 * n4 + t; i < n; i += SBS) mx = fmaxf(mx, a.logits[i] / T);
      mx = block_max(mx, shf);
    }
    // the sum in double, rounded once: the float nearest the exact sum of the
    // float exponentials (the reference adds them in float, in index order)
    double s = 0.0;
#pragma unroll 4
    for (int i = t; i < n4; i += SBS) {
      const float4 v = l4[i];
      float4 e;
      e.x = expf(v.x / T - mx);
      e.y = expf(v.y / T - mx);
      e.z = expf(v.z / T - mx);
      e.w = expf(v.w / T - mx);
      p4[i] = e;
      s += ((double)e.x + (double)e.y) + ((double)e.z + (double)e.w);
    }
    for (int i = 4 * n4 + t; i < n; i += SBS) {
      const float e = expf(a.logits[i] / T - mx);
      a.probs[i] = e;
      s += (double)e;
    }
    const float sum = (float)block_sum_d(s, shd);
    const float coin = a.coins[a.coin_index];
    const float topp = a.topp;
    const bool categorical = topp <= 0.0f || topp >= 1.0f;
    // ToppSampler's candidates: p >= (1 - topp) / (n - 1) (ToppSampler.java:63-70)
    const float cutoff = categorical ? 0.0f : (1.0f - topp) / (float)(n - 1);
    // probabilities in place, in the waves' ranges: each wave totals its range's
    // fixed-point mass (categorical) or histograms its candidates by exponent and
    // lists their indices, in index order, in cand[r0 ..] (top-p; the later
    // passes visit the list only: at low temperatures it is a few tokens)
    int *cand = (int *)(a.probs + n);
    for (int b = t; b < SW * NEXP; b += SBS) {
      hcnt[b] = 0u;
      hsum[b] = 0ull;
    }
    __syncthreads();
    const int R = wave_range(n), r0 = wave * R, r1 = min(n, r0 + R);
    u64 tot = 0;
    unsigned nc = 0;  // this wave's candidates so far
#pragma unroll 2
    for (int g = r0 / 4 + lane; g < (r0 + R) / 4; g += GL3_WAVE) {
      float q[4];
      if (4 * g + 3 < n) {
        float4 v = p4[g];
        v.x = v.x / sum;
        v.y = v.y / sum;
        v.z = v.z / sum;
        v.w = v.w / sum;
        p4[g] = v;
        q[0] = v.x;
        q[1] = v.y;
        q[2] = v.z;
        q[3] = v.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = 4 * g + j;
          q[j] = 0.0f;
          if (i < r1) {
            q[j] = a.probs[i] / sum;
            a.probs[i] = q[j];
          }
        }
      }
      unsigned mine = 0;  // this lane's candidates (bit j: element 4 g + j)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * g + j;
        if (categorical) {
          tot += i < r1 ? to_fx(q[j]) : 0ull;
        } else if (i < r1 && q[j] >= cutoff) {
          const unsigned b = (key_of(q[j]) >> 23) & 0xffu;
          atomicAdd(&hcnt[wave * NEXP + b], 1u);
          atomicAdd(&hsum[wave * NEXP + b], to_fx(q[j]));
          mine |= 1u << j;
        }
      }
      if (!categorical) {
        // lanes in order, each lane's elements in order: index order
        const unsigned c = (unsigned)__builtin_popcount(mine);
        unsigned inc = c;
        for (int o = 1; o < GL3_WAVE; o <<= 1) {
          const unsigned v = __shfl_up(inc, o);
          if (lane >= o) inc += v;
        }
        unsigned at = nc + inc - c;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (mine & (1u << j)) cand[r0 + at++] = 4 * g + j;
        nc += __shfl(inc, GL3_WAVE - 1);
      }
    }
    if (!categorical && lane == 0) ccnt[wave] = nc;
    if (categorical) {
      tot = wave_sum_u64(tot);
      if (lane == 0) wt[wave] = tot;
    }
    __syncthreads();
    u64 *piece = hsum;  // the staging of first_crossing reuses the histograms' LDS
    if (categorical) {
      // CategoricalSampler (CategoricalSampler.java:31-42): the first token whose
      // cumulative mass exceeds the draw
      token = first_crossing(FxProb{a.probs}, n, (u64)((double)coin * FX), wt, piece, shi);
      if (token < 0) token = n - 1;  // the reference's fallback for rounding
    } else {
      // the smallest set of the most probable candidates whose mass exceeds topp
      // (ToppSampler.java:119-131), then the draw scaled by that mass walks them in
      // descending order (:134-150)
      for (int b = t; b < NEXP; b += SBS) {
        unsigned c = 0;
        u64 m = 0;
        for (int w = 0; w < SW; ++w) {
          c += hcnt[w * NEXP + b];
          m += hsum[w * NEXP + b];
        }
        hecnt[b] = c;
        hesum[b] = m;
      }
      __syncthreads();
      const u64 target = (u64)((double)topp * FX);
      radix_select(a.probs, cand, ccnt, R, target, hecnt, hesum, hcnt, hsum, shu, &sel);
      u64 mass;
      if (sel.found) {
        const u64 ptau = to_fx(__uint_as_float(sel.prefix));
        const u64 m = ptau > 0 ? (target - sel.above) / ptau + 1 : (u64)sel.cnt;
        mass = sel.above + m * ptau;
      } else {
        // the candidates' mass never exceeds topp: the nucleus is every candidate
        u64 c = 0;
        for (int b = t; b < NEXP; b += SBS) c += hesum[b];
        u64 all;
        block_scan_u64(c, shu, &all);
        mass = all;
      }
      __syncthreads();
      const u64 r = (u64)((double)coin * (double)mass);
      radix_select(a.probs, cand, ccnt, R, r, hecnt, hesum, hcnt, hsum, shu, &sel);
      token = -1;
      const int c0 = r0, c1 = r0 + (int)ccnt[wave];  // this wave's part of the candidate list
      if (sel.found) {
        const u64 psig = to_fx(__uint_as_float(sel.prefix));
        const u64 j = psig > 0 ? (r - sel.above) / psig + 1 : 1;
        // the j-th candidate with that probability, in index order
        const KeyCount kc{a.probs, cand, sel.prefix};
        u64 c = 0;
        for (int i = c0 + lane; i < c1; i += GL3_WAVE) c += kc(i);
        c = wave_sum_u64(c);
        __syncthreads();
        if (lane == 0) wt[wave] = c;
        __syncthreads();
        const int at = first_crossing_in(kc, c0, c1, j - 1, wt, piece, shi);
        token = at >= 0 ? cand[at] : -1;
      }
      if (token < 0) {
        // rounding only: the last candidate of the walk (the least probable one)
        unsigned long long best = 0;
        for (int c = c0 + lane; c < c1; c += GL3_WAVE) {
          const int i = cand[c];
          const float q = a.probs[i];
          // smallest probability, then the largest index (last in the walk order)
          const unsigned long long k = ((unsigned long long)(~key_of(q)) << 32) | (unsigned)i;
          best = k > best ? k : best;
        }
        for (int o = 32; o >= 1; o >>= 1) {
          const unsigned long long other = __shfl_xor(best, o);
          best = other > best ? other : best;
        }
        __syncthreads();
        if (t % GL3_WAVE == 0) shu[t / GL3_WAVE] = best;
        __syncthreads();
        best = 0;
        for (int i = 0; i < SW; ++i) best = shu[i] > best ? shu[i] : best;
        token = (int)(unsigned)(best & 0xffffffffu);
      }
    }
  }
  if (t == 0) {
    if (a.token_out) *a.token_out = token;
    if (a.rec) a.rec[a.coin_index] = token;
    if (a.st) {
      int *s = (int *)a.st;
      __hip_atomic_store(s + 1, token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(s + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

hipError_t launch_sample(const float *logits, int n, float temperature, float topp, const float *coins, int coin_index,
                         float *probs, int *token_out, DecodeState *st, int *rec, const unsigned long long *best,
                         hipStream_t s) {
  SampleArgs a{logits, n, temperature, topp, coins, coin_index, probs, token_out, st, rec, best};
  hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(SBS), 0, s, a);
  return hipGetLastError();
}

}  // namespace gl3
