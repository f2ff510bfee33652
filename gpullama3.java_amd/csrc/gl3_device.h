// Device-side building blocks of the gfx950 decode path: fp16 conversion,
// wavefront reductions, coherent loads/stores for data exchanged between
// workgroups, and the grid barrier of the persistent per-token kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define GL3_WAVE 64
#define GL3_BLOCK 256         // threads per workgroup of the per-phase kernels
#define GL3_STEP_BLOCK 256    // threads per workgroup of the persistent per-token kernel and attention

namespace gl3 {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- fp16

// Exact binary16 -> binary32 (subnormals preserved: fp16 denormals are not
// flushed on gfx950 in the default float mode).
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ float h2f_lo(unsigned w) { return h2f((uint16_t)(w & 0xffffu)); }
__device__ __forceinline__ float h2f_hi(unsigned w) { return h2f((uint16_t)(w >> 16)); }
// binary32 -> binary16, round to nearest even
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// signed byte k of w as float (one v_cvt_f32_i32_sdwa with sext, src0_sel:BYTE_k)
template <int K>
__device__ __forceinline__ float sbyte(unsigned w) { return (float)(signed char)((w >> (8 * K)) & 0xffu); }

// ------------------------------------------------- coherent data exchange
// Activations written by one workgroup and read by another inside the same
// kernel go through agent-scope relaxed atomics: they bypass the per-XCD L2
// (which is not coherent across XCDs) without the cost of a release fence.

__device__ __forceinline__ float ld_coherent(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_coherent_u32(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent_u32(unsigned *p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_coherent_i32(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_coherent_u64(const unsigned long long *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte coherent load (buffer_load_dwordx4 with the agent-scope sc1 bit).
// `base` builds the buffer descriptor and must be the same in every lane of
// the wave (a per-lane base turns the load into a loop over distinct bases);
// per-lane positions go in byte_off.
// Unlike the atomic loads above, the compiler may batch these, so a loop of
// them keeps many requests in flight.  Out-of-range offsets read zeros.
__device__ __forceinline__ u32x4 ld_coherent_x4(const void *base, unsigned byte_off) {
  // the base is wave-uniform by contract: read it from lane 0 so the descriptor lives in SGPRs
  const unsigned long long b = (unsigned long long)base;
  // (readfirstlane returns int: widen through unsigned, never by sign extension)
  const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((unsigned)(b >> 32));
  const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((unsigned)b);
  const unsigned long long ub = ((unsigned long long)hi << 32) | (unsigned long long)lo;
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)ub, 0, 0x7fffffff, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16 /* sc1 */);
}
__device__ __forceinline__ float4 ld_coherent_f4(const float *base, unsigned index) {
  u32x4 v = ld_coherent_x4(base, index * 4u);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// Wait until this wave's outstanding vector-memory operations (including the
// coherent stores above) have completed.  Used instead of a release fence
// before signalling another workgroup.
__device__ __forceinline__ void vmem_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Streaming (read-once) 16-byte load of weights / KV.
__device__ __forceinline__ u32x4 ld_stream(const void *p) { return __builtin_nontemporal_load((const u32x4 *)p); }

// ------------------------------------------------------------ lane / wave ids
// Lane and wave indices as values the compiler cannot hoist out of the layer
// loop of the persistent kernel: address arithmetic derived from them stays in
// the phase that uses it instead of holding registers for the whole kernel.
__device__ __forceinline__ int lane_id() {
  int l = (int)(threadIdx.x % GL3_WAVE);
  asm volatile("" : "+v"(l));
  return l;
}
__device__ __forceinline__ int wave_id() {
  int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / GL3_WAVE));
  asm volatile("" : "+s"(w));
  return w;
}

// ------------------------------------------------------------ reductions

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets the row sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x128>(v);  // row_ror:8
  return v;
}
// Sum over the wavefront, result uniform in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Sum / max over the four lanes l, l^16, l^32, l^48 (one value per 16-lane row),
// result identical in all four: v_permlane16_swap then v_permlane32_swap, no LDS.
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float xrow_sum(float v) {
  u32x2_t a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  u32x2_t b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float xrow_max(float v) {
  u32x2_t a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  u32x2_t b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Block-wide sum over BS threads; red must hold BS/64 floats.  Ends with the
// result visible to every thread; red may be reused after the call.
template <int BS>
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int wave = threadIdx.x / GL3_WAVE, lane = threadIdx.x % GL3_WAVE;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < BS / GL3_WAVE; ++w) s += red[w];
  return s;
}

// Sum over aligned groups of LP lanes (LP = 8 or 16); every lane of a group
// gets the group's sum.  quad_perm xor 1, xor 2, then row_half_mirror (the
// other quad of the 8-lane half row) and, for 16, row_mirror (the other half).
template <int LP>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  if (LP == 16) v += dpp<0x140>(v);
  return v;
}

// ------------------------------------------------------------ grid barrier
// Fence-free barrier for the persistent kernel (all workgroups co-resident,
// guaranteed by the cooperative launch).  Workgroup b arrives on counter
// b % 64 with a no-return atomic (few arrivals per address); wave 0 then polls
// the 64 counters, one per lane, in parallel.  Counters only grow: the barrier with global index e (across all
// launches since the last reset) completes when counter j reaches
// e * size_of_group(j).  Each poll is bounded: after spin_limit polls the
// barrier raises *err and every workgroup leaves the kernel at its next
// barrier, so a lost workgroup can never hang the GPU.
struct GridBarrier {
  unsigned *ctr;     // GL3_BAR_GROUPS counters, GL3_BAR_STRIDE words apart
  unsigned *err;     // error flag (0 = ok)
  unsigned spin_limit;
};

#define GL3_BAR_STRIDE 64  // words between counters (one cache line each)
#define GL3_BAR_GROUPS 64  // counters; workgroup b arrives on counter b % 64

// Arrival: this workgroup's earlier writes are complete, then one no-return
// atomic on its group counter.  Loads issued between grid_arrive and grid_wait
// (e.g. weights of the next phase) overlap the wait.
__device__ __forceinline__ void grid_arrive(const GridBarrier &gb) {
  vmem_drain();
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(gb.ctr + (blockIdx.x % GL3_BAR_GROUPS) * GL3_BAR_STRIDE, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until every workgroup has arrived at barrier `epoch`; false when the
// barrier timed out or another workgroup raised the error flag.
__device__ __forceinline__ bool grid_wait(const GridBarrier &gb, unsigned epoch) {
  const unsigned nb = gridDim.x;
  __shared__ int bar_ok;
  if (threadIdx.x < GL3_WAVE) {
    const unsigned g = threadIdx.x % GL3_BAR_GROUPS;
    const unsigned gsize = nb / GL3_BAR_GROUPS + (g < (nb % GL3_BAR_GROUPS) ? 1u : 0u);
    const unsigned target = epoch * gsize;
    unsigned spins = 0;
    bool ok = true;
    for (;;) {
      unsigned v = (threadIdx.x < GL3_BAR_GROUPS) ? ld_coherent_u32(gb.ctr + g * GL3_BAR_STRIDE) : target;
      if (__all((int)(v - target) >= 0)) break;
      if (ld_coherent_u32(gb.err) != 0u || ++spins > gb.spin_limit) {
        if (threadIdx.x == 0) st_coherent_u32(gb.err, 1u);
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (threadIdx.x == 0) bar_ok = ok ? 1 : 0;
  }
  __syncthreads();
  return bar_ok != 0;
}

__device__ __forceinline__ bool grid_barrier(const GridBarrier &gb, unsigned epoch) {
  grid_arrive(gb);
  return grid_wait(gb, epoch);
}

// ------------------------------------------------------------ tagged cells
// Inside the persistent kernel, the vectors passed from one phase to the next
// are arrays of 8-byte cells {fp32 value, 32-bit tag}.  The producer writes a
// cell with one agent-scope 8-byte store (single-copy atomic), so a consumer
// that reads a cell carrying the tag it expects has read that phase's value:
// the read itself is the synchronization, with no barrier, fence or flag.  Tags
// come from a counter that does not repeat within the life of a plan, so a
// stale cell never carries the expected tag.  A consumer retries a cell that
// is not ready; after spin_limit retries it raises *err, and every later wait
// gives up at once, so a lost producer cannot hang the GPU.
struct TagWait {
  unsigned *err;
  unsigned spin_limit;
};

__device__ __forceinline__ void st_tagged(uint2 *p, float v, unsigned tag) {
  const unsigned long long w = ((unsigned long long)tag << 32) | (unsigned long long)__float_as_uint(v);
  __hip_atomic_store((unsigned long long *)p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Slow path of a tagged read: one more poll after a short sleep; false once
// the wait has given up.  The shared error word is read only every 32nd
// retry: read by every waiting thread at every retry it becomes a hot spot.
__device__ __forceinline__ bool tag_retry(const TagWait &tw, unsigned &spins) {
  ++spins;
  if (spins > tw.spin_limit || ((spins & 31u) == 0u && ld_coherent_u32(tw.err) != 0u)) {
    st_coherent_u32(tw.err, 1u);
    return false;
  }
  __builtin_amdgcn_s_sleep(1);
  return true;
}

// v[n] = the 4 values of cells e[n] .. e[n] + 3 (e[n] a multiple of 4); all
// first reads are issued before any is checked, then missing cells are polled
// one float4 at a time (polling all of them at once multiplies the polling
// traffic, which competes with the weight stream: measured slower).
//
// Load side of the cell protocol: each 16-byte load covers two cells and is
// accepted only when both carry the tag.  What it relies on is that each
// naturally aligned 8-byte half of the load is observed whole, i.e. never
// pairs the value of one store with the tag of another.  The 16 bytes lie in
// one 64-byte line and reach the memory side as one request, while every
// write to a cell is one aligned 8-byte store; a torn half would need the
// 16-byte read to be split below 8-byte granularity and interleaved with a
// store, which the cache hierarchy (line-granular requests) does not do.  This
// is an observed hardware property, not one the programming model states for
// loads wider than 8 bytes; the per-token parity tests (every cell of every
// exchanged vector, thousands of tokens per run) would show a torn read as a
// wrong value, and ld_tagged1 (one 8-byte atomic load per cell) is the drop-in
// replacement if a target ever breaks it.
template <int N>
__device__ __forceinline__ void ld_tagged4(const uint2 *p, const int (&e)[N], unsigned tag, const TagWait &tw,
                                           float4 (&v)[N]) {
  u32x4 a[N], b[N];
#pragma unroll
  for (int n = 0; n < N; ++n) {
    a[n] = ld_coherent_x4(p, (unsigned)e[n] * 8u);
    b[n] = ld_coherent_x4(p, (unsigned)e[n] * 8u + 16u);
  }
#pragma unroll
  for (int n = 0; n < N; ++n) {
    unsigned spins = 0;
    while (!(a[n].y == tag && a[n].w == tag && b[n].y == tag && b[n].w == tag)) {
      if (!tag_retry(tw, spins)) break;
      a[n] = ld_coherent_x4(p, (unsigned)e[n] * 8u);
      b[n] = ld_coherent_x4(p, (unsigned)e[n] * 8u + 16u);
    }
    v[n] = make_float4(__uint_as_float(a[n].x), __uint_as_float(a[n].z), __uint_as_float(b[n].x),
                       __uint_as_float(b[n].z));
  }
}

__device__ __forceinline__ float ld_tagged1(const uint2 *p, int e, unsigned tag, const TagWait &tw) {
  unsigned long long w = ld_coherent_u64((const unsigned long long *)(p + e));
  unsigned spins = 0;
  while ((unsigned)(w >> 32) != tag) {
    if (!tag_retry(tw, spins)) break;
    w = ld_coherent_u64((const unsigned long long *)(p + e));
  }
  return __uint_as_float((unsigned)w);
}

}  // namespace gl3
