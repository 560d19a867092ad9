// Device-side helpers shared by the mvsd kernels (gfx950, wave64).
//
// Conventions used throughout:
//   * workgroups are 256 threads = 4 wavefronts of 64 lanes;
//   * streaming loads are 16-byte vector loads (4 x fp32 or 8 x bf16/fp16) laid out so
//     that consecutive lanes touch consecutive 16-byte segments (fully coalesced);
//   * argmax ties resolve to the lowest index and NaN ranks above every number, which is
//     torch.argmax's rule and the first-index rule of the reference's Triton reduction
//     (minivllm/sample/rejection_sampler.py:921-925).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mvsd.h"

namespace mvsd {

constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// ------------------------------------------------------------------ element types ----

template <int DT>
struct Elem;

template <>
struct Elem<MVSD_F32> {
  using storage = float;
  static constexpr int kVec = 4;  // elements per 16-byte load
  __device__ static inline float cvt(float v) { return v; }
  __device__ static inline float ninf() { return -INFINITY; }
};

template <>
struct Elem<MVSD_BF16> {
  using storage = uint16_t;
  static constexpr int kVec = 8;
  __device__ static inline float cvt(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }
  __device__ static inline uint16_t ninf() { return 0xff80; }
};

template <>
struct Elem<MVSD_F16> {
  using storage = _Float16;
  static constexpr int kVec = 8;
  __device__ static inline float cvt(_Float16 v) { return static_cast<float>(v); }
  __device__ static inline _Float16 ninf() { return static_cast<_Float16>(-INFINITY); }
};

// Load kVec consecutive elements starting at p[idx] and convert them to fp32.  Elements at
// or beyond `limit` are replaced by `fill`.  `aligned` (wave-uniform) says p + idx is 16-byte
// aligned whenever idx is a multiple of kVec; otherwise scalar loads are used.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ inline void load_vec(const typename Elem<DT>::storage* __restrict__ p, int64_t idx,
                                int64_t limit, bool aligned, float fill,
                                float (&out)[Elem<DT>::kVec]) {
  constexpr int V = Elem<DT>::kVec;
  using S = typename Elem<DT>::storage;
  if (aligned && idx + V <= limit) {
    const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + idx));
    const S* s = reinterpret_cast<const S*>(&raw);
#pragma unroll
    for (int j = 0; j < V; ++j) out[j] = Elem<DT>::cvt(s[j]);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) out[j] = (idx + j < limit) ? Elem<DT>::cvt(p[idx + j]) : fill;
  }
}

// ------------------------------------------------------------------ comparisons ------

// True when (a, ia) ranks above (b, ib): NaN above numbers, larger value, then lower index.
// Written branch-free (bitwise logic only): the short-circuit form was lowered by the gfx950
// backend into a control-flow diamond whose phi moves dropped the update for the first
// element of an unrolled argmax loop.
__device__ inline bool argmax_better(float a, int ia, float b, int ib) {
  const bool an = a != a;
  const bool bn = b != b;
  const bool lower = ia < ib;
  const bool num = (a > b) | ((a == b) & lower);
  return (an & (!bn | lower)) | (!an & !bn & num);
}

// (bv, bi) <- (v, i) when (v, i) ranks above it and `valid`; branch-free select.
__device__ inline void argmax_update(float& bv, int& bi, float v, int i, bool valid) {
  const bool take = valid & argmax_better(v, i, bv, bi);
  bv = take ? v : bv;
  bi = take ? i : bi;
}

// ------------------------------------------------------------------ reciprocal -------
// 1.0f / b, correctly rounded, from the hardware reciprocal: v_rcp_f32 is faithful (one of
// the two floats bracketing 1/b) for normal b with a normal reciprocal, and one FMA correction
// step then rounds to nearest except when the mantissa of b is all ones and the rcp result is
// the lower neighbour (r2 then sits on a power of two; the correct result is one ulp above,
// and both candidates already differ from that power only in the last bit).  Checked against
// IEEE division for every mantissa of every exponent in [2^-126, 2^126) (mvsd_selftest).
// Outside that range (and for NaN / inf / negative b) the IEEE division is used.
__device__ inline float recip_rn(float b) {
  float r = __builtin_amdgcn_rcpf(b);
  r = fmaf(fmaf(-b, r, 1.0f), r, r);
  r = (__float_as_uint(b) & 0x7fffffu) == 0x7fffffu ? __uint_as_float(__float_as_uint(r) | 1u) : r;
  if (!(b >= 0x1p-126f && b < 0x1p126f)) r = 1.0f / b;
  return r;
}

// ------------------------------------------------------------------ division ---------
// x / t correctly rounded for a fixed divisor t > 0.  For t in [2^-20, 2^20] and |x| in
// [2^-100, 2^100], Markstein's correction: with rt = 1 / t correctly rounded, q0 = x * rt is
// within an ulp of x / t, the FMA residual x - q0 * t is exact (its granularity, 2^(e_x - 46)
// or coarser, stays above the smallest subnormal), and q0 + residual * rt rounds to the IEEE
// quotient.  Every other x (zeros, subnormals, huge values, inf, NaN) and every other t take
// the IEEE divide.  Checked against the IEEE divide for every float x at a set of divisors
// (mvsd_selftest).
struct Divider {
  float t, rt, lo, hi;
};

__device__ inline Divider make_divider(float t) {
  Divider d;
  d.t = t;
  d.rt = 1.0f / t;
  const bool ok = t >= 0x1p-20f && t <= 0x1p20f;
  d.lo = ok ? 0x1p-100f : INFINITY;
  d.hi = ok ? 0x1p100f : 0.f;
  return d;
}

__device__ inline float divide(const Divider& d, float x) {
  const float ax = fabsf(x);
  if (ax >= d.lo && ax <= d.hi) {
    const float q0 = x * d.rt;
    return fmaf(fmaf(-q0, d.t, x), d.rt, q0);
  }
  return x / d.t;
}

// ------------------------------------------------------------------ wave reductions --
// Cross-lane steps use DPP row permutations (VALU, no LDS round trip): quad swaps for lane
// xor 1 and 2, then the half-row and row mirrors, after which every lane of a 16-lane row
// holds the row's result; the four row results are combined from v_readlane in a fixed
// order, so every lane gets the same, deterministic value.  All combining operations here
// are commutative.

constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within each row

template <int CTRL>
__device__ inline int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ inline float dpp_f32(float v) {
  return __int_as_float(dpp_i32<CTRL>(__float_as_int(v)));
}
__device__ inline float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppMirror>(v));
  return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)),
               fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

__device__ inline float wave_sum(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppHalfMirror>(v);
  v += dpp_f32<kDppMirror>(v);
  return (readlane_f32(v, 0) + readlane_f32(v, 16)) + (readlane_f32(v, 32) + readlane_f32(v, 48));
}

template <int CTRL>
__device__ inline void argmax_step(float& v, int& i) {
  argmax_update(v, i, dpp_f32<CTRL>(v), dpp_i32<CTRL>(i), true);
}

__device__ inline void wave_argmax(float& v, int& i) {
  argmax_step<kDppXor1>(v, i);
  argmax_step<kDppXor2>(v, i);
  argmax_step<kDppHalfMirror>(v, i);
  argmax_step<kDppMirror>(v, i);
  float bv = readlane_f32(v, 0);
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r)
    argmax_update(bv, bi, readlane_f32(v, 16 * r), __builtin_amdgcn_readlane(i, 16 * r), true);
  v = bv;
  i = bi;
}

__device__ inline int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ inline int wave_id() { return threadIdx.x / kWave; }

// ------------------------------------------------------------------ block reductions -
// Reduce N independent values across a block of NW wavefronts (default: the 256-thread
// block).  `scratch` must hold NW * N entries; every thread receives the results.  Two
// barriers.

template <int N, int NW = kWaves>
__device__ inline void block_max(float (&v)[N], float* scratch) {
#pragma unroll
  for (int g = 0; g < N; ++g) v[g] = wave_max(v[g]);
  if (lane_id() == 0) {
#pragma unroll
    for (int g = 0; g < N; ++g) scratch[g * NW + wave_id()] = v[g];
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < N; ++g) {
    float m = scratch[g * NW];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, scratch[g * NW + w]);
    v[g] = m;
  }
  __syncthreads();
}

template <int N, int NW = kWaves>
__device__ inline void block_sum(float (&v)[N], float* scratch) {
#pragma unroll
  for (int g = 0; g < N; ++g) v[g] = wave_sum(v[g]);
  if (lane_id() == 0) {
#pragma unroll
    for (int g = 0; g < N; ++g) scratch[g * NW + wave_id()] = v[g];
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < N; ++g) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += scratch[g * NW + w];
    v[g] = s;
  }
  __syncthreads();
}

template <int N, int NW = kWaves>
__device__ inline void block_argmax(float (&v)[N], int (&i)[N], float* sv, int* si) {
#pragma unroll
  for (int g = 0; g < N; ++g) wave_argmax(v[g], i[g]);
  if (lane_id() == 0) {
#pragma unroll
    for (int g = 0; g < N; ++g) {
      sv[g * NW + wave_id()] = v[g];
      si[g * NW + wave_id()] = i[g];
    }
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < N; ++g) {
    float bv = sv[g * NW];
    int bi = si[g * NW];
#pragma unroll
    for (int w = 1; w < NW; ++w) argmax_update(bv, bi, sv[g * NW + w], si[g * NW + w], true);
    v[g] = bv;
    i[g] = bi;
  }
  __syncthreads();
}

// ------------------------------------------------------------------ argmax keys ------
// An (value, index) pair as one 64-bit key whose unsigned maximum is the argmax under the
// rule above: the high word orders floats (NaN mapped above +inf), the low word is
// 0xffffffff - index so that equal values prefer the lower index.  Key 0 is below every
// real pair (the smallest float, -inf, maps to 0x007fffff).

// Order-preserving key of a float: -0.0 and +0.0 share a key (they compare equal), NaN is
// above every number.
__device__ inline uint32_t ordered_bits(float x) {
  const uint32_t b = __float_as_uint(x);
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (x != x) ? 0xffffffffu : (x == 0.f ? 0x80000000u : o);
}

__device__ inline uint64_t argmax_key(float v, int idx) {
  return ((uint64_t)ordered_bits(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}

__device__ inline int key_index(uint64_t key) { return (int)(0xffffffffu - (uint32_t)key); }

template <int CTRL>
__device__ inline uint64_t dpp_u64(uint64_t k) {
  const uint32_t lo = (uint32_t)dpp_i32<CTRL>((int)(uint32_t)k);
  const uint32_t hi = (uint32_t)dpp_i32<CTRL>((int)(uint32_t)(k >> 32));
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint64_t readlane_u64(uint64_t k, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ inline uint64_t wave_max_u64(uint64_t k) {
  k = umax64(k, dpp_u64<kDppXor1>(k));
  k = umax64(k, dpp_u64<kDppXor2>(k));
  k = umax64(k, dpp_u64<kDppHalfMirror>(k));
  k = umax64(k, dpp_u64<kDppMirror>(k));
  return umax64(umax64(readlane_u64(k, 0), readlane_u64(k, 16)),
                umax64(readlane_u64(k, 32), readlane_u64(k, 48)));
}

// Per-row maximum of N keys over a block of NW wavefronts; only thread g (< N) receives row
// g's result (returned; other threads get 0).  `scratch` holds N * NW keys.  One barrier.
template <int N, int NW>
__device__ inline uint64_t block_max_key_to_row_thread(const uint64_t (&k)[N], uint64_t* scratch) {
#pragma unroll
  for (int g = 0; g < N; ++g) {
    const uint64_t w = wave_max_u64(k[g]);
    if (lane_id() == 0) scratch[g * NW + wave_id()] = w;
  }
  __syncthreads();
  uint64_t best = 0;
  const int t = threadIdx.x;
  if (t < N) {
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint64_t v = scratch[t * NW + w];
      best = v > best ? v : best;
    }
  }
  return best;
}

// Per-row sums of N values; only thread g (< N) receives row g's sum.  One barrier.
template <int N, int NW>
__device__ inline float block_sum_to_row_thread(const float (&v)[N], float* scratch) {
#pragma unroll
  for (int g = 0; g < N; ++g) {
    const float w = wave_sum(v[g]);
    if (lane_id() == 0) scratch[g * NW + wave_id()] = w;
  }
  __syncthreads();
  float s = 0.f;
  const int t = threadIdx.x;
  if (t < N) {
#pragma unroll
    for (int w = 0; w < NW; ++w) s += scratch[t * NW + w];
  }
  return s;
}

// ------------------------------------------------------------------ atomics ----------
// Agent-scope acquire/release on plain device memory; see the AMDGPU memory model for
// gfx942/gfx950 (release writes back L2, acquire invalidates stale L1/L2 lines), which
// makes partial results written by a workgroup on one XCD visible to another XCD.

__device__ inline int atomic_add_release(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int atomic_add_acq_rel(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int atomic_add_relaxed(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int atomic_load_acquire(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int atomic_load_relaxed(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void atomic_store_relaxed(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ partial slots ----
// 64-bit self-describing slots exchanged between workgroups with relaxed agent-scope atomics
// (coherent across XCDs without any fence, hence without L2 write-back or invalidation).  An
// empty slot holds 0 and no written slot can be 0, so a reader polls the data itself.

__device__ inline void slot_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t slot_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// (chunk max, chunk sumexp).  Unmasked, s >= 1 whenever m is finite and m = -inf has a
// non-zero bit pattern.  Masked, the max covers every entry but the sum only the kept ones, so
// a chunk whose entries are all masked and whose max is +0.0 has the pair (+0, +0): its sum is
// then stored as -0.0, which adds nothing where the sums are combined, so that a written stats
// slot is never 0.  NaN maxima are stored canonically.
__device__ inline uint64_t pack_stats(float m, float s) {
  const uint32_t mb = (m != m) ? 0x7fc00000u : __float_as_uint(m);
  uint32_t sb = __float_as_uint(s);
  if ((mb | sb) == 0) sb = 0x80000000u;
  return (uint64_t)mb | ((uint64_t)sb << 32);
}
__device__ inline float2 unpack_stats(uint64_t v) {
  return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}

// (value, index): the index is stored + 1 so that a written slot is never 0.
__device__ inline uint64_t pack_arg(float v, int idx) {
  return (uint64_t)__float_as_uint(v) | ((uint64_t)(uint32_t)(idx + 1) << 32);
}
__device__ inline void unpack_arg(uint64_t s, float& v, int& idx) {
  v = __uint_as_float((uint32_t)s);
  idx = (int)(uint32_t)(s >> 32) - 1;
}

// One wavefront waits until the n slots at `slots` are all written.  Returns false when the
// bounded spin runs out (the caller flags the error and carries on, so every wave exits).
// Wait until slots[0..n) are all written.  Gives up (returns false) after spin_limit polls,
// or early once the sticky failure flag *abort is set by any wave, so that one wait that
// cannot complete ends every other wait quickly instead of each running to its own limit.
__device__ inline bool wave_wait_slots(const uint64_t* slots, int n, int spin_limit, const int* abort) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int spins = 0;; ++spins) {
    int ready = 1;
    for (int c = lane; c < n; c += kWave) ready &= slot_load(slots + c) != 0;
    if (__all(ready)) return true;
    if (spins >= spin_limit) return false;
    if ((spins & 255) == 255 && atomic_load_relaxed(abort) != 0) return false;
    __builtin_amdgcn_s_sleep(1);
  }
}

}  // namespace mvsd
