// Sampling constraints of the verify rows (top-k / top-p per request) as per-row thresholds,
// for the verify kernel to apply while it streams the raw rows.
//
// Reference: apply_sampling_constraints (minivllm/sample/rejection_sampler.py:537-571) divides
// the gathered fp32 verify rows by the request temperature (greedy T = 0 -> 1; nothing at all
// when every request is greedy) and calls apply_top_k_top_p
// (minivllm/sample/ops/topk_topp_sampler.py:48-79): ascending sort; top-k masks the values
// below the k-th largest (:61-69); top-p masks the ascending prefix whose cumulative softmax
// mass is <= 1 - p and never the last entry (:71-77).  Equal values keep index order, as a
// stable sort keeps them.
//
// With v = fl(x / T), the masked entries of a row are a prefix of the order (v, index), so the
// first kept entry (v_f, i_f) describes them: entry i is masked iff v < v_f, or v == v_f and
// i < i_f.  Division by T > 0 is monotone, hence v < v_f iff x < A with
// A = min{x : fl(x / T) >= v_f}, and v <= v_f iff x < B with B = min{x : fl(x / T) > v_f}:
//     masked(x, i) = x < A || (x < B && i <= J),   J = i_f - 1,
// a test on the raw values that needs no division.  A row with only top-k has B = -inf.
//
// Per row (one 512-thread workgroup):
//   pass 1   the row maximum and every thread's own maximum;
//   top-k    for k <= 512 the k-th largest thread maximum bounds the k-th largest entry from
//            below, so the entries at or above it (about k of them) are gathered into LDS,
//            sorted by (v, index), and read off; otherwise (or if too many tie) a bisection
//            over the value keys counts entries per pass;
//   top-p    masses floor(2^40 * exp(v - v_max)) in 64-bit fixed point, so sums are exact and
//            independent of order.  With a top-k candidate set the prefix is found in LDS;
//            otherwise a histogram over 4096 logarithmic mass bins (96 per factor of two)
//            locates the bin of the first kept entry, whose entries are gathered, sorted and
//            scanned; an overfull bin falls back to bisection over (v, index).
// The limit floor((1 - p) * S) is computed exactly in integers.
#include <float.h>
#include <string.h>

#include "mvsd_device.h"
#include "verify.h"

namespace mvsd {
namespace {

#ifndef MVSD_CONSTRAINT_BATCH
#define MVSD_CONSTRAINT_BATCH 3   // 16-byte vectors per thread per batch of a row walk
#endif

#ifndef MVSD_CONSTRAINT_THREADS
#define MVSD_CONSTRAINT_THREADS 512
#endif
#ifndef MVSD_CONSTRAINT_CAP
#define MVSD_CONSTRAINT_CAP 4096
#endif

constexpr int kCT = MVSD_CONSTRAINT_THREADS;  // threads per row
constexpr int kCW = kCT / kWave;
constexpr int kCap = MVSD_CONSTRAINT_CAP;     // candidates gathered in LDS
constexpr int kBins = 4096;              // top-p histogram bins
constexpr float kBinScale = 96.f * 1.44269504088896340736f;  // bins per unit of v_max - v
constexpr float kLog2e = 1.44269504088896340736f;
constexpr uint32_t kNanKey = 0xffffffffu;

struct ConstraintSmem {
  union {
    unsigned long long hist[kBins];
    unsigned long long cand[kCap];     // ordered_bits(v) << 32 | index, sorted ascending
  } u;
  unsigned long long part[kCT];        // scan partials
  unsigned long long red[kCW];
  unsigned long long bcast[4];
  int count;
};

// Inverse of ordered_bits (the shared zero key gives +0; unused keys map monotonically).
__device__ inline float key_float(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

template <int DT>
__device__ inline float vec_elem(const u32x4& r, int j);
template <>
__device__ inline float vec_elem<MVSD_F32>(const u32x4& r, int j) {
  return __uint_as_float(r[j]);
}
template <>
__device__ inline float vec_elem<MVSD_BF16>(const u32x4& r, int j) {
  const uint32_t w = r[j / 2];
  return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
}
template <>
__device__ inline float vec_elem<MVSD_F16>(const u32x4& r, int j) {
  const uint32_t w = r[j / 2];
  return static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? (w >> 16) : w)));
}

// Calls g(vector index, 16-byte vector) for every vector of a row of nvec vectors: full
// batches of U vectors per thread, two batches in flight (each iteration issues one buffer's
// next loads before consuming the other, and the loads of a full batch are unconditional, the
// last one clamped to the last full batch, so each wait covers exactly one batch), then the
// remaining vectors one per thread and step.
template <typename G>
__device__ inline void for_each_vector(const u32x4* xv, int nvec, G&& g) {
  constexpr int U = MVSD_CONSTRAINT_BATCH;
  constexpr int step = U * kCT;
  const int tid = threadIdx.x;
  const int nfull = nvec / step;
  auto load = [&](u32x4 (&buf)[U], int j) {
    const int base = min(j, nfull - 1) * step + tid;
#pragma unroll
    for (int u = 0; u < U; ++u) buf[u] = xv[base + u * kCT];
  };
  auto consume = [&](const u32x4 (&buf)[U], int j) {
#pragma unroll
    for (int u = 0; u < U; ++u) g(j * step + tid + u * kCT, buf[u]);
  };
  if (nfull > 0) {
    u32x4 a[U], b[U];
    load(a, 0);
    for (int j = 0;;) {
      load(b, j + 1);
      // a compiler barrier: the loads above stay issued ahead of the consumption below
      asm volatile("" ::: "memory");
      consume(a, j);
      if (++j == nfull) break;
      load(a, j + 1);
      asm volatile("" ::: "memory");
      consume(b, j);
      if (++j == nfull) break;
    }
  }
  for (int v = nfull * step + tid; v < nvec; v += kCT) g(v, xv[v]);
}

// Calls f(index, value) for every entry of the row: vector walk for rows that are 16-byte
// aligned with V a multiple of the vector width, a batched scalar walk otherwise.
template <int DT, typename F>
__device__ inline void for_each_entry(const typename Elem<DT>::storage* __restrict__ x, int V,
                                      bool aligned, F&& f) {
  constexpr int VEC = Elem<DT>::kVec;
  if (aligned && V % VEC == 0) {
    for_each_vector(reinterpret_cast<const u32x4*>(x), V / VEC, [&](int vi, const u32x4& r) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) f(vi * VEC + j, vec_elem<DT>(r, j));
    });
  } else {
    constexpr int US = 8;
    for (int i0 = threadIdx.x; i0 < V; i0 += US * kCT) {
      typename Elem<DT>::storage e[US];
#pragma unroll
      for (int u = 0; u < US; ++u) e[u] = x[min(i0 + u * kCT, V - 1)];
#pragma unroll
      for (int u = 0; u < US; ++u)
        if (i0 + u * kCT < V) f(i0 + u * kCT, Elem<DT>::cvt(e[u]));
    }
  }
}

// Calls f(i0, v, n) for every group of consecutive entries: v[0, n) are entries i0, i0 + 1,
// ...; a group is one 16-byte vector (n = VEC) on the vector walk and one entry (n = 1) on the
// scalar walk.  Per-group work lets a pass test a whole vector with one branch.
template <int DT, typename F>
__device__ inline void for_each_group(const typename Elem<DT>::storage* __restrict__ x, int V,
                                      bool aligned, F&& f) {
  constexpr int VEC = Elem<DT>::kVec;
  if (aligned && V % VEC == 0) {
    for_each_vector(reinterpret_cast<const u32x4*>(x), V / VEC, [&](int vi, const u32x4& r) {
      float v[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = vec_elem<DT>(r, j);
      f(vi * VEC, v, VEC);
    });
  } else {
    for_each_entry<DT>(x, V, aligned, [&](int i, float e) {
      float v[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = e;
      f(i, v, 1);
    });
  }
}

// q[j] = x[j] / T for a group; one branch per group to the IEEE divide when any entry is
// outside the range of the corrected division.
template <int N>
__device__ inline void divide_group(const Divider& d, const float (&x)[N], float (&q)[N]) {
  bool ok = true;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float ax = fabsf(x[j]);
    ok &= (ax >= d.lo) & (ax <= d.hi);
    const float q0 = x[j] * d.rt;
    q[j] = fmaf(fmaf(-q0, d.t, x[j]), d.rt, q0);
  }
  if (!ok) {
#pragma unroll
    for (int j = 0; j < N; ++j) q[j] = x[j] / d.t;
  }
}

__device__ inline unsigned long long block_sum_u64(unsigned long long v, ConstraintSmem& sm) {
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  if (lane_id() == 0) sm.red[wave_id()] = v;
  __syncthreads();
  unsigned long long s = 0;
  for (int w = 0; w < kCW; ++w) s += sm.red[w];
  __syncthreads();
  return s;
}

__device__ inline uint32_t block_max_u32(uint32_t v, ConstraintSmem& sm) {
  for (int off = kWave / 2; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off));
  if (lane_id() == 0) sm.red[wave_id()] = v;
  __syncthreads();
  uint32_t m = 0;
  for (int w = 0; w < kCW; ++w) m = max(m, (uint32_t)sm.red[w]);
  __syncthreads();
  return m;
}

// Inclusive scan of one value per thread in thread order.
__device__ inline unsigned long long block_scan_u64(unsigned long long v, ConstraintSmem& sm) {
  const int t = threadIdx.x;
  sm.part[t] = v;
  __syncthreads();
  for (int off = 1; off < kCT; off <<= 1) {
    const unsigned long long add = t >= off ? sm.part[t - off] : 0ull;
    __syncthreads();
    sm.part[t] += add;
    __syncthreads();
  }
  const unsigned long long r = sm.part[t];
  __syncthreads();
  return r;
}

// exp(-d) for d = v_max - v >= 0 (or +inf), in [0, 1].
__device__ inline float mass_exp(float d) { return __builtin_amdgcn_exp2f(-d * kLog2e); }

// floor(2^40 * e): the 64-bit fixed-point mass.
__device__ inline unsigned long long mass_from_e(float e) {
  const float h = e * 256.f;  // e * 2^8, exact
  const float hi = floorf(h);
  const uint32_t lo = (uint32_t)((h - hi) * 4294967296.f);  // exact fraction * 2^32 < 2^32
  return ((unsigned long long)(uint32_t)hi << 32) | lo;
}

// Histogram bin of d = v_max - v: 96 bins per factor of two of mass, bin 0 at the maximum,
// clamped to the last bin past d = 29.6 (masses there are below 2^-40 of the maximum's, 0 in
// fixed point).  A non-decreasing function of d, computed with correctly rounded operations,
// so the entries of one bin are an interval of v, and of x.
__device__ inline int mass_bin(float d) {
  const float y = d * kBinScale;
  return y < (float)(kBins - 1) ? (y > 0.f ? (int)y : 0) : kBins - 1;
}

__device__ inline unsigned long long mass_of(float d) { return mass_from_e(mass_exp(d)); }

// floor(t * S) for fp32 t in (0, 1] and S < 2^64, exactly (t = mant * 2^(e - 24)).
__device__ inline unsigned long long scaled_floor(float t, unsigned long long S) {
  int e;
  const float fr = frexpf(t, &e);
  const unsigned long long mant = (unsigned long long)(fr * 16777216.0f);
  const int sh = 24 - e;
  const unsigned long long lo = mant * S;
  const unsigned long long hi = __umul64hi(mant, S);
  return sh >= 64 ? (hi >> (sh - 64)) : ((hi << (64 - sh)) | (lo >> sh));
}

// Smallest non-NaN float x with fl(x / T) >= v (v not NaN); monotone bisection over keys.
__device__ inline float min_x_reaching(float v, float T) {
  uint32_t lo = ordered_bits(-INFINITY), hi = ordered_bits(INFINITY);  // pred(hi) holds
  if (key_float(lo) / T >= v) return -INFINITY;
  while (hi - lo > 1) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (key_float(mid) / T >= v) hi = mid;
    else lo = mid;
  }
  return key_float(hi);
}

// Next float above v in the order where -0 == +0 (v finite).
__device__ inline float next_up(float v) {
  return v == 0.f ? __uint_as_float(1u) : key_float(ordered_bits(v) + 1u);
}

// Appends key to the LDS candidate list where pred holds (one LDS atomic per wave).
__device__ inline void append(bool pred, unsigned long long key, ConstraintSmem& sm) {
  const unsigned long long mask = __ballot(pred);
  if (mask == 0) return;
  const int leader = __ffsll((long long)mask) - 1;
  int base = 0;
  if (lane_id() == leader) base = atomicAdd(&sm.count, __popcll(mask));
  base = __shfl(base, leader);
  if (pred) {
    const int pos = base + __popcll(mask & ((1ull << lane_id()) - 1ull));
    if (pos < kCap) sm.u.cand[pos] = key;
  }
}

// Appends the keys of this lane's flagged entries (c[j]: key(j)) to the LDS candidate list:
// per-lane positions from the wave's ballots, one LDS atomic per wave.  Safe with inactive
// lanes (ballots count active lanes only).
__device__ inline int lanes_below(unsigned long long mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

template <int N, typename K>
__device__ inline void append_group(const bool (&c)[N], K&& key, ConstraintSmem& sm) {
  int total = 0, pos = 0;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const unsigned long long m = __ballot(c[j]);
    total += __popcll(m);
    pos += lanes_below(m);
  }
  if (total == 0) return;
  const int leader = __ffsll((long long)__ballot(true)) - 1;
  int base = 0;
  if (lane_id() == leader) base = atomicAdd(&sm.count, total);
  pos += __shfl(base, leader);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    if (c[j]) {
      if (pos < kCap) sm.u.cand[pos] = key(j);
      ++pos;
    }
  }
}

// Smallest non-NaN x whose bin mass_bin(vmax - fl(x / T)) is at most b: the bin of x falls as x
// grows, so the entries of bin b are exactly those with min_x_in_bins(b) <= x <
// min_x_in_bins(b - 1).  Bisection over the ordered keys with the histogram's own arithmetic.
__device__ inline float min_x_in_bins(float vmax, const Divider& dv, int b) {
  if (b < 0) return INFINITY;  // no x has a negative bin; +inf bounds every finite entry
  auto in = [&](uint32_t key) { return mass_bin(vmax - divide(dv, key_float(key))) <= b; };
  uint32_t lo = ordered_bits(-INFINITY), hi = ordered_bits(INFINITY);  // in(hi) holds
  if (in(lo)) return -INFINITY;
  while (hi - lo > 1) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (in(mid)) hi = mid;
    else lo = mid;
  }
  return key_float(hi);
}

// The k-th largest (1 <= k <= kCT) of the block's keys, one per thread (`mine`), by radix
// selection: four rounds of an 8-bit digit, each counting the keys that share the digits found
// so far per next digit (LDS atomics on 256 counters), after which one wave picks the digit
// holding the k-th largest.  Every thread receives the key.  Uses sm.part and sm.bcast.
__device__ inline uint32_t kth_largest_key(uint32_t mine, int k, ConstraintSmem& sm) {
  int* cnt = reinterpret_cast<int*>(sm.part);  // 256 counters
  const int tid = threadIdx.x;
  uint32_t prefix = 0, pmask = 0;
  int need = k;  // rank of the wanted key among the keys matching the prefix
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = tid; b < 256; b += kCT) cnt[b] = 0;
    __syncthreads();
    if ((mine & pmask) == prefix) atomicAdd(&cnt[(mine >> shift) & 255u], 1);
    __syncthreads();
    if (tid < kWave) {
      // lane l holds digits 255 - 4l .. 252 - 4l, the largest first
      int c[4], own = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = cnt[255 - 4 * tid - j];
        own += c[j];
      }
      int incl = own;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int t = __shfl_up(incl, off);
        if (tid >= off) incl += t;
      }
      const int above = incl - own;  // keys with a larger digit than this lane's
      if (above < need && need <= incl) {
        int run = above, j = 0;
        while (run + c[j] < need) run += c[j++];
        sm.bcast[0] = (unsigned long long)(255 - 4 * tid - j);
        sm.bcast[1] = (unsigned long long)(need - run);
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sm.bcast[0] << shift;
    pmask |= 0xffu << shift;
    need = (int)sm.bcast[1];
    __syncthreads();
  }
  return prefix;
}

// Bitonic sort of cand[0, n), ascending; n <= kCap.
__device__ inline void sort_candidates(int n, ConstraintSmem& sm) {
  int N = 1;
  while (N < n) N <<= 1;
  for (int i = n + (int)threadIdx.x; i < N; i += kCT) sm.u.cand[i] = ~0ull;
  __syncthreads();
  for (int size = 2; size <= N; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < N / 2; i += kCT) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const unsigned long long a = sm.u.cand[lo], b = sm.u.cand[hi];
        if ((a > b) == up) {
          sm.u.cand[lo] = b;
          sm.u.cand[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

// First position f in the sorted cand[s, e) where base + (mass of cand[s..f]) > limit, or
// e - 1 when there is none (the last entry is always kept).  mass(key) is a candidate's mass.
template <typename M>
__device__ inline int first_over(int s, int e, unsigned long long base, unsigned long long limit,
                                 ConstraintSmem& sm, M&& mass) {
  const int len = e - s;
  const int per = (len + kCT - 1) / kCT;
  const int b0 = s + (int)threadIdx.x * per, b1 = min(e, b0 + per);
  unsigned long long seg = 0;
  for (int i = b0; i < b1; ++i) seg += mass(sm.u.cand[i]);
  if (threadIdx.x == 0) sm.bcast[0] = (unsigned long long)(e - 1);
  const unsigned long long incl = block_scan_u64(seg, sm);
  unsigned long long run = base + (incl - seg);
  if (run <= limit && limit < base + incl) {
    for (int i = b0; i < b1; ++i) {
      run += mass(sm.u.cand[i]);
      if (run > limit) {
        sm.bcast[0] = (unsigned long long)i;
        break;
      }
    }
  }
  __syncthreads();
  const int f = (int)sm.bcast[0];
  __syncthreads();
  return f;
}

// Request of verify row `row` (the first r with cu[r] > row; -1 past the last request), or the
// row itself when there is no cu (one row per request).
__device__ inline int request_of(const VerifyParams& p, int row) {
  if (!p.cu) return row < p.B ? row : -1;
  if (p.B <= 0 || row >= p.cu[p.B - 1]) return -1;
  int lo = 0, hi = p.B - 1;
  while (lo < hi) {
    const int mid = (lo + hi) / 2;
    if (p.cu[mid] > row) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// How much work the verify rows of request r take in the constraints kernel: 0 none (no
// constraint, or a greedy request with top-k only: see row_thresholds), 1 random with top-p
// (three passes per row), 2 random with top-k only (one pass), 3 greedy with top-p (one pass,
// more when a row's maximum is tied).
__device__ inline int request_class(const VerifyParams& p, int r) {
  if (p.all_greedy) return 0;
  const int64_t kk = p.top_k ? p.top_k[r] : (int64_t)p.V;
  const bool has_k = kk > 0 && kk < p.V;
  const bool has_p = p.top_p && 1.0f - p.top_p[r] > 0.f;
  const bool greedy = p.temperature != nullptr && p.temperature[r] == 0.f;
  if ((!has_k && !has_p) || (greedy && !has_p)) return 0;
  return greedy ? 3 : (has_p ? 1 : 2);
}

// The plan of a masked call (one 1024-thread workgroup, one request per thread at a time):
// the neutral mask for every row of class 0, and the other rows listed by class, as row + 1,
// so that the rows with the most passes start first.  The order inside a class does not
// matter: each row's mask depends on its own row only.
__global__ __launch_bounds__(1024) void constraint_plan_kernel(VerifyParams p) {
  __shared__ int cnt[4], base[4];
  const int tid = threadIdx.x;
  if (tid < 4) cnt[tid] = 0;
  __syncthreads();
  const float4 neutral = make_float4(-INFINITY, -INFINITY, __int_as_float(-1), 0.f);
  // rows past the last request belong to none
  for (int j = max(p.B > 0 ? p.cu[p.B - 1] : 0, 0) + tid; j < p.P; j += 1024) p.masks[j] = neutral;
  for (int r = tid; r < p.B; r += 1024) {
    const int begin = max(r == 0 ? 0 : p.cu[r - 1], 0), end = min(p.cu[r], p.P);
    const int c = request_class(p, r);
    if (c == 0) {
      for (int j = begin; j < end; ++j) p.masks[j] = neutral;
    } else if (end > begin) {
      atomicAdd(&cnt[c], end - begin);
    }
  }
  __syncthreads();
  if (tid == 0) {
    base[1] = 0;
    base[2] = cnt[1];
    base[3] = cnt[1] + cnt[2];
    cnt[1] = cnt[2] = cnt[3] = 0;
  }
  __syncthreads();
  for (int r = tid; r < p.B; r += 1024) {
    const int begin = max(r == 0 ? 0 : p.cu[r - 1], 0), end = min(p.cu[r], p.P);
    const int c = request_class(p, r);
    if (c != 0 && end > begin) {
      const int at = base[c] + atomicAdd(&cnt[c], end - begin);
      for (int j = begin; j < end; ++j) p.order[at + (j - begin)] = j + 1;
    }
  }
}

// Top-p of a greedy row whose maximum is tied (ties >= 2 entries at raw key mkey), without
// top-k.  Only the row's argmax matters, and the temperature is 1, so v = x and the tied
// entries are exactly the entries at the maximum, each of mass mass_of(0) = 2^40.  The masked
// prefix of the order (v, index) reaches them only when the mass below the maximum is at most
// the limit; then it takes every entry below the maximum and the first m tied entries in index
// order, m = floor((limit - below) / 2^40) (at most ties - 1: the last entry is always kept).
// One pass sums the masses; a second gathers the tied entries' indices only when the prefix
// reaches them.  Returns 0 (no mask changes the argmax: the neutral mask), 1 (A, B, J set), or
// -1 (more tied entries than LDS holds: the general path).
template <int DT>
__device__ inline int greedy_tied_top_p(const typename Elem<DT>::storage* __restrict__ x, int V,
                                        bool aligned, const Divider& dv, float T, float t,
                                        uint32_t mkey, unsigned long long ties,
                                        ConstraintSmem& sm, float& A, float& Bv, int& J) {
  constexpr int VEC = Elem<DT>::kVec;
  const float vmax = divide(dv, key_float(mkey));
  if (vmax != vmax || fabsf(vmax) == INFINITY) return 0;
  unsigned long long s = 0;
  for_each_group<DT>(x, V, aligned, [&](int, const float (&v)[VEC], int n) {
    float q[VEC];
    divide_group(dv, v, q);
#pragma unroll
    for (int j = 0; j < VEC; ++j)
      if (j < n) s += mass_of(vmax - q[j]);
  });
  const unsigned long long total = block_sum_u64(s, sm);
  const unsigned long long limit = scaled_floor(fminf(t, 1.f), total);
  constexpr unsigned long long kUnit = 1ull << 40;  // mass_of(0)
  const unsigned long long below = total - ties * kUnit;
  if (limit < below + kUnit) return 0;  // the first maximum is kept
  if (ties > (unsigned long long)kCap) return -1;
  unsigned long long m = (limit - below) / kUnit;
  if (m > ties - 1) m = ties - 1;
  if (threadIdx.x == 0) sm.count = 0;
  __syncthreads();
  for_each_group<DT>(x, V, aligned, [&](int i0, const float (&v)[VEC], int n) {
    bool c[VEC], any = false;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      c[j] = (j < n) && ordered_bits(v[j]) == mkey;
      any |= c[j];
    }
    if (__ballot(any) == 0) return;
#pragma unroll
    for (int j = 0; j < VEC; ++j)
      append(c[j], c[j] ? (((unsigned long long)mkey << 32) | (uint32_t)(i0 + j)) : 0ull, sm);
  });
  __syncthreads();
  const int n = sm.count;  // == ties
  sort_candidates(n, sm);
  const int i_f = (int)(uint32_t)sm.u.cand[min((int)m, n - 1)];
  A = min_x_reaching(vmax, T);
  Bv = min_x_reaching(next_up(vmax), T);
  J = i_f - 1;
  return 1;
}

// The row's mask (A, B, J) from its request's top-k / top-p; false when nothing is masked.
template <int DT>
__device__ __forceinline__ bool row_thresholds(const VerifyParams& p, int row, ConstraintSmem& sm, float& A,
                               float& Bv, int& J) {
  using S = typename Elem<DT>::storage;
  const int tid = threadIdx.x;
  A = -INFINITY;
  Bv = -INFINITY;
  J = -1;
  const int r = request_of(p, row);
  if (p.all_greedy || r < 0) return false;
  const int64_t kk = p.top_k ? p.top_k[r] : (int64_t)p.V;
  const float t = p.top_p ? 1.0f - p.top_p[r] : 0.f;
  const bool has_k = kk > 0 && kk < p.V;
  const bool has_p = t > 0.f;  // p >= 1 keeps every entry of non-zero probability
  if (!has_k && !has_p) return false;
  // A greedy row only needs its argmax (the first maximum, or the first NaN).  Top-k keeps
  // every entry at or above the k-th largest, so it never masks a maximum or a NaN; top-p
  // masks an ascending prefix that never includes the last entry of the order (v, index), so
  // it masks a maximum only when the maximum is tied (a NaN makes every mass NaN and masks
  // nothing).  Such a row gets no mask unless it has top-p and a tied maximum.  (The in-place
  // top-k / top-p of the sampler passes no temperatures: none of its rows is greedy.)
  const bool greedy_row = p.temperature != nullptr && p.temperature[r] == 0.f;
  if (greedy_row && !has_p) return false;
  const float T = req_temperature(p, r);
  const Divider dv = make_divider(T);
  const int V = p.V;
  const S* x = static_cast<const S*>(p.target) + target_row(p, row) * p.target_stride;
  const bool aligned = ((uintptr_t)x % 16) == 0;

  // ---- pass 1: row maximum and per-thread maxima (ordered keys of the raw values); rows with
  // top-k only also keep each thread's four largest keys ----
  const bool k_only = has_k && !has_p && kk <= kCT;
  uint32_t t0 = 0, t1 = 0, t2 = 0, t3 = 0;
  constexpr int VEC = Elem<DT>::kVec;
  if (k_only) {
    // The four largest values in floats (NaN read as -inf and flagged): max / min pairs.  A
    // row with a NaN, which ranks above every number, takes the key-based walk below.
    float f0 = -INFINITY, f1 = -INFINITY, f2 = -INFINITY, f3 = -INFINITY;
    int seen = 0;
    bool nan = false;
    for_each_group<DT>(x, V, aligned, [&](int, const float (&v)[VEC], int n) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        if (j < n) {
          nan |= v[j] != v[j];
          float c = v[j] == v[j] ? v[j] : -INFINITY, m;
          m = fmaxf(f0, c); c = fminf(f0, c); f0 = m;
          m = fmaxf(f1, c); c = fminf(f1, c); f1 = m;
          m = fmaxf(f2, c); c = fminf(f2, c); f2 = m;
          f3 = fmaxf(f3, c);
        }
      }
      seen += n;
    });
    // a slot no entry filled keeps key 0, below every entry's key
    t0 = seen > 0 ? ordered_bits(f0) : 0u;
    t1 = seen > 1 ? ordered_bits(f1) : 0u;
    t2 = seen > 2 ? ordered_bits(f2) : 0u;
    t3 = seen > 3 ? ordered_bits(f3) : 0u;
    if (__syncthreads_or(nan)) {
      t0 = t1 = t2 = t3 = 0;
      for_each_group<DT>(x, V, aligned, [&](int, const float (&v)[VEC], int n) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          if (j < n) {
            uint32_t c = ordered_bits(v[j]), m;
            m = max(t0, c); c = min(t0, c); t0 = m;
            m = max(t1, c); c = min(t1, c); t1 = m;
            m = max(t2, c); c = min(t2, c); t2 = m;
            t3 = max(t3, c);
          }
        }
      });
    }
  } else {
    // The thread maximum in floats, the number of entries equal to it (for the greedy tie
    // test; -0 and +0 compare equal, as their keys do) and a NaN flag (NaN ranks above every
    // number, so the thread's key is then the NaN key).
    float fm = -INFINITY;
    uint32_t ties = 0;
    bool nan = false;
    for_each_group<DT>(x, V, aligned, [&](int, const float (&v)[VEC], int n) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        if (j < n) {
          nan |= v[j] != v[j];
          ties = v[j] > fm ? 1u : ties + (v[j] == fm);
          fm = fmaxf(fm, v[j]);
        }
      }
    });
    t0 = nan ? kNanKey : (ties > 0 ? ordered_bits(fm) : 0u);
    t1 = ties;
  }
  const uint32_t mkey = block_max_u32(t0, sm);
  if (greedy_row) {
    const unsigned long long ties = block_sum_u64(t0 == mkey ? t1 : 0u, sm);
    if (mkey == kNanKey || ties < 2) return false;
    if (!has_k) {
      const int g = greedy_tied_top_p<DT>(x, V, aligned, dv, T, t, mkey, ties, sm, A, Bv, J);
      if (g >= 0) return g == 1;
    }
  }

  // ---- top-k: v_k, the k-th largest v, and the entries with v >= v_k in LDS if they fit ----
  bool cand_ok = false;
  int n = 0, lo_k = 0;
  if (has_k) {
    const int k = (int)kk;
    uint32_t theta = 0;
    if (k <= kCT) {
      // theta: the k-th largest thread maximum; at least k entries are >= theta
      theta = kth_largest_key(t0, k, sm);
      if (tid == 0) sm.count = 0;
      __syncthreads();
    }
    bool k_done = false;
    uint32_t vk_key = 0;
    if (k_only && theta != 0) {
      // Every entry >= theta is among its thread's four largest unless that thread's fourth
      // largest is >= theta too; then the general path below runs instead.
      const int overflow = __syncthreads_or(t3 >= theta);
      if (!overflow) {
        uint32_t* ck = reinterpret_cast<uint32_t*>(sm.u.cand);
        auto put = [&](uint32_t key) {
          const bool c = key >= theta;
          const unsigned long long mask = __ballot(c);
          if (mask == 0) return;
          const int leader = __ffsll((long long)mask) - 1;
          int base = 0;
          if (lane_id() == leader) base = atomicAdd(&sm.count, __popcll(mask));
          base = __shfl(base, leader);
          if (c) ck[base + __popcll(mask & ((1ull << lane_id()) - 1ull))] = key;
        };
        put(t0);
        put(t1);
        put(t2);
        __syncthreads();
        const int nk = sm.count;  // <= 3 * kCT, and >= k
        // the k-th largest key: the entry with k - 1 entries above it (ties by position)
        for (int i = tid; i < nk; i += kCT) {
          const uint32_t mine = ck[i];
          int rank = 0;
          for (int j = 0; j < nk; ++j) {
            const uint32_t o = ck[j];
            rank += (o > mine) | ((o == mine) & (j < i));
          }
          if (rank == k - 1) sm.bcast[1] = mine;
        }
        __syncthreads();
        vk_key = ordered_bits(divide(dv, key_float((uint32_t)sm.bcast[1])));
        k_done = true;
      }
    }
    if (!k_done && k <= kCT) {
      // Gather every entry whose v reaches fl(theta / T) (x >= theta2): that includes every
      // entry with v >= v_k.  (theta = 0: fewer than k threads hold entries; NaN theta:
      // gather everything.)
      const float theta2 = theta == 0 ? -INFINITY
                           : (theta == kNanKey ? NAN : min_x_reaching(divide(dv, key_float(theta)), T));
      if (tid == 0) sm.count = 0;
      __syncthreads();
      for_each_group<DT>(x, V, aligned, [&](int i0, const float (&v)[VEC], int n) {
        bool c[VEC], any = false;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          c[j] = (j < n) && !(v[j] < theta2);
          any |= c[j];
        }
        if (__ballot(any) == 0) return;
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          append(c[j], c[j] ? (((unsigned long long)ordered_bits(divide(dv, v[j])) << 32) | (uint32_t)(i0 + j)) : 0ull, sm);
      });
      __syncthreads();
      n = sm.count;
      cand_ok = n <= kCap;
    }
    if (k_done) {
      // v_k found from the per-thread keys
    } else if (cand_ok) {
      sort_candidates(n, sm);
      vk_key = (uint32_t)(sm.u.cand[max(n - k, 0)] >> 32);
      int below = 0;
      for (int i = tid; i < n; i += kCT) below += (uint32_t)(sm.u.cand[i] >> 32) < vk_key;
      lo_k = (int)block_sum_u64((unsigned long long)below, sm);
    } else {
      // largest raw key K with count(key(x) >= K) >= k, by bisection (one pass per step)
      uint64_t lo = 0, hi = 0x100000000ull;  // count(>= lo) >= k > count(>= hi)
      while (hi - lo > 1) {
        const uint64_t mid = (lo + hi) / 2;
        unsigned long long c = 0;
        for_each_entry<DT>(x, V, aligned, [&](int, float v) { c += ordered_bits(v) >= (uint32_t)mid; });
        if (block_sum_u64(c, sm) >= (unsigned long long)k) lo = mid;
        else hi = mid;
      }
      vk_key = ordered_bits(divide(dv, key_float((uint32_t)lo)));
    }
    // A NaN k-th value compares false with everything: the reference then masks nothing.
    if (vk_key != kNanKey) A = min_x_reaching(key_float(vk_key), T);
  }

  // ---- top-p over the entries top-k keeps (x >= A) ----
  // A NaN or infinite maximum makes every softmax value NaN in the reference, and then no
  // cumulative sum compares <= 1 - p.
  const float vmax = cand_ok ? key_float((uint32_t)(sm.u.cand[max(n - 1, 0)] >> 32))
                             : divide(dv, key_float(mkey));
  if (!has_p || mkey == kNanKey || vmax != vmax || fabsf(vmax) == INFINITY) return A != -INFINITY;
  const float tl = fminf(t, 1.f);
  unsigned long long fkey;  // ordered_bits(v_f) << 32 | i_f of the first kept entry
  if (cand_ok) {
    unsigned long long seg = 0;
    for (int i = lo_k + tid; i < n; i += kCT)
      seg += mass_of(vmax - key_float((uint32_t)(sm.u.cand[i] >> 32)));
    const unsigned long long total = block_sum_u64(seg, sm);
    fkey = sm.u.cand[max(first_over(lo_k, n, 0, scaled_floor(tl, total), sm,
                                    [&](unsigned long long key) {
                                      return mass_of(vmax - key_float((uint32_t)(key >> 32)));
                                    }), 0)];
  } else {
    for (int b = tid; b < kBins; b += kCT) sm.u.hist[b] = 0;
    __syncthreads();
    for_each_group<DT>(x, V, aligned, [&](int, const float (&v)[VEC], int n) {
      float q[VEC];
      divide_group(dv, v, q);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        // one branch per entry: the mass is computed for every entry and cleared for a masked
        // entry or a lane past n
        const float d = vmax - q[j];
        const unsigned long long keep = 0ull - (unsigned long long)(j < n && !(v[j] < A));
        const unsigned long long m = mass_of(d) & keep;
        if (m) atomicAdd(&sm.u.hist[mass_bin(d)], m);
      }
    });
    __syncthreads();
    // Bins run from large v (bin 0) to small v, so the mass below a bin is a suffix sum.
    // Thread t owns bins [per t, per (t + 1)); the scan runs over reversed thread order.
    constexpr int per = kBins / kCT;
    unsigned long long s4 = 0;
    for (int j = 0; j < per; ++j) s4 += sm.u.hist[tid * per + j];
    const int rt = kCT - 1 - tid;
    sm.part[rt] = s4;
    __syncthreads();
    for (int off = 1; off < kCT; off <<= 1) {
      const unsigned long long add = rt >= off ? sm.part[rt - off] : 0ull;
      __syncthreads();
      sm.part[rt] += add;
      __syncthreads();
    }
    const unsigned long long incl = sm.part[rt];  // mass of bins >= per t
    const unsigned long long total = sm.part[kCT - 1];
    if (tid == 0) {
      sm.bcast[2] = 0;
      sm.bcast[3] = 0;
    }
    __syncthreads();
    const unsigned long long limit = scaled_floor(tl, total);
    if (limit >= total) {
      // every entry but the last of the order (v, index) is masked
      unsigned long long best = 0;
      for_each_entry<DT>(x, V, aligned, [&](int i, float v) {
        if (!(v < A)) {
          const unsigned long long key = ((unsigned long long)ordered_bits(divide(dv, v)) << 32) | (uint32_t)i;
          best = key > best ? key : best;
        }
      });
      best = wave_max_u64(best);
      if (lane_id() == 0) sm.red[wave_id()] = best;
      __syncthreads();
      for (int w = 0; w < kCW; ++w) best = sm.red[w] > best ? sm.red[w] : best;
      __syncthreads();
      fkey = best;
    } else {
      if (tid == 0) sm.count = 0;
      unsigned long long run = incl - s4;  // mass of bins >= per (t + 1)
      if (run <= limit && limit < incl) {
        for (int j = per - 1; j >= 0; --j) {
          const unsigned long long h = sm.u.hist[tid * per + j];
          if (run + h > limit) {
            sm.bcast[2] = (unsigned long long)(tid * per + j);
            sm.bcast[3] = run;
            break;
          }
          run += h;
        }
      }
      __syncthreads();
      const int bin = (int)sm.bcast[2];
      const unsigned long long base = sm.bcast[3];  // mass below the bin
      // the bin's entries as an interval of raw values (no divide or exp per entry), kept by
      // top-k too (x >= A)
      const float blo = fmaxf(min_x_in_bins(vmax, dv, bin), A);
      const float bhi = min_x_in_bins(vmax, dv, bin - 1);
      for_each_group<DT>(x, V, aligned, [&](int i0, const float (&v)[VEC], int n) {
        bool c[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) c[j] = (j < n) && v[j] >= blo && v[j] < bhi;
        append_group(c, [&](int j) {
          return ((unsigned long long)ordered_bits(divide(dv, v[j])) << 32) | (uint32_t)(i0 + j);
        }, sm);
      });
      __syncthreads();
      const int nb = sm.count;
      if (nb <= kCap) {
        sort_candidates(nb, sm);
        fkey = sm.u.cand[max(first_over(0, nb, base, limit, sm, [&](unsigned long long key) {
                               return mass_of(vmax - key_float((uint32_t)(key >> 32)));
                             }), 0)];
      } else {
        // Too many entries in one bin (long runs of equal values): bisection over the value
        // keys, then over the indices within the value, with exact sums per pass.
        const unsigned long long rem = limit - base;
        int64_t klo = -1, khi = 0xffffffffll;  // cum(klo) <= rem < cum(khi)
        unsigned long long cum_lo = 0;
        while (khi - klo > 1) {
          const int64_t mid = (klo + khi) / 2;
          unsigned long long c = 0;
          for_each_entry<DT>(x, V, aligned, [&](int, float v) {
            const float q = divide(dv, v);
            const float d = vmax - q;
            if (!(v < A) && mass_bin(d) == bin && ordered_bits(q) <= (uint32_t)mid) c += mass_of(d);
          });
          const unsigned long long cm = block_sum_u64(c, sm);
          if (cm > rem) {
            khi = mid;
          } else {
            klo = mid;
            cum_lo = cm;
          }
        }
        const uint32_t f_key = (uint32_t)khi;
        const unsigned long long mu = mass_of(vmax - key_float(f_key));
        const unsigned long long j = mu ? (rem - cum_lo) / mu : 0;  // entries of v_f masked
        int ilo = -1, ihi = V - 1;  // count(v_f, index <= ilo) <= j < count(v_f, index <= ihi)
        while (ihi - ilo > 1) {
          const int mid = (ilo + ihi) / 2;
          unsigned long long c = 0;
          for_each_entry<DT>(x, V, aligned, [&](int i, float v) {
            c += (i <= mid) & !(v < A) & (ordered_bits(divide(dv, v)) == f_key);
          });
          if (block_sum_u64(c, sm) > j) ihi = mid;
          else ilo = mid;
        }
        fkey = ((unsigned long long)f_key << 32) | (uint32_t)ihi;
      }
    }
  }
  const float vf = key_float((uint32_t)(fkey >> 32));
  A = min_x_reaching(vf, T);
  Bv = min_x_reaching(next_up(vf), T);
  J = (int)(uint32_t)fkey - 1;
  return true;
}

// WRITE = false: one row mask per verify row into p.masks.  WRITE = true (fp32 rows, no
// temperature): the masked entries of each row are set to -inf in place.
template <int DT, bool WRITE>
__global__ __launch_bounds__(kCT) void constraints_kernel(VerifyParams p) {
  __shared__ ConstraintSmem sm;
  __shared__ int s_row;
  int row = blockIdx.x;
  if (p.order) {
    // take this workgroup's entry of the plan, and clear it for the next call
    if (threadIdx.x == 0) {
      s_row = p.order[blockIdx.x] - 1;
      p.order[blockIdx.x] = 0;
    }
    __syncthreads();
    row = s_row;
    if (row < 0) return;
  }
  float A, Bv;
  int J;
  const bool any = row_thresholds<DT>(p, row, sm, A, Bv, J);
  if constexpr (!WRITE) {
    if (threadIdx.x == 0) p.masks[row] = make_float4(A, Bv, __int_as_float(J), 0.f);
  } else {
    if (!any) return;
    float* x = const_cast<float*>(static_cast<const float*>(p.target)) + target_row(p, row) * p.target_stride;
    const float4 m = make_float4(A, Bv, __int_as_float(J), 0.f);
    const int V = p.V;
    if (((uintptr_t)x % 16) == 0 && V % 4 == 0) {
      u32x4* xv = reinterpret_cast<u32x4*>(x);
      for_each_vector(xv, V / 4, [&](int vi, u32x4 r) {
        bool any_masked = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = __uint_as_float(r[j]);
          if (row_masked(m, v, vi * 4 + j) && v != -INFINITY) {
            r[j] = __float_as_uint(-INFINITY);
            any_masked = true;
          }
        }
        if (any_masked) xv[vi] = r;
      });
    } else {
      for (int i = threadIdx.x; i < V; i += kCT) {
        const float v = x[i];
        if (row_masked(m, v, i) && v != -INFINITY) x[i] = -INFINITY;
      }
    }
  }
}

}  // namespace

hipError_t launch_constraints(const VerifyParams& params, int target_dtype, hipStream_t stream) {
  if (params.P == 0) return hipSuccess;
  if (params.order)
    hipLaunchKernelGGL(constraint_plan_kernel, dim3(1), dim3(1024), 0, stream, params);
  const dim3 grid((unsigned)params.P), block(kCT);
  switch (target_dtype) {
    case MVSD_F32: hipLaunchKernelGGL((constraints_kernel<MVSD_F32, false>), grid, block, 0, stream, params); break;
    case MVSD_BF16: hipLaunchKernelGGL((constraints_kernel<MVSD_BF16, false>), grid, block, 0, stream, params); break;
    case MVSD_F16: hipLaunchKernelGGL((constraints_kernel<MVSD_F16, false>), grid, block, 0, stream, params); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_topk_topp(float* logits, int64_t stride, const int64_t* top_k, const float* top_p,
                            int64_t num_rows, int64_t vocab_size, hipStream_t stream) {
  if (num_rows == 0) return hipSuccess;
  VerifyParams p;
  memset(&p, 0, sizeof(p));
  p.target = logits;
  p.target_stride = stride;
  p.target_num_rows = num_rows;
  p.B = (int)num_rows;
  p.P = (int)num_rows;
  p.V = (int)vocab_size;
  p.top_k = top_k;
  p.top_p = top_p;
  hipLaunchKernelGGL((constraints_kernel<MVSD_F32, true>), dim3((unsigned)num_rows), dim3(kCT), 0,
                     stream, p);
  return hipGetLastError();
}

}  // namespace mvsd
