// Top-k / top-p masking of fp32 logits rows, in place, without sorting.
//
// Reference: apply_top_k_top_p, minivllm/sample/ops/topk_topp_sampler.py:48-79 — ascending
// sort; top-k masks values < the k-th largest (:61-69); top-p masks the ascending prefix whose
// cumulative softmax mass is <= 1 - p, never the largest entry (:71-77); scatter back (:79).
//
// Here, per row (one 512-thread workgroup):
//   * top-k: radix select of the k-th largest order-preserving 32-bit key, three digit passes
//     (11, 11, 10 bits) with LDS count histograms;
//   * top-p: the same digit passes over cumulative MASS from the smallest key up find, exactly,
//     the entry where the cumulative mass first exceeds (1 - p) * S.  Masses e = exp(x - max)
//     are summed as 2^40 fixed-point integers (deterministic, independent of summation order)
//     and floor((1 - p) * S) is computed exactly in integers.  Equal values are ordered by
//     index, as a stable sort orders them; when the crossing falls inside a run of equal
//     values, a radix select over their indices finds the last masked one;
//   * one write pass sets masked entries to -inf.
// Entries masked by top-k carry zero mass, as their -inf does in the reference.
#include "mvsd_device.h"
#include "topk.h"

namespace mvsd {
namespace {

constexpr int kTT = 512;          // threads per row
constexpr int kTW = kTT / kWave;  // wavefronts per row
constexpr int kMaxBins = 2048;    // 11-bit digits
constexpr double kMassScale = 1099511627776.0;  // 2^40

// digit levels of a 32-bit key: bits [31:21], [20:10], [9:0]
__device__ inline int digit_shift(int lv) { return lv == 0 ? 21 : (lv == 1 ? 10 : 0); }
__device__ inline int digit_width(int lv) { return lv == 2 ? 10 : 11; }

// Inverse of ordered_bits for non-NaN keys.
__device__ inline float key_value(uint32_t key) {
  const uint32_t b = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
  return __uint_as_float(b);
}

__device__ inline unsigned long long mass_of(float v, float row_max) {
  return (unsigned long long)((double)expf(v - row_max) * kMassScale);
}

struct TopkSmem {
  union {
    uint32_t cnt[kMaxBins];
    unsigned long long mass[kMaxBins];
  } h;
  unsigned long long part[kTT];
  unsigned long long red[kTW];
  unsigned long long result[4];
};

// Calls f(index, value) for every element of the row; 16-byte loads where aligned.
template <typename F>
__device__ inline void for_each(const float* __restrict__ x, int V, bool aligned, F&& f) {
  for (int i = threadIdx.x * 4; i < V; i += kTT * 4) {
    if (aligned && i + 4 <= V) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) f(i + j, __uint_as_float(v[j]));
    } else {
      for (int j = 0; j < 4 && i + j < V; ++j) f(i + j, x[i + j]);
    }
  }
}

// Inclusive scan of one value per thread, in thread order (ascending) or reverse order.
__device__ inline unsigned long long block_scan(unsigned long long v, bool ascending,
                                                TopkSmem& sm) {
  const int pos = ascending ? (int)threadIdx.x : kTT - 1 - (int)threadIdx.x;
  sm.part[pos] = v;
  __syncthreads();
  for (int off = 1; off < kTT; off <<= 1) {
    const unsigned long long add = pos >= off ? sm.part[pos - off] : 0ull;
    __syncthreads();
    sm.part[pos] += add;
    __syncthreads();
  }
  const unsigned long long r = sm.part[pos];
  __syncthreads();
  return r;
}

template <typename T>
__device__ inline unsigned long long bin_sum(const T* h, int per) {
  unsigned long long s = 0;
  for (int j = 0; j < per; ++j) s += h[threadIdx.x * per + j];
  return s;
}

// Bin holding the rank-th largest entry (counts from the top), and the count above it.
__device__ inline void rank_from_top(const uint32_t* cnt, int nbins, unsigned long long rank,
                                     TopkSmem& sm, int& bin, unsigned long long& above) {
  const int per = nbins / kTT;
  const unsigned long long s = bin_sum(cnt, per);
  const unsigned long long incl = block_scan(s, false, sm);  // threads >= this one
  const unsigned long long excl = incl - s;
  if (excl < rank && rank <= incl) {
    unsigned long long run = excl;
    for (int j = per - 1; j >= 0; --j) {
      const uint32_t c = cnt[threadIdx.x * per + j];
      if (run + c >= rank) {
        sm.result[0] = (unsigned long long)(threadIdx.x * per + j);
        sm.result[1] = run;
        break;
      }
      run += c;
    }
  }
  __syncthreads();
  bin = (int)sm.result[0];
  above = sm.result[1];
  __syncthreads();
}

// Bin holding the rank-th smallest entry (counts from the bottom), and the count below it.
__device__ inline void rank_from_bottom(const uint32_t* cnt, int nbins, unsigned long long rank,
                                        TopkSmem& sm, int& bin, unsigned long long& below) {
  const int per = nbins / kTT;
  const unsigned long long s = bin_sum(cnt, per);
  const unsigned long long incl = block_scan(s, true, sm);
  const unsigned long long excl = incl - s;
  if (excl < rank && rank <= incl) {
    unsigned long long run = excl;
    for (int j = 0; j < per; ++j) {
      const uint32_t c = cnt[threadIdx.x * per + j];
      if (run + c >= rank) {
        sm.result[0] = (unsigned long long)(threadIdx.x * per + j);
        sm.result[1] = run;
        break;
      }
      run += c;
    }
  }
  __syncthreads();
  bin = (int)sm.result[0];
  below = sm.result[1];
  __syncthreads();
}

// First bin (smallest first) whose cumulative mass exceeds `limit`, and the mass below it;
// found = false when the total is <= limit.
__device__ inline void mass_from_bottom(const unsigned long long* mass, int nbins,
                                        unsigned long long limit, TopkSmem& sm, int& bin,
                                        unsigned long long& below, bool& found) {
  const int per = nbins / kTT;
  if (threadIdx.x == 0) sm.result[2] = 0;
  const unsigned long long s = bin_sum(mass, per);
  const unsigned long long incl = block_scan(s, true, sm);
  const unsigned long long excl = incl - s;
  if (excl <= limit && limit < incl) {
    unsigned long long run = excl;
    for (int j = 0; j < per; ++j) {
      const unsigned long long m = mass[threadIdx.x * per + j];
      if (run + m > limit) {
        sm.result[0] = (unsigned long long)(threadIdx.x * per + j);
        sm.result[1] = run;
        sm.result[2] = 1;
        break;
      }
      run += m;
    }
  }
  __syncthreads();
  bin = (int)sm.result[0];
  below = sm.result[1];
  found = sm.result[2] != 0;
  __syncthreads();
}

// floor(t * S) for fp32 t in (0, 1] and S < 2^64, exactly: t = mant * 2^(e - 24).
__device__ inline unsigned long long scaled_floor(float t, unsigned long long S) {
  int e;
  const float fr = frexpf(t, &e);  // t = fr * 2^e, fr in [0.5, 1)
  const unsigned long long mant = (unsigned long long)(fr * 16777216.0f);
  const int sh = 24 - e;           // >= 23 since t <= 1
  const unsigned long long lo = mant * S;
  const unsigned long long hi = __umul64hi(mant, S);
  return sh >= 64 ? (hi >> (sh - 64)) : ((hi << (64 - sh)) | (lo >> sh));
}

__global__ __launch_bounds__(kTT) void topk_topp_kernel(float* logits, int64_t stride,
                                                        const int64_t* top_k, const float* top_p,
                                                        int V) {
  __shared__ TopkSmem sm;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  float* x = logits + (int64_t)row * stride;
  const bool aligned = ((uintptr_t)x % 16) == 0;

  const int64_t kk = top_k ? top_k[row] : (int64_t)V;
  const bool has_k = kk > 0 && kk < V;  // k >= V keeps everything (rows without top-k)
  const float t = top_p ? 1.0f - top_p[row] : -1.f;
  const bool has_p = top_p != nullptr && t >= 0.f;  // t < 0 masks nothing
  if (!has_k && !has_p) return;

  // ---- row max key, and the highest index holding it (the last entry of a stable sort) ----
  unsigned long long best = 0;
  for_each(x, V, aligned, [&](int i, float v) {
    const unsigned long long kv = ((unsigned long long)ordered_bits(v) << 32) | (uint32_t)i;
    best = kv > best ? kv : best;
  });
  best = wave_max_u64(best);
  if (lane_id() == 0) sm.red[wave_id()] = best;
  __syncthreads();
  best = 0;
  for (int w = 0; w < kTW; ++w) best = sm.red[w] > best ? sm.red[w] : best;
  __syncthreads();
  const uint32_t max_key = (uint32_t)(best >> 32);
  const int max_idx = (int)(uint32_t)best;
  const float row_max = key_value(max_key);

  // ---- top-k: keys >= tau survive ----
  uint32_t tau = 0;
  if (has_k) {
    uint32_t prefix = 0;
    unsigned long long rank = (unsigned long long)kk;
    for (int lv = 0; lv < 3; ++lv) {
      const int shift = digit_shift(lv), nbins = 1 << digit_width(lv), hi = shift + digit_width(lv);
      for (int b = tid; b < kMaxBins; b += kTT) sm.h.cnt[b] = 0;
      __syncthreads();
      for_each(x, V, aligned, [&](int, float v) {
        const uint32_t key = ordered_bits(v);
        if (hi == 32 || (key >> hi) == (prefix >> hi))
          atomicAdd(&sm.h.cnt[(key >> shift) & (nbins - 1)], 1u);
      });
      __syncthreads();
      int bin;
      unsigned long long above;
      rank_from_top(sm.h.cnt, nbins, rank, sm, bin, above);
      prefix |= (uint32_t)bin << shift;
      rank -= above;
    }
    tau = prefix;
  }

  // ---- top-p: masked = key < kappa, or key == kappa with index <= tie_idx ----
  bool p_all = false;  // every entry but the last (max_key, max_idx) is masked
  uint32_t kappa = 0;
  int tie_idx = -1;
  if (has_p) {
    uint32_t prefix = 0;
    unsigned long long below_total = 0, limit = 0;
    bool found = true;
    for (int lv = 0; lv < 3 && found; ++lv) {
      const int shift = digit_shift(lv), nbins = 1 << digit_width(lv), hi = shift + digit_width(lv);
      for (int b = tid; b < kMaxBins; b += kTT) sm.h.mass[b] = 0;
      __syncthreads();
      for_each(x, V, aligned, [&](int, float v) {
        const uint32_t key = ordered_bits(v);
        if ((!has_k || key >= tau) && (hi == 32 || (key >> hi) == (prefix >> hi))) {
          const unsigned long long m = mass_of(v, row_max);
          if (m) atomicAdd(&sm.h.mass[(key >> shift) & (nbins - 1)], m);
        }
      });
      __syncthreads();
      if (lv == 0) {
        const unsigned long long total = block_scan(bin_sum(sm.h.mass, nbins / kTT), true, sm);
        if (tid == kTT - 1) sm.result[3] = total;
        __syncthreads();
        const unsigned long long S = sm.result[3];
        __syncthreads();
        limit = t == 0.f ? 0ull : scaled_floor(t, S);
      }
      int bin;
      unsigned long long below;
      mass_from_bottom(sm.h.mass, nbins, limit - below_total, sm, bin, below, found);
      if (found) {
        prefix |= (uint32_t)bin << shift;
        below_total += below;
      }
    }
    if (!found) {
      p_all = true;
    } else {
      kappa = prefix;
      // entries equal to kappa have equal mass mu; the first j of them (by index) are masked
      const unsigned long long mu = mass_of(key_value(kappa), row_max);
      const unsigned long long j = mu ? (limit - below_total) / mu : 0;
      if (j > 0) {
        uint32_t iprefix = 0;
        unsigned long long rank = j;  // the j-th smallest index among the ties
        for (int lv = 0; lv < 3; ++lv) {
          const int shift = digit_shift(lv), nbins = 1 << digit_width(lv), hi = shift + digit_width(lv);
          for (int b = tid; b < kMaxBins; b += kTT) sm.h.cnt[b] = 0;
          __syncthreads();
          for_each(x, V, aligned, [&](int i, float v) {
            const uint32_t ui = (uint32_t)i;
            if (ordered_bits(v) == kappa && (hi == 32 || (ui >> hi) == (iprefix >> hi)))
              atomicAdd(&sm.h.cnt[(ui >> shift) & (nbins - 1)], 1u);
          });
          __syncthreads();
          int bin;
          unsigned long long below;
          rank_from_bottom(sm.h.cnt, nbins, rank, sm, bin, below);
          iprefix |= (uint32_t)bin << shift;
          rank -= below;
        }
        tie_idx = (int)iprefix;
      }
    }
  }

  // ---- write pass ----
  for (int i = tid * 4; i < V; i += kTT * 4) {
    float v[4];
    const int n = min(4, V - i);
    const bool vec = aligned && n == 4;
    if (vec) {
      const u32x4 r = *reinterpret_cast<const u32x4*>(x + i);
      for (int j = 0; j < 4; ++j) v[j] = __uint_as_float(r[j]);
    } else {
      for (int j = 0; j < n; ++j) v[j] = x[i + j];
    }
    bool any = false;
    for (int j = 0; j < n; ++j) {
      const uint32_t key = ordered_bits(v[j]);
      bool masked = has_k && key < tau;
      if (has_p) {
        if (p_all) masked |= !(key == max_key && i + j == max_idx);
        else masked |= key < kappa || (key == kappa && i + j <= tie_idx);
      }
      if (masked && !(v[j] == -INFINITY)) {
        v[j] = -INFINITY;
        any = true;
      }
    }
    if (any) {
      if (vec) {
        u32x4 w;
        for (int j = 0; j < 4; ++j) w[j] = __float_as_uint(v[j]);
        *reinterpret_cast<u32x4*>(x + i) = w;
      } else {
        for (int j = 0; j < n; ++j) x[i + j] = v[j];
      }
    }
  }
}

}  // namespace

hipError_t launch_topk_topp(float* logits, int64_t stride, const int64_t* top_k,
                            const float* top_p, int64_t num_rows, int64_t vocab_size,
                            hipStream_t stream) {
  hipLaunchKernelGGL(topk_topp_kernel, dim3((unsigned)num_rows), dim3(kTT), 0, stream, logits,
                     stride, top_k, top_p, (int)vocab_size);
  return hipGetLastError();
}

}  // namespace mvsd
