// Speculative logprobs: for every output position of a verification step, the log-softmax
// (or the logits themselves) of the row that position was sampled from, its top-k and the
// sampled token's logprob and rank (minivllm/sample/rejection_sampler.py:229-300 with
// Sampler.compute_logprobs / gather_logprobs / batched_count_greater_than,
// minivllm/sample/sampler.py:313-349).
//
// Position (r, j) of request r (j <= max_spec_len) reads compact row start_r + j (clamped to
// the last row), where the compact rows are each request's K_r verify rows followed by its
// bonus row and start_r is the request's first compact row.  A verify row comes from `target`
// (through target_rows when given), a bonus row from `bonus`.  Placeholder ids (-1) read
// token 0.  Per row:
//   lp(x) = (x - M) - log(sum exp(x - M))   (log-softmax, fp32)   or   lp(x) = x  (logits mode)
//   out[0] = (token, lp(x_token)), out[1 .. k] = top-k of lp by (value desc, index asc),
//   rank = #{i : lp(x_i) >= lp(x_token)}.
// One 512-thread workgroup per position: pass 1 reduces (M, S); pass 2 keeps per-thread lists
// of the KMAX largest (value, index) keys, counts the rank, then merges the lists per wave and
// across waves by rounds of key maxima.  For k > KMAX, pass 2 repeats over the keys below the
// last one found, KMAX at a time (ceil(k / 32) passes for k > 8).
#include "logprobs.h"
#include "mvsd_device.h"

namespace mvsd {

constexpr int kLpThreads = 512;
constexpr int kLpWaves = kLpThreads / kWave;

__device__ inline uint64_t umax_key(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <int KMAX>
__global__ __launch_bounds__(kLpThreads) void spec_logprobs_kernel(LogprobParams p) {
#pragma clang fp contract(off)
  __shared__ float s_m[kLpWaves], s_s[kLpWaves];
  __shared__ uint64_t s_cand[kLpWaves * KMAX];
  __shared__ int s_cnt[kLpWaves];
  __shared__ uint64_t s_bound;
  const int tid = threadIdx.x, lane = lane_id(), wid = wave_id();
  const int n = blockIdx.x;  // position r * W + j
  const float* x;
  int token;
  if (p.flat) {
    x = p.bonus + (int64_t)n * p.bstride;
    token = p.tokens[n];
  } else {
    const int r = n / p.W, j = n - r * p.W;
    const int start = r == 0 ? 0 : p.cu_sampled[r - 1];
    const int last = p.P + p.B - 1;
    const int c = min(start + j, last);
    // request owning compact row c: the first q with cu_sampled[q] > c
    int lo = 0, hi = p.B - 1;
    while (lo < hi) {
      const int mid = (lo + hi) / 2;
      if (p.cu_sampled[mid] > c) hi = mid;
      else lo = mid + 1;
    }
    const int q = lo;
    const int qstart = q == 0 ? 0 : p.cu_sampled[q - 1];
    const int kq = p.cu_sampled[q] - qstart - 1;  // verify rows of request q
    if (c - qstart < kq) {
      const int vrow = c - q;  // verify rows before c: c minus the bonus rows of requests < q
      const int64_t trow = p.target_rows ? p.target_rows[vrow] : vrow;
      x = p.target + trow * p.tstride;
    } else {
      x = p.bonus + (int64_t)q * p.bstride;
    }
    token = p.tokens[(int64_t)r * p.tok_stride + j];
  }
  token = token == -1 ? 0 : min(max(token, 0), p.V - 1);

  // ---- pass 1: row max and sum of exp(x - max) ----
  float lpm = 0.f, L = 0.f;
  if (!p.logits_mode) {
    float m = -INFINITY, s = 0.f;
    for (int i = tid; i < p.V; i += kLpThreads) {
      const float v = x[i];
      if (v > m) {
        s = s * expf(m - v);
        m = v;
      }
      if (v != -INFINITY) s += expf(v - m);  // masked entries add nothing (and no NaN)
    }
    const float wm = wave_max(m);
    const float ws = wave_sum(m == -INFINITY ? 0.f : s * expf(m - wm));
    if (lane == 0) {
      s_m[wid] = wm;
      s_s[wid] = ws;
    }
    __syncthreads();
    float M = -INFINITY;
    for (int w = 0; w < kLpWaves; ++w) M = fmaxf(M, s_m[w]);
    float S = 0.f;
    for (int w = 0; w < kLpWaves; ++w)
      if (s_m[w] != -INFINITY) S += s_s[w] * expf(s_m[w] - M);
    lpm = M;
    L = logf(S);
  }
  auto lp = [&](float v) { return p.logits_mode ? v : (v - lpm) - L; };
  const float tlp = lp(x[token]);
  // the order the top-k and the rank use: the log-softmax, or the raw values
  auto ord = [&](float v) { return p.rank_raw ? v : lp(v); };
  const float tord = ord(x[token]);

  // ---- pass 2 (repeated): per-thread top-KMAX keys below `bound`, and the rank count ----
  // Round t collects the next min(KMAX, k - done) largest keys strictly below the last key of
  // round t - 1; keys are distinct (the index is in the low word), so the rounds partition
  // the top-k exactly.
  const int k = p.k;
  const int n_out = k + 1;
  uint64_t bound = ~0ull;
  int done = 0;
  bool first_pass = true;
  while (first_pass || done < k) {
    const int need = min(KMAX, k - done);
    uint64_t key[KMAX];
#pragma unroll
    for (int i = 0; i < KMAX; ++i) key[i] = 0;
    int cnt = 0;
    for (int i = tid; i < p.V; i += kLpThreads) {
      const float v = ord(x[i]);
      cnt += v >= tord ? 1 : 0;
      uint64_t kk = argmax_key(v, i);
      if (kk < bound && kk > key[KMAX - 1]) {
        // insertion into the descending list (one compare-exchange step per slot)
#pragma unroll
        for (int s2 = 0; s2 < KMAX; ++s2) {
          const uint64_t a = key[s2];
          const bool sw = kk > a;
          key[s2] = sw ? kk : a;
          kk = sw ? a : kk;
        }
      }
    }
    if (first_pass) {
      // rank: block sum of the counts
      int c2 = cnt;
      for (int off = kWave / 2; off > 0; off >>= 1) c2 += __shfl_xor(c2, off, kWave);
      if (lane == 0) s_cnt[wid] = c2;
    }

    // per-wave merge: `need` rounds, the lane holding the largest head pops it
    for (int round = 0; round < need; ++round) {
      const uint64_t best = wave_max_u64(key[0]);
      if (lane == 0) s_cand[wid * KMAX + round] = best;
      if (key[0] == best && best != 0) {
#pragma unroll
        for (int s2 = 0; s2 + 1 < KMAX; ++s2) key[s2] = key[s2 + 1];
        key[KMAX - 1] = 0;
      }
    }
    __syncthreads();
    // block merge by wave 0: lanes hold the waves' sorted candidate lists
    if (wid == 0) {
      constexpr int PER = (kLpWaves * KMAX + kWave - 1) / kWave;
      uint64_t cand[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int ci = lane * PER + i;
        cand[i] = ci < kLpWaves * KMAX && (ci % KMAX) < need ? s_cand[ci] : 0;
      }
      // sort each lane's few candidates (descending)
#pragma unroll
      for (int a = 0; a < PER; ++a)
#pragma unroll
        for (int b = a + 1; b < PER; ++b) {
          const uint64_t hi2 = umax_key(cand[a], cand[b]);
          const uint64_t lo2 = cand[a] ^ cand[b] ^ hi2;
          cand[a] = hi2;
          cand[b] = lo2;
        }
      uint64_t last = bound;
      for (int round = 0; round < need; ++round) {
        const uint64_t best = wave_max_u64(cand[0]);
        if (lane == 0) {
          // the value is recomputed from the index (the key's order bits merge -0.0 and +0.0)
          const int idx = min(max(key_index(best), 0), p.V - 1);
          p.ids[(int64_t)n * n_out + 1 + done + round] = idx;
          p.lps[(int64_t)n * n_out + 1 + done + round] = lp(x[idx]);
        }
        last = best;
        if (cand[0] == best && best != 0) {
#pragma unroll
          for (int s2 = 0; s2 + 1 < PER; ++s2) cand[s2] = cand[s2 + 1];
          cand[PER - 1] = 0;
        }
      }
      if (lane == 0) {
        s_bound = last;
        if (first_pass) {
          int rank = 0;
          for (int w = 0; w < kLpWaves; ++w) rank += s_cnt[w];
          p.ids[(int64_t)n * n_out] = token;
          p.lps[(int64_t)n * n_out] = tlp;
          p.ranks[n] = rank;
        }
      }
    }
    __syncthreads();
    bound = s_bound;
    done += need;
    first_pass = false;
  }
}

hipError_t launch_spec_logprobs(const LogprobParams& p, hipStream_t stream) {
  const int n = p.B * p.W;
  if (n <= 0) return hipSuccess;
  if (p.k <= 8)
    hipLaunchKernelGGL(spec_logprobs_kernel<8>, dim3(n), dim3(kLpThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(spec_logprobs_kernel<32>, dim3(n), dim3(kLpThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mvsd
