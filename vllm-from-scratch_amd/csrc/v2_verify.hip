// V2 speculative-decoding verification (the V2 model runner's rejection sampler) for gfx950.
//
// Replaces rejection_sample (minivllm/worker/gpu/spec_decode/rejection_sampler_utils.py:935-1201),
// standard and block verification, with these launches on the caller's stream:
//   1. v2_stats_kernel     one workgroup per (verify row, 4096-column chunk): greedy rows keep
//                          the chunk's (max, first argmax); random rows keep (max, sum exp) of
//                          the target row and of the temperature-scaled draft row (:206-316);
//   2. v2_rowstat_kernel   one wavefront per verify row combines the chunk partials: a greedy
//                          row's argmax; a random row's target and draft log-sum-exp and the
//                          log-probabilities of the row's draft token (:134-203);
//   3. v2_residual_kernel  block verification with draft logits only: one workgroup per
//                          (verify row, chunk) sums max(p_i M_b(x) - M_s(x), 0) over the chunk,
//                          p_i the running joint ratio of the rows before it (:318-446);
//   4. v2_chain_kernel     one wavefront per request decides its chain (:497-706): the
//                          per-step inputs and acceptance uniforms are loaded and drawn one step
//                          per lane, the decisions then run in order over the lanes;
//   5. v2_resample_kernel  one workgroup per (request, chunk) scores the rejected (or bonus)
//                          row: residual log-probabilities log(p_tau p - q) (or the target row,
//                          or the target row without the rejected draft) plus Gumbel noise drawn
//                          per vocabulary index (:709-866, gumbel.py:95-131);
//   6. v2_insert_kernel    one wavefront per request takes the first chunk maximum and writes
//                          the resampled token and the sampled count (:869-932).
// The counter stream is Philox4x32 with ten rounds keyed by the 64-bit seed and counted by
// the 64-bit position (or the 32-bit vocabulary index), the generator behind Triton's
// tl.randint4x / tl.rand that gumbel.py:72-91 uses (Salmon et al., SC 2011).
//
// HBM traffic per call: every verify row of the target once (and the draft row of random
// requests once) in pass 1, again in pass 3 for block verification with draft logits, one
// target row (and one draft row) per request in pass 5; the partials are a few hundred bytes
// per row.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "mvsd_device.h"

namespace mvsd {

int record_hip_error(hipError_t err);  // capi.hip: keeps err for mvsd_last_hip_error()

namespace {

constexpr int kV2Chunk = 4096;                 // columns per workgroup in passes 1 and 3
constexpr int kV2PerThread = kV2Chunk / kThreads;  // 16

// ------------------------------------------------------------------ counter RNG -------

struct U32x4 {
  uint32_t x, y, z, w;
};

__device__ inline U32x4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                      uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    // One 32x32->64 multiply per product (v_mad_u64_u32) instead of separate lo and hi.
    const uint64_t p0 = (uint64_t)0xCD9E8D57u * c2, p2 = (uint64_t)0xD2511F53u * c0;
    const uint32_t h0 = (uint32_t)(p0 >> 32), l0 = (uint32_t)p0;
    const uint32_t h2 = (uint32_t)(p2 >> 32), l2 = (uint32_t)p2;
    c0 = h0 ^ c1 ^ k0;
    c2 = h2 ^ c3 ^ k1;
    c1 = l0;
    c3 = l2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return {c0, c1, c2, c3};
}

// a ^ b ^ k in one VALU instruction: gfx950's three-input bitwise op v_bitop3_b32 with the
// truth table of a three-way xor (0x96).  k is read from a scalar register, so it must be
// uniform across the wavefront.
__device__ inline uint32_t xor3_uniform(uint32_t a, uint32_t b, uint32_t k) {
  uint32_t r;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(r) : "v"(a), "v"(b), "s"(k));
  return r;
}

// philox4x32_10 for a key (k0, k1) that is uniform across the wavefront: the same rounds,
// with each round's pair of xors fused from round 3 on (the first two rounds of the races'
// counters (col, 0, 0, 0) fold to fewer operations, which the compiler finds itself).
__device__ inline U32x4 philox4x32_10_uniform_key(uint32_t c0, uint32_t c1, uint32_t c2,
                                                  uint32_t c3, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xCD9E8D57u * c2, p2 = (uint64_t)0xD2511F53u * c0;
    if (r < 2) {
      c0 = (uint32_t)(p0 >> 32) ^ c1 ^ k0;
      c2 = (uint32_t)(p2 >> 32) ^ c3 ^ k1;
    } else {
      c0 = xor3_uniform((uint32_t)(p0 >> 32), c1, k0);
      c2 = xor3_uniform((uint32_t)(p2 >> 32), c3, k1);
    }
    c1 = (uint32_t)p0;
    c3 = (uint32_t)p2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return {c0, c1, c2, c3};
}

// tl.randint4x(seed, offset) with a 64-bit offset: counter (lo, hi, 0, 0), key (seed lo, hi).
__device__ inline U32x4 randint4x64(int64_t seed, int64_t offset) {
  return philox4x32_10((uint32_t)offset, (uint32_t)((uint64_t)offset >> 32), 0u, 0u,
                       (uint32_t)seed, (uint32_t)((uint64_t)seed >> 32));
}



// uint_to_uniform_float for 32 bits, clamped away from zero (tl_rand32, includes_zero=False).
__device__ inline float uniform_f32(uint32_t bits) {
  int32_t i = (int32_t)bits;
  i = i < 0 ? -i - 1 : i;
  const float u = (float)i * 4.6566127342e-10f;
  return fmaxf(u, 4.6566127342e-10f);
}

// tl_rand64(includes_zero=False): (hi << 32 | lo) * 2^-64, clamped to the smallest normal.
__device__ inline double uniform_f64(uint32_t lo, uint32_t hi) {
  const uint64_t r = ((uint64_t)hi << 32) | lo;
  const double u = (double)r * 5.421010862427522170037e-20;
  return fmax(u, 2.2250738585072014e-308);
}

// ------------------------------------------------------------------ fast math ---------
// The per-vocabulary-entry work uses the hardware exponential and logarithm: __expf, and
// v_log_f32 (base 2, within 1 ulp over the normal range) scaled by ln 2.  The reference's
// Triton kernels likewise use the approximate tl.exp / tl.log forms.

// Natural logarithm of a positive normal x (0 gives -inf).
__device__ inline float hw_log(float x) { return __builtin_amdgcn_logf(x) * 0.693147182f; }

// log(1 + a) for -1 <= a <= 0: w = 1 + a rounded, and the rounding of w corrected by the
// factor a / (w - 1) (Goldberg, "What every computer scientist should know about
// floating-point arithmetic", 1991, Theorem 4), a itself when w rounds to 1; within about
// 3 ulp.  log1p(-1) = -inf.  Both branches are computed and one is selected.
__device__ inline float fast_log1p(float a) {
  const float w = 1.f + a;
  const float r = hw_log(w) * (a * __builtin_amdgcn_rcpf(w - 1.f));
  return w == 1.f ? a : r;
}

// ------------------------------------------------------------------ arguments ---------

// What the resampling pass does for one request, written by the chain kernel so that a
// resampling workgroup starts its row loads after one descriptor load.
enum ResampleMode : int32_t {
  kResampleNone = 0,      // greedy request with a rejection: the chain wrote the argmax
  kResampleArgmax = 1,    // greedy bonus row: argmax of the target row
  kResampleTarget = 2,    // bonus row, or a placeholder draft: the target row as it is
  kResampleResidual = 3,  // rejected draft with draft logits: log max(p_tau p - q, 0)
  kResampleExclude = 4,   // rejected one-hot draft: the target row without that id
};

struct ResampleDesc {
  int64_t row;     // target row
  int64_t draft;   // element offset of the draft row (draft logits)
  float tl, dl;    // target / draft log-sum-exp of the row
  float shift;     // log p_tau (block verification), else 0
  float temp;      // temperature of the request's state
  uint32_t gseed;  // key of the row's Gumbel race, tl.randint(seed, pos)
  int32_t rej;     // the rejected draft id (kResampleExclude)
  int32_t mode;    // ResampleMode
  // High word of the race's Philox key: always 0 (tl.randint's 32-bit seed).  Read at run
  // time so that the key schedule stays in scalar registers, where the rounds' xors can
  // take it as an operand, instead of folding into literals.
  uint32_t key_hi;
};
static_assert(sizeof(ResampleDesc) == 48, "descriptor layout");

struct V2Params {
  int64_t* sampled;
  int64_t sampled_stride;
  int32_t* num_sampled;
  const void* target;
  int64_t target_stride;
  const void* draft;  // [states, K, V] or null
  int64_t draft_stride0, draft_stride1;
  const int32_t* draft_sampled;
  const int32_t* cu_num_logits;
  const int64_t* pos;
  const int32_t* idx_mapping;
  const int32_t* exp_idx_mapping;
  const int32_t* exp_local_pos;
  const float* temperature;
  const int64_t* seed;
  const float* rates;  // synthetic conditional rates [K] or null
  int64_t num_logits;
  int32_t num_reqs, num_states, vocab, K, nchunks;
  int use_fp64;
  int use_block;  // block verification (Sun et al. 2024) instead of the per-token test
  bool target_aligned, draft_aligned;
  // workspace
  float *tmax, *tsum, *dmax, *dsum;  // [num_logits, nchunks] chunk partials
  int32_t* targ;
  float *rtl, *rdl;      // [num_logits] target / draft log-sum-exp of a random verify row
  float *rtlp, *rdlp;    // [num_logits] log p and log q of the row's draft token
  int32_t* rarg;         // [num_logits] target argmax of a greedy verify row
  float* rmass;          // [num_logits, nchunks] block residual-mass partials
  int32_t* acc;  // accepted length per request, -1 for a malformed request
  struct ResampleDesc* desc;  // [num_reqs] what the resampling pass scores, from the chain
  double* rval;
  int32_t* ridx;
};

__device__ inline int clamp_state(int s, int n) { return s < 0 ? 0 : (s >= n ? n - 1 : s); }

// Load this thread's kV2Chunk / NT columns of a chunk as fp32 (NT threads per workgroup);
// columns at or past `limit` read -inf.
template <int DT, int NT = kThreads>
__device__ inline void load_chunk(const void* base, int64_t row_off, int c0, int limit,
                                  bool aligned, float (&x)[kV2Chunk / NT]) {
  using S = typename Elem<DT>::storage;
  constexpr int VEC = Elem<DT>::kVec;
  const S* p = reinterpret_cast<const S*>(base) + row_off;
#pragma unroll
  for (int j = 0; j < kV2Chunk / NT / VEC; ++j) {
    const int col = c0 + (j * NT + (int)threadIdx.x) * VEC;
    float v[VEC];
    load_vec<DT>(p, col, limit, aligned, -INFINITY, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) x[j * VEC + e] = v[e];
  }
}

template <int NT = kThreads>
__device__ inline int chunk_col(int c0, int k, int VEC) {
  const int j = k / VEC, e = k % VEC;
  return c0 + (j * NT + (int)threadIdx.x) * VEC + e;
}

// Best (value, index) over the block: larger value, then lower index.  Doubles so the fp64
// Gumbel scores reduce with the same code.
template <int NW = kWaves>
__device__ inline void block_best(double& v, int& i, double* s_v, int* s_i) {
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) {
    const double ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(i, off);
    const bool take = (ov > v) | ((ov == v) & (oi < i));
    v = take ? ov : v;
    i = take ? oi : i;
  }
  if (lane_id() == 0) {
    s_v[wave_id()] = v;
    s_i[wave_id()] = i;
  }
  __syncthreads();
  v = s_v[0];
  i = s_i[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    const bool take = (s_v[w] > v) | ((s_v[w] == v) & (s_i[w] < i));
    v = take ? s_v[w] : v;
    i = take ? s_i[w] : i;
  }
}

// ------------------------------------------------------------------ pass 1 ------------

// (max, sum exp(x - max)) of G rows of the block's values at once; sum is 0 when the max
// is -inf.
template <int G>
__device__ inline void block_max_sumexp_rows(float (&x)[G][kV2PerThread], float* s_red,
                                             float (&m)[G], float (&sm)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
#pragma unroll
    for (int k = 0; k < kV2PerThread; ++k) m[g] = fmaxf(m[g], x[g][k]);
  }
  block_max<G>(m, s_red);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    sm[g] = 0.f;
    if (m[g] > -INFINITY) {
#pragma unroll
      for (int k = 0; k < kV2PerThread; ++k) sm[g] += __expf(x[g][k] - m[g]);
    }
  }
  block_sum<G>(sm, s_red);
#pragma unroll
  for (int g = 0; g < G; ++g) sm[g] = m[g] > -INFINITY ? sm[g] : 0.f;
}

template <int TDT, int DDT, bool HAS_DRAFT>
__global__ __launch_bounds__(kThreads) void v2_stats_kernel(V2Params p) {
  __shared__ float s_red[2 * kWaves];
  __shared__ double s_v[kWaves];
  __shared__ int s_i[kWaves];
  const int64_t row = blockIdx.x;
  const int c = blockIdx.y;
  const int step = p.exp_local_pos[row];
  const int st_raw = p.exp_idx_mapping[row];
  if (step < 0 || step >= p.K) return;
  const int c0 = c * kV2Chunk;
  const int64_t slot = row * p.nchunks + c;
  constexpr int G = HAS_DRAFT ? 2 : 1;
  float x[G][kV2PerThread];
  // the target loads go out before the temperature is known; the draft loads (random rows
  // only) right after, so both rows are in flight together
  load_chunk<TDT>(p.target, row * p.target_stride, c0, p.vocab, p.target_aligned, x[0]);
  const int st = clamp_state(st_raw, p.num_states);
  const float temp = p.temperature[st];
  if constexpr (HAS_DRAFT) {
    if (temp != 0.f)
      load_chunk<DDT>(p.draft, (int64_t)st * p.draft_stride0 + (int64_t)step * p.draft_stride1,
                      c0, p.vocab, p.draft_aligned, x[1]);
  }
  if (temp == 0.f) {
    double bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < kV2PerThread; ++k) {
      const int col = chunk_col(c0, k, Elem<TDT>::kVec);
      const bool take =
          col < p.vocab && (((double)x[0][k] > bv) | (((double)x[0][k] == bv) & (col < bi)));
      bv = take ? (double)x[0][k] : bv;
      bi = take ? col : bi;
    }
    block_best(bv, bi, s_v, s_i);
    if (threadIdx.x == 0) {
      p.tmax[slot] = (float)bv;
      p.targ[slot] = bi == 0x7fffffff ? c0 : bi;
    }
    return;
  }
  if constexpr (HAS_DRAFT) {
    const Divider dv = make_divider(temp);
#pragma unroll
    for (int k = 0; k < kV2PerThread; ++k) x[1][k] = divide(dv, x[1][k]);
  }
  float m[G], sm[G];
  block_max_sumexp_rows<G>(x, s_red, m, sm);
  if (threadIdx.x == 0) {
    p.tmax[slot] = m[0];
    p.tsum[slot] = sm[0];
    if constexpr (HAS_DRAFT) {
      p.dmax[slot] = m[1];
      p.dsum[slot] = sm[1];
    }
  }
}

// ------------------------------------------------------------------ pass 2 ------------

// Log-sum-exp of a row from its chunk partials (every lane of the wave gets it).
__device__ inline float wave_lse(const float* maxes, const float* sums, int64_t base, int n) {
  float gm = -INFINITY;
  for (int c = lane_id(); c < n; c += kWave) gm = fmaxf(gm, maxes[base + c]);
  gm = wave_max(gm);
  float s = 0.f;
  for (int c = lane_id(); c < n; c += kWave) s += sums[base + c] * expf(maxes[base + c] - gm);
  s = wave_sum(s);
  return gm + logf(s);
}

__device__ inline bool draft_valid(int d, int vocab) { return d >= 0 && d < vocab; }

// Per verify row: the greedy row's global argmax (first index among equal maxima,
// :106-131), or the random row's log-sum-exps and the log-probabilities of its draft token
// (:134-203).  Draft ids outside [0, V) are placeholders; their log-probabilities are
// written from column 0 and never read.
template <int TDT, int DDT, bool HAS_DRAFT>
__global__ __launch_bounds__(kThreads) void v2_rowstat_kernel(V2Params p) {
  const int64_t row = (int64_t)blockIdx.x * kWaves + wave_id();
  if (row >= p.num_logits) return;
  const int step = p.exp_local_pos[row];
  if (step < 0 || step >= p.K) return;
  const int st = clamp_state(p.exp_idx_mapping[row], p.num_states);
  const float temp = p.temperature[st];
  const int64_t base = row * p.nchunks;
  if (temp == 0.f) {
    float bv = -INFINITY;
    int bc = 0x7fffffff;
    for (int c = lane_id(); c < p.nchunks; c += kWave) {
      float v = p.tmax[base + c];
      v = v != v ? -INFINITY : v;
      argmax_update(bv, bc, v, c, true);
    }
    wave_argmax(bv, bc);
    if (lane_id() == 0) p.rarg[row] = p.targ[base + (bc == 0x7fffffff ? 0 : bc)];
    return;
  }
  int d = row + 1 < p.num_logits ? p.draft_sampled[row + 1] : -1;
  d = draft_valid(d, p.vocab) ? d : 0;
  using TS = typename Elem<TDT>::storage;
  const float xt = Elem<TDT>::cvt(reinterpret_cast<const TS*>(p.target)[row * p.target_stride + d]);
  float xd = 0.f;
  if constexpr (HAS_DRAFT) {
    using DS = typename Elem<DDT>::storage;
    xd = Elem<DDT>::cvt(reinterpret_cast<const DS*>(
        p.draft)[(int64_t)st * p.draft_stride0 + (int64_t)step * p.draft_stride1 + d]);
  }
  const float t_lse = wave_lse(p.tmax, p.tsum, base, p.nchunks);
  float d_lse = 0.f, dlp = 0.f;
  if constexpr (HAS_DRAFT) {
    d_lse = wave_lse(p.dmax, p.dsum, base, p.nchunks);
    dlp = divide(make_divider(temp), xd) - d_lse;
  }
  if (lane_id() == 0) {
    p.rtl[row] = t_lse;
    p.rdl[row] = d_lse;
    p.rtlp[row] = xt - t_lse;
    p.rdlp[row] = dlp;
  }
}

// One step of the running joint ratio, log p_{i+1} = min(log p_i + log p - log q, 0)
// (:365-381).  The residual pass and the chain fold the same values in the same order.
__device__ inline float fold_log_ratio(float log_p, float tlp, float dlp) {
  return fminf(log_p + (tlp - dlp), 0.f);
}

// ------------------------------------------------------------------ pass 3 (block) ----

// Residual mass of the rows the block threshold looks ahead to (:387-446): rows at draft
// step 1..K-1 of a random request whose own draft is verifiable.  Each wave folds the joint
// ratio of the rows before this one (one step per lane, then in order over the lanes).
template <int TDT, int DDT>
__global__ __launch_bounds__(kThreads) void v2_residual_kernel(V2Params p) {
  __shared__ float s_sum[kWaves];
  const int64_t row = blockIdx.x;
  const int c = blockIdx.y;
  const int step = p.exp_local_pos[row];
  if (step < 1 || step >= p.K || step > row || row + 1 >= p.num_logits) return;
  if (!draft_valid(p.draft_sampled[row + 1], p.vocab)) return;
  const int st = clamp_state(p.exp_idx_mapping[row], p.num_states);
  const float temp = p.temperature[st];
  if (temp == 0.f) return;
  const int64_t start = row - step;
  float log_p = 0.f;
  for (int b = 0; b < step; b += kWave) {
    const int j = b + lane_id();
    const bool in = j < step;
    const bool v = in && draft_valid(p.draft_sampled[start + j + 1], p.vocab);
    const float tlp = in ? p.rtlp[start + j] : 0.f;
    const float dlp = in ? p.rdlp[start + j] : 0.f;
    const uint64_t vm = __ballot(v);
    const int n = step - b < kWave ? step - b : kWave;
    for (int k = 0; k < n; ++k)
      if ((vm >> k) & 1) log_p = fold_log_ratio(log_p, readlane_f32(tlp, k), readlane_f32(dlp, k));
  }
  const float prefix = expf(log_p);
  const float t_lse = p.rtl[row], d_lse = p.rdl[row];
  const int c0 = c * kV2Chunk;
  float x[kV2PerThread], q[kV2PerThread];
  load_chunk<TDT>(p.target, row * p.target_stride, c0, p.vocab, p.target_aligned, x);
  load_chunk<DDT>(p.draft, (int64_t)st * p.draft_stride0 + (int64_t)step * p.draft_stride1, c0,
                  p.vocab, p.draft_aligned, q);
  float part[1] = {0.f};
  const Divider dv = make_divider(temp);
#pragma unroll
  for (int k = 0; k < kV2PerThread; ++k) {
    const float m_b = __expf(x[k] - t_lse);
    const float m_s = __expf(divide(dv, q[k]) - d_lse);
    part[0] += fmaxf(prefix * m_b - m_s, 0.f);
  }
  block_sum<1>(part, s_sum);
  if (threadIdx.x == 0) p.rmass[row * p.nchunks + c] = part[0];
}

// ------------------------------------------------------------------ pass 4 ------------

template <int TDT, bool HAS_DRAFT>
__global__ __launch_bounds__(kThreads) void v2_chain_kernel(V2Params p) {
  const int r = blockIdx.x * kWaves + wave_id();
  if (r >= p.num_reqs) return;
  const int64_t start = p.cu_num_logits[r], end = p.cu_num_logits[r + 1];
  if (start < 0 || end > p.num_logits || end <= start || end - start - 1 > p.K) {
    if (lane_id() == 0) {
      p.acc[r] = -1;
      p.desc[r] = ResampleDesc{};
    }
    return;
  }
  const int nd = (int)(end - start - 1);
  const int st = clamp_state(p.idx_mapping[r], p.num_states);
  const int64_t seed = p.seed[st];
  const float temp = p.temperature[st];
  const bool greedy = temp == 0.f;
  const bool block = p.use_block && !greedy;
  using TS = typename Elem<TDT>::storage;
  const TS* tgt = reinterpret_cast<const TS*>(p.target);
  int acc = 0;
  bool verifying = true;
  float log_p = 0.f, lpt = 0.f;
  int64_t* out = p.sampled + (int64_t)r * p.sampled_stride;
  for (int b = 0; b < nd && verifying; b += kWave) {
    // one step per lane: draft id, acceptance uniform and the row's precomputed inputs
    const int j = b + lane_id();
    const bool in = j < nd;
    const int64_t li = start + j;
    const int d = in ? p.draft_sampled[li + 1] : -1;
    const bool valid = draft_valid(d, p.vocab);
    const float u = in ? uniform_f32(randint4x64(seed, p.pos[li]).x) : 1.f;
    int am = 0;
    float tlp = 0.f, dlp = 0.f, res = 0.f, tnext = 0.f, lse_next = 0.f;
    bool next_valid = false;
    if (in && greedy) am = p.rarg[li];
    if (in && !greedy) {
      tlp = p.rtlp[li];
      dlp = p.rdlp[li];
    }
    if (in && block && j + 1 < nd) {
      // the block threshold looks at the next row (:612-634)
      const int nx = p.draft_sampled[li + 2];
      next_valid = draft_valid(nx, p.vocab);
      if (next_valid) {
        if constexpr (HAS_DRAFT) {
          const int64_t base = (li + 1) * p.nchunks;
          for (int c = 0; c < p.nchunks; ++c) res += p.rmass[base + c];
        } else {
          tnext = Elem<TDT>::cvt(tgt[(li + 1) * p.target_stride + nx]);
          lse_next = p.rtl[li + 1];
        }
      }
    }
    const uint64_t vm = __ballot(valid), nm = __ballot(next_valid);
    const int n = nd - b < kWave ? nd - b : kWave;
    for (int k = 0; k < n; ++k) {
      const bool v = (vm >> k) & 1;
      const int dk = __builtin_amdgcn_readlane(valid ? d : 0, k);
      const float uk = readlane_f32(u, k);
      if (!greedy) verifying = verifying && v;
      if (!verifying) break;
      if (greedy) {
        const int amk = __builtin_amdgcn_readlane(am, k);
        bool ok = p.rates ? (uk < p.rates[b + k]) : (amk == dk);
        ok = ok && v;
        verifying = ok;
        acc += ok;
        if (lane_id() == 0) out[b + k] = ok ? dk : amk;
      } else if (block) {
        // Sun et al. 2024 (:608-640): accept b + k + 1 tokens when u <= h; the last
        // position that passes decides.
        log_p = fold_log_ratio(log_p, readlane_f32(tlp, k), readlane_f32(dlp, k));
        const float prefix = expf(log_p);
        float h = prefix;
        if ((nm >> k) & 1) {
          float rm;
          if constexpr (HAS_DRAFT) {
            rm = readlane_f32(res, k);
          } else {
            // one-hot drafts: p_i (1 - M_b(next draft)) in closed form (:87-104)
            rm = prefix * (1.f - expf(readlane_f32(tnext, k) - readlane_f32(lse_next, k)));
          }
          const float denom = rm + 1.f - prefix;
          h = denom > 0.f ? rm / denom : 1.f;
        }
        if (uk <= h) {
          acc = b + k + 1;
          lpt = log_p;
        }
        if (lane_id() == 0) out[b + k] = dk;
      } else {
        const bool ok = p.rates ? (uk < p.rates[b + k])
                                : (readlane_f32(tlp, k) > logf(uk) + readlane_f32(dlp, k));
        verifying = ok;
        acc += ok;
        if (lane_id() == 0) out[b + k] = dk;
      }
    }
  }
  if (lane_id() == 0) {
    p.acc[r] = acc;
    // The resampling of row start + acc (:709-866): its state and temperature come from the
    // expanded mapping of that row, as in the reference.
    const int64_t ri = start + acc;
    const bool is_bonus = acc == nd;
    const int rst = clamp_state(p.exp_idx_mapping[ri], p.num_states);
    const float rtemp = p.temperature[rst];
    const int rej = is_bonus ? -1 : p.draft_sampled[ri + 1];
    ResampleDesc d{};
    d.row = ri;
    d.draft = (int64_t)rst * p.draft_stride0 + (int64_t)acc * p.draft_stride1;
    d.temp = rtemp;
    d.rej = rej;
    if (rtemp == 0.f) {
      d.mode = is_bonus ? kResampleArgmax : kResampleNone;
    } else {
      d.gseed = randint4x64(p.seed[rst], p.pos[ri]).x;
      if (is_bonus || !draft_valid(rej, p.vocab)) {
        d.mode = kResampleTarget;
      } else if (HAS_DRAFT) {
        // statistics of the rejected row (:683-700)
        d.mode = kResampleResidual;
        d.tl = p.rtl[ri];
        d.dl = p.rdl[ri];
        // block verification scales the target by p_tau (:820-829); p_0 = 1
        d.shift = block && acc > 0 ? lpt : 0.f;
      } else {
        d.mode = kResampleExclude;
      }
    }
    p.desc[r] = d;
  }
}

// ------------------------------------------------------------------ pass 5 ------------

// Gumbel score of residual logit x at vocabulary index col: x + (-log(-log(u))) with u the
// request's counter draw for col (gumbel.py:95-131): tl_rand32 and -log(-log1p(-u)) in fp32,
// or tl_rand64 and -log(-log(u)) in fp64.
// gseed and key_hi are uniform across the workgroup (one race per row).
template <bool FP64>
__device__ inline auto gumbel_score(float x, uint32_t gseed, int col, uint32_t key_hi) {
  const U32x4 rn = philox4x32_10_uniform_key((uint32_t)col, 0u, 0u, 0u, gseed, key_hi);
  if constexpr (FP64) {
    return (double)x + (-log(-log(uniform_f64(rn.x, rn.y))));
  } else {
    const float u = uniform_f32(rn.x);
    return x + (-hw_log(-fast_log1p(-u)));
  }
}

constexpr int kResThreads = 256;  // resampling workgroup: 16 columns per thread of a chunk
constexpr int kResWaves = kResThreads / kWave;
constexpr int kResPer = kV2Chunk / kResThreads;

template <int TDT, int DDT, bool HAS_DRAFT, bool FP64>
__global__ __launch_bounds__(kResThreads) void v2_resample_kernel(V2Params p) {
  __shared__ double s_v[kResWaves];
  __shared__ int s_i[kResWaves];
  // per wave: the live entries of its 512 columns (residual logit, column offset)
  __shared__ float s_x[kResWaves][kWave * kResPer];
  __shared__ uint16_t s_c[kResWaves][kWave * kResPer];
  const int r = blockIdx.x;
  const int c = blockIdx.y;
  const ResampleDesc d = p.desc[r];
  if (d.mode == kResampleNone) return;
  const int c0 = c * kV2Chunk;
  float x[kResPer];
  load_chunk<TDT, kResThreads>(p.target, d.row * p.target_stride, c0, p.vocab, p.target_aligned, x);
  constexpr int TV = Elem<TDT>::kVec;
  if constexpr (HAS_DRAFT) {
    if (d.mode == kResampleResidual) {
      float q[kResPer];
      load_chunk<DDT, kResThreads>(p.draft, d.draft, c0, p.vocab, p.draft_aligned, q);
      const Divider dv = make_divider(d.temp);
#pragma unroll
      for (int k = 0; k < kResPer; ++k) {
        const float tlp = (x[k] - d.tl) + d.shift;
        const float dlp = divide(dv, q[k]) - d.dl;
        // log max(p - q, 0) = log p + log(1 - q / p) (:831-842)
        const float ratio = __expf(dlp - tlp);
        x[k] = ratio < 1.f ? tlp + fast_log1p(-ratio) : -INFINITY;
      }
    }
  }
  if (d.mode == kResampleExclude) {
#pragma unroll
    for (int k = 0; k < kResPer; ++k)
      x[k] = chunk_col<kResThreads>(c0, k, TV) == d.rej ? -INFINITY : x[k];
  }
  using Score = typename std::conditional<FP64, double, float>::type;
  Score bv = -INFINITY;
  int bi = 0x7fffffff;
  if (d.mode == kResampleArgmax) {
#pragma unroll
    for (int k = 0; k < kResPer; ++k) {
      const int col = chunk_col<kResThreads>(c0, k, TV);
      const bool take = col < p.vocab && ((x[k] > bv) | ((x[k] == bv) & (col < bi)));
      bv = take ? x[k] : bv;
      bi = take ? col : bi;
    }
  } else if (d.mode != kResampleResidual) {
    // the target row (less at most one id): every entry draws, straight from registers
#pragma unroll
    for (int k = 0; k < kResPer; ++k) {
      const int col = chunk_col<kResThreads>(c0, k, TV);
      if (col >= p.vocab) continue;
      const Score sc = gumbel_score<FP64>(x[k], d.gseed, col, d.key_hi);
      const bool take = (sc > bv) | ((sc == bv) & (col < bi));
      bv = take ? sc : bv;
      bi = take ? col : bi;
    }
  } else {
    // Entries whose residual logit is -inf (or NaN) score -inf (or NaN) and cannot win: only
    // the live ones draw noise.  Each wave packs its live entries into LDS and then scores
    // them four per lane at a time (independent draws for the lane to interleave).
    float* wx = s_x[wave_id()];
    uint16_t* wc = s_c[wave_id()];
    int n = 0;
#pragma unroll
    for (int k = 0; k < kResPer; ++k) {
      const int col = chunk_col<kResThreads>(c0, k, TV);
      const bool live = col < p.vocab && x[k] > -INFINITY;
      const uint64_t m = __ballot(live);
      if (live) {
        const int o = n + (int)__builtin_amdgcn_mbcnt_hi(
                              (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        wx[o] = x[k];
        wc[o] = (uint16_t)(col - c0);
      }
      n += __popcll(m);
    }
    __syncthreads();
    constexpr int kIlp = 4;
    for (int i0 = 0; i0 < n; i0 += kIlp * kWave) {
      Score sc[kIlp];
      int col[kIlp];
#pragma unroll
      for (int j = 0; j < kIlp; ++j) {
        const int i = i0 + j * kWave + lane_id();
        const bool in = i < n;
        col[j] = in ? c0 + wc[i] : 0x7fffffff;
        sc[j] = gumbel_score<FP64>(in ? wx[i] : -INFINITY, d.gseed, col[j], d.key_hi);
      }
#pragma unroll
      for (int j = 0; j < kIlp; ++j) {
        const bool take = (sc[j] > bv) | ((sc[j] == bv) & (col[j] < bi));
        bv = take ? sc[j] : bv;
        bi = take ? col[j] : bi;
      }
    }
  }
  double bvd = (double)bv;
  block_best<kResWaves>(bvd, bi, s_v, s_i);
  if (threadIdx.x == 0) {
    const int64_t slot = (int64_t)r * p.nchunks + c;
    p.rval[slot] = bvd;
    p.ridx[slot] = bi == 0x7fffffff ? c0 : bi;
  }
}

// ------------------------------------------------------------------ pass 6 ------------

__global__ __launch_bounds__(kThreads) void v2_insert_kernel(V2Params p) {
  const int r = blockIdx.x * kWaves + wave_id();
  if (r >= p.num_reqs) return;
  const int acc = p.acc[r];
  if (acc < 0) {
    if (lane_id() == 0) p.num_sampled[r] = 0;
    return;
  }
  if (lane_id() == 0) p.num_sampled[r] = acc + 1;
  if (p.desc[r].mode == kResampleNone) return;
  const int64_t base = (int64_t)r * p.nchunks;
  double bv = -INFINITY;
  int bc = 0x7fffffff;
  for (int c = lane_id(); c < p.nchunks; c += kWave) {
    double v = p.rval[base + c];
    v = v != v ? -INFINITY : v;
    const bool take = (v > bv) | ((v == bv) & (c < bc));
    bv = take ? v : bv;
    bc = take ? c : bc;
  }
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) {
    const double ov = __shfl_xor(bv, off);
    const int oc = __shfl_xor(bc, off);
    const bool take = (ov > bv) | ((ov == bv) & (oc < bc));
    bv = take ? ov : bv;
    bc = take ? oc : bc;
  }
  if (lane_id() == 0) p.sampled[(int64_t)r * p.sampled_stride + acc] = p.ridx[base + (bc == 0x7fffffff ? 0 : bc)];
}

// ------------------------------------------------------------------ after the call ----

// flatten_sampled (minivllm/worker/gpu/spec_decode/rejection_sampler.py:73-108): one thread
// per logits row i writes flat[i]: sampled[r, i - cu[r]] when request r's rows [cu[r], cu[r+1])
// hold i and i - cu[r] < num_sampled[r], else 0 (the reference zero-fills flat first, so rows
// outside every request's range, such as padding after cu[num_reqs], hold 0 too).
__global__ __launch_bounds__(kThreads) void v2_flatten_kernel(int64_t* flat, const int64_t* sampled,
                                                               int64_t stride, const int32_t* num_sampled,
                                                               const int32_t* cu, int32_t num_reqs,
                                                               int64_t num_logits) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= num_logits) return;
  // last request r with cu[r] <= i (cu is non-decreasing); -1 if none
  int lo = 0, hi = num_reqs;  // answer in [lo - 1, hi)
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if ((int64_t)cu[mid] <= i) lo = mid + 1;
    else hi = mid;
  }
  const int r = lo - 1;
  int64_t v = 0;
  if (r >= 0 && i < (int64_t)cu[r + 1]) {
    const int64_t j = i - cu[r];
    if (j < num_sampled[r] && j < stride) v = sampled[(int64_t)r * stride + j];
  }
  flat[i] = v;
}

// get_num_sampled_and_rejected (minivllm/worker/gpu/input_batch.py:507-553): a request
// still prefilling (seq_len < prefill_len of its state) samples and rejects nothing; else it
// rejects num_logits - num_sampled.
__global__ __launch_bounds__(kThreads) void v2_counts_kernel(int32_t* num_sampled, int32_t* num_rejected,
                                                              const int32_t* seq_lens, const int32_t* cu,
                                                              const int32_t* idx_mapping,
                                                              const int32_t* prefill_len,
                                                              int32_t num_reqs, int32_t num_states) {
  const int r = blockIdx.x * kThreads + threadIdx.x;
  if (r >= num_reqs) return;
  const int st = clamp_state(idx_mapping[r], num_states);
  const bool prefilling = seq_lens[r] < prefill_len[st];
  const int ns = prefilling ? 0 : num_sampled[r];
  num_sampled[r] = ns;
  num_rejected[r] = prefilling ? 0 : (cu[r + 1] - cu[r]) - ns;
}

template <int TDT, int DDT, bool HAS_DRAFT>
hipError_t launch_all(const V2Params& p, hipStream_t stream) {
  if (p.num_logits > 0 && p.K > 0) {
    hipLaunchKernelGGL((v2_stats_kernel<TDT, DDT, HAS_DRAFT>),
                       dim3((unsigned)p.num_logits, p.nchunks), dim3(kThreads), 0, stream, p);
  }
  if (p.num_logits > 0 && p.K > 0) {
    const unsigned rw = (unsigned)((p.num_logits + kWaves - 1) / kWaves);
    hipLaunchKernelGGL((v2_rowstat_kernel<TDT, DDT, HAS_DRAFT>), dim3(rw), dim3(kThreads), 0,
                       stream, p);
    if constexpr (HAS_DRAFT) {
      if (p.use_block)
        hipLaunchKernelGGL((v2_residual_kernel<TDT, DDT>), dim3((unsigned)p.num_logits, p.nchunks),
                           dim3(kThreads), 0, stream, p);
    }
  }
  const unsigned wg = (unsigned)((p.num_reqs + kWaves - 1) / kWaves);
  hipLaunchKernelGGL((v2_chain_kernel<TDT, HAS_DRAFT>), dim3(wg), dim3(kThreads), 0, stream, p);
  if (p.use_fp64)
    hipLaunchKernelGGL((v2_resample_kernel<TDT, DDT, HAS_DRAFT, true>),
                       dim3((unsigned)p.num_reqs, p.nchunks), dim3(kResThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((v2_resample_kernel<TDT, DDT, HAS_DRAFT, false>),
                       dim3((unsigned)p.num_reqs, p.nchunks), dim3(kResThreads), 0, stream, p);
  hipLaunchKernelGGL(v2_insert_kernel, dim3(wg), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

template <int TDT>
hipError_t dispatch_draft(const V2Params& p, int draft_dtype, hipStream_t stream) {
  if (!p.draft) return launch_all<TDT, MVSD_F32, false>(p, stream);
  switch (draft_dtype) {
    case MVSD_F32: return launch_all<TDT, MVSD_F32, true>(p, stream);
    case MVSD_BF16: return launch_all<TDT, MVSD_BF16, true>(p, stream);
    case MVSD_F16: return launch_all<TDT, MVSD_F16, true>(p, stream);
  }
  return hipErrorInvalidValue;
}

inline int64_t align256(int64_t b) { return (b + 255) & ~(int64_t)255; }

}  // namespace
}  // namespace mvsd

extern "C" {

int64_t mvsd_v2_workspace_bytes(int64_t num_logits, int64_t num_reqs, int64_t vocab_size) {
  if (num_logits < 0 || num_reqs < 0 || vocab_size <= 0) return -1;
  const int64_t nch = (vocab_size + mvsd::kV2Chunk - 1) / mvsd::kV2Chunk;
  const int64_t rows = num_logits * nch, reqs = num_reqs * nch;
  return 6 * mvsd::align256(rows * 4) + 5 * mvsd::align256(num_logits * 4) +
         mvsd::align256(num_reqs * 4) + mvsd::align256(num_reqs * 48) + mvsd::align256(reqs * 8) +
         mvsd::align256(reqs * 4);
}

int mvsd_v2_rejection_sample(
    int64_t* sampled, int64_t sampled_stride, int32_t* num_sampled, const void* target_logits,
    int target_dtype, int64_t target_stride, int64_t num_logits, const void* draft_logits,
    int draft_dtype, int64_t draft_stride0, int64_t draft_stride1, const int32_t* draft_sampled,
    const int32_t* cu_num_logits, const int64_t* pos, const int32_t* idx_mapping,
    const int32_t* expanded_idx_mapping, const int32_t* expanded_local_pos,
    const float* temperature, const int64_t* seed, int64_t num_req_states, int64_t num_reqs,
    int64_t vocab_size, int32_t num_speculative_steps, const float* synthetic_conditional_rates,
    int use_fp64, int use_block_verification, void* workspace, int64_t workspace_bytes,
    mvsd_stream_t stream) {
  using namespace mvsd;
  if (num_reqs < 0 || num_logits < 0 || num_speculative_steps < 0) return MVSD_E_INVALID;
  if (num_reqs == 0) return MVSD_OK;
  if (!sampled || !num_sampled || !target_logits || !draft_sampled || !cu_num_logits || !pos ||
      !idx_mapping || !expanded_idx_mapping || !expanded_local_pos || !temperature || !seed ||
      !workspace)
    return MVSD_E_INVALID;
  if (vocab_size <= 0 || num_req_states <= 0 || sampled_stride < num_speculative_steps + 1 ||
      target_stride < vocab_size)
    return MVSD_E_INVALID;
  if (target_dtype != MVSD_F32 && target_dtype != MVSD_BF16 && target_dtype != MVSD_F16)
    return MVSD_E_INVALID;
  if (draft_logits && draft_dtype != MVSD_F32 && draft_dtype != MVSD_BF16 && draft_dtype != MVSD_F16)
    return MVSD_E_INVALID;
  // block verification is incompatible with synthetic acceptance rates (:1043-1045)
  if (use_block_verification && synthetic_conditional_rates) return MVSD_E_INVALID;
  if (draft_logits && (draft_stride1 < vocab_size || draft_stride0 < draft_stride1 * num_speculative_steps))
    return MVSD_E_INVALID;
  if (vocab_size > 0x7fffffff - kV2Chunk || num_reqs > 0x7fffffff || num_req_states > 0x7fffffff ||
      num_logits > 0x7fffffff || num_speculative_steps > 128)
    return MVSD_E_RANGE;
  const int64_t need = mvsd_v2_workspace_bytes(num_logits, num_reqs, vocab_size);
  if (workspace_bytes < need || ((uintptr_t)workspace & 255) != 0) return MVSD_E_WORKSPACE;
  const int nch = (int)((vocab_size + kV2Chunk - 1) / kV2Chunk);
  if (nch > 65535 || (int64_t)nch * num_reqs > 0x7fffffff) return MVSD_E_RANGE;

  V2Params p{};
  p.sampled = sampled;
  p.sampled_stride = sampled_stride;
  p.num_sampled = num_sampled;
  p.target = target_logits;
  p.target_stride = target_stride;
  p.draft = draft_logits;
  p.draft_stride0 = draft_stride0;
  p.draft_stride1 = draft_stride1;
  p.draft_sampled = draft_sampled;
  p.cu_num_logits = cu_num_logits;
  p.pos = pos;
  p.idx_mapping = idx_mapping;
  p.exp_idx_mapping = expanded_idx_mapping;
  p.exp_local_pos = expanded_local_pos;
  p.temperature = temperature;
  p.seed = seed;
  p.rates = synthetic_conditional_rates;
  p.num_logits = num_logits;
  p.num_reqs = (int32_t)num_reqs;
  p.num_states = (int32_t)num_req_states;
  p.vocab = (int32_t)vocab_size;
  p.K = num_speculative_steps;
  p.nchunks = nch;
  p.use_fp64 = use_fp64 != 0;
  p.use_block = use_block_verification != 0;
  const int tsz = target_dtype == MVSD_F32 ? 4 : 2;
  const int dsz = draft_dtype == MVSD_F32 ? 4 : 2;
  p.target_aligned = ((uintptr_t)target_logits % 16 == 0) && ((target_stride * tsz) % 16 == 0);
  p.draft_aligned = draft_logits && ((uintptr_t)draft_logits % 16 == 0) &&
                    ((draft_stride0 * dsz) % 16 == 0) && ((draft_stride1 * dsz) % 16 == 0);
  char* w = static_cast<char*>(workspace);
  const int64_t rows = num_logits * nch, reqs = num_reqs * (int64_t)nch;
  auto take = [&](int64_t bytes) {
    char* q = w;
    w += align256(bytes);
    return q;
  };
  p.tmax = reinterpret_cast<float*>(take(rows * 4));
  p.tsum = reinterpret_cast<float*>(take(rows * 4));
  p.dmax = reinterpret_cast<float*>(take(rows * 4));
  p.dsum = reinterpret_cast<float*>(take(rows * 4));
  p.targ = reinterpret_cast<int32_t*>(take(rows * 4));
  p.rmass = reinterpret_cast<float*>(take(rows * 4));
  p.rtl = reinterpret_cast<float*>(take(num_logits * 4));
  p.rdl = reinterpret_cast<float*>(take(num_logits * 4));
  p.rtlp = reinterpret_cast<float*>(take(num_logits * 4));
  p.rdlp = reinterpret_cast<float*>(take(num_logits * 4));
  p.rarg = reinterpret_cast<int32_t*>(take(num_logits * 4));
  p.acc = reinterpret_cast<int32_t*>(take(num_reqs * 4));
  p.desc = reinterpret_cast<ResampleDesc*>(take(num_reqs * (int64_t)sizeof(ResampleDesc)));
  p.rval = reinterpret_cast<double*>(take(reqs * 8));
  p.ridx = reinterpret_cast<int32_t*>(take(reqs * 4));

  hipError_t err = hipErrorInvalidValue;
  switch (target_dtype) {
    case MVSD_F32: err = dispatch_draft<MVSD_F32>(p, draft_dtype, (hipStream_t)stream); break;
    case MVSD_BF16: err = dispatch_draft<MVSD_BF16>(p, draft_dtype, (hipStream_t)stream); break;
    case MVSD_F16: err = dispatch_draft<MVSD_F16>(p, draft_dtype, (hipStream_t)stream); break;
  }
  return record_hip_error(err);
}

int mvsd_v2_flatten_sampled(int64_t* flat_sampled, const int64_t* sampled, int64_t sampled_stride,
                            const int32_t* num_sampled, const int32_t* cu_num_logits,
                            int64_t num_reqs, int64_t num_logits, mvsd_stream_t stream) {
  using namespace mvsd;
  if (num_reqs < 0 || num_logits < 0 || sampled_stride < 0) return MVSD_E_INVALID;
  if (num_logits == 0) return MVSD_OK;
  if (!flat_sampled || (num_reqs > 0 && (!sampled || !num_sampled || !cu_num_logits)))
    return MVSD_E_INVALID;
  if (num_reqs > 0x7fffffff) return MVSD_E_RANGE;
  if (num_logits > 0x7fffffffLL * kThreads) return MVSD_E_RANGE;
  const unsigned wg = (unsigned)((num_logits + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(v2_flatten_kernel, dim3(wg), dim3(kThreads), 0, (hipStream_t)stream,
                     flat_sampled, sampled, sampled_stride, num_sampled, cu_num_logits,
                     (int32_t)num_reqs, num_logits);
  return record_hip_error(hipGetLastError());
}

int mvsd_v2_num_sampled_and_rejected(int32_t* num_sampled, int32_t* num_rejected,
                                     const int32_t* seq_lens, const int32_t* cu_num_logits,
                                     const int32_t* idx_mapping, const int32_t* prefill_len,
                                     int64_t num_reqs, int64_t num_req_states,
                                     mvsd_stream_t stream) {
  using namespace mvsd;
  if (num_reqs < 0 || num_req_states <= 0) return MVSD_E_INVALID;
  if (num_reqs == 0) return MVSD_OK;
  if (!num_sampled || !num_rejected || !seq_lens || !cu_num_logits || !idx_mapping || !prefill_len)
    return MVSD_E_INVALID;
  if (num_reqs > 0x7fffffff || num_req_states > 0x7fffffff) return MVSD_E_RANGE;
  const unsigned wg = (unsigned)((num_reqs + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(v2_counts_kernel, dim3(wg), dim3(kThreads), 0, (hipStream_t)stream,
                     num_sampled, num_rejected, seq_lens, cu_num_logits, idx_mapping, prefill_len,
                     (int32_t)num_reqs, (int32_t)num_req_states);
  return record_hip_error(hipGetLastError());
}

}  // extern "C"
