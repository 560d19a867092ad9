// Fused rejection sampling for one speculative-decoding verification step.
//
// What it computes (reference: minivllm/sample/rejection_sampler.py:414-534 and the three
// Triton kernels at :678-740, :744-822, :850-928), per request r with K_r draft rows:
//   greedy r : out[r, j] = argmax(target row j) for the accepted prefix and the first
//              mismatch; bonus appended when every draft matches.
//   random r : p = softmax(target / T_r); accept draft d at row j iff q[d] > 0 and
//              p[d] / q[d] >= u_j (fp32 ratio compared in fp64); on the first rejection
//              write the recovered id argmax_v max(p_v - q_v, 0) * (1 / E[r, v]) and stop;
//              bonus appended when all are accepted.
//
// How (one persistent launch, every input byte read once):
//   * A task is (row group, vocab chunk): up to G rows of one request and CHUNK columns.
//     Tasks are handed out by an atomic ticket in group-major order, so the NC chunk
//     tasks of a group hold consecutive tickets.
//   * Phase 1 loads the group's target slice into registers, reduces a per-chunk
//     (max, sumexp) for each row and publishes it into that row's stats slot.  Random rows
//     then wait until all NC slots of their rows are written; the tasks writing them were
//     claimed earlier (or are being claimed by running workgroups), never wait before
//     publishing, and therefore finish: the wait cannot deadlock.  A spin bound still ends
//     every wave.  The request's noise chunk is loaded before the wait and the first draft
//     chunk right after it, so the wait overlaps with HBM traffic.
//   * Phase 2 combines the NC partials into the row's (M, S) and scores
//     p_v = e_v * exp(m_c - M) / S straight from the registers, keeping a chunk-local argmax
//     that goes into the row's argmax slot.
//   * The last task to finish a request reduces the argmax slots, decides every position in
//     parallel, writes [B, max_spec_len + 1] and clears the request's slots and counter.
//   * Slots are 64-bit values exchanged with relaxed agent-scope atomics; 0 means empty and
//     no written slot is 0, so readers poll the data itself and no fence (no L2 write-back or
//     invalidation) is needed.  Every call leaves the workspace zeroed for the next one.
//
// Full, 16-byte-aligned chunks take a fast path with unconditional vector loads (all of a
// task's loads in flight together); the last chunk of a row and unaligned rows take a
// bounds-checked path.
#include <float.h>
#include <stdlib.h>

#include <type_traits>

#include "mvsd_device.h"
#include "verify.h"

namespace mvsd {

// Polls before a wait gives up and sets the sticky flag (ctrl[1]); with a poll every ~1-2 us
// this is a fraction of a second, far beyond any wait of a healthy run.
constexpr int kSpinLimit = 1 << 18;

// Request r's verify rows [begin, begin + K), clamped so that inconsistent metadata can
// produce wrong tokens but never an out-of-bounds access: 0 <= begin <= begin + K <= P and
// K <= max_spec_len.
__device__ inline void req_range(const VerifyParams& p, int r, int& begin, int& K) {
  int b = r == 0 ? 0 : p.cu[r - 1];
  int e = p.cu[r];
  b = min(max(b, 0), p.P);
  e = min(max(e, b), p.P);
  begin = b;
  K = min(e - b, p.max_spec_len);
}

// log2(e) / T rounded once from double.
__device__ inline float exp2_scale(float temp) {
  return (float)(1.4426950408889634074 / (double)temp);
}

// Group descriptor flags.
constexpr int kGreedy = 1;
constexpr int kFull = 2;  // random request whose recovered ids come from in-kernel scores

// Per-request metadata in LDS: first verify row, rows (clamped as by req_range) with the group
// flags above bit 16, and log2(e) / T.
struct RequestMeta {
  int* begin;
  int* kflags;
  float* c1;
};

// ------------------------------------------------------------------ loads ------------
// Column of element k of this thread in the sub-chunk starting at v0: 16-byte vectors of kVec
// elements, consecutive lanes on consecutive vectors.
template <int DT, int EPT>
__device__ inline int elem_index(int64_t v0, int k) {
  constexpr int VEC = Elem<DT>::kVec;
  return (int)(v0 + ((int64_t)(k / VEC) * kVThreads + threadIdx.x) * VEC + (k % VEC));
}

// ------------------------------------------------------------------ init kernel ------
// One 1024-thread block: fill the output with -1 (bonus in column 0 for requests without
// drafts) and exclusive-scan the per-request group counts.  Everything else in the workspace
// is already zero (every call clears what it used); the spin-limit flag ctrl[1] is sticky
// so that a timed-out call stays detectable.
__global__ __launch_bounds__(1024) void verify_init_kernel(VerifyParams p) {
  const int tid = threadIdx.x;
  const int width = p.max_spec_len + 1;
  const int64_t n_out = (int64_t)p.B * width;
  for (int64_t i = tid; i < n_out; i += 1024) {
    const int r = (int)(i / width);
    const int col = (int)(i - (int64_t)r * width);
    int v = -1;
    if (col == 0) {
      int b, k;
      req_range(p, r, b, k);
      if (k == 0) v = p.bonus[r];
    }
    p.out[(int64_t)r * p.out_stride + col] = v;
  }
  __shared__ int s_scan[1024];
  __shared__ int s_carry;
  if (tid == 0) s_carry = 0;
  __syncthreads();
  for (int base = 0; base < p.B; base += 1024) {
    const int r = base + tid;
    int b = 0, k = 0;
    if (r < p.B) req_range(p, r, b, k);
    const int ng = (k + p.G - 1) / p.G;
    s_scan[tid] = ng;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int add = tid >= off ? s_scan[tid - off] : 0;
      __syncthreads();
      s_scan[tid] += add;
      __syncthreads();
    }
    const int carry = s_carry;
    if (r < p.B) {
      const int first = carry + s_scan[tid] - ng;
      p.grp_off[r] = first;
      if (ng > 0) {
        const bool greedy = req_is_greedy(p, r);
        const int flags = (greedy ? kGreedy : 0) | (!greedy && !p.recovered ? kFull : 0);
        const int c1 = __float_as_int(exp2_scale(req_temperature(p, r)));
        for (int g = 0; g < ng; ++g)
          p.grp_desc[first + g] = make_int4(
              r, b + g * p.G, min(p.G, k - g * p.G) | ng << 8 | flags << 16 | g << 24, c1);
      }
    }
    __syncthreads();
    if (tid == 1023) s_carry = carry + s_scan[1023];
    __syncthreads();
  }
  if (tid == 0) p.grp_off[p.B] = s_carry;
  __syncthreads();

  // Queue lists: queue q holds the groups of requests q, q + nq, ... in request order.  One
  // queue is the identity list and is not materialised.
  if (p.nq == 1) {
    if (tid == 0) {
      p.qcount[0] = s_carry;
      p.qoff[0] = 0;
    }
    return;
  }
  __shared__ int s_qoff;
  if (tid == 0) s_qoff = 0;
  __syncthreads();
  for (int q = 0; q < p.nq; ++q) {
    if (tid == 0) {
      s_carry = 0;
      p.qoff[q] = s_qoff;
    }
    __syncthreads();
    for (int base = q; base < p.B; base += 1024 * p.nq) {
      const int r = base + tid * p.nq;
      const int ng = r < p.B ? p.grp_off[r + 1] - p.grp_off[r] : 0;
      s_scan[tid] = ng;
      __syncthreads();
      for (int off = 1; off < 1024; off <<= 1) {
        const int add = tid >= off ? s_scan[tid - off] : 0;
        __syncthreads();
        s_scan[tid] += add;
        __syncthreads();
      }
      const int lo = s_qoff + s_carry + s_scan[tid] - ng;
      for (int j = 0; j < ng; ++j) p.qgi[lo + j] = p.grp_off[r] + j;
      __syncthreads();
      if (tid == 1023) s_carry += s_scan[1023];
      __syncthreads();
    }
    if (tid == 0) {
      p.qcount[q] = s_carry;
      s_qoff += s_carry;
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ row statistics ---
// Softmax statistics travel as (raw chunk max mx, sum of exp2((x - mx) * c1)) with
// c1 = log2(e) / T: for T > 0 the max of x / T is the max of x divided by T, so no per-element
// division is needed, and p = exp((x - MX) / T) / S = exp2(fma(x - MX, c1, -log2 S)).

// One wavefront: wait until the n stats slots of a row are written, then combine them into
// the row's raw max MX and S = sum_c s_c * 2^((mx_c - MX) * c1).  Up to 4 * 64 slots are kept
// in registers from the last poll.
__device__ inline bool wave_row_stats(const uint64_t* slots, int n, float c1, const int* abort,
                                      float& MX, float& S) {
  const int lane = lane_id();
  constexpr int R = 4;
  uint64_t v[R];
  bool ok = true;
  for (int spins = 0;; ++spins) {
    int ready = 1;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int c = lane + j * kWave;
      v[j] = c < n ? slot_load(slots + c) : 0;
      ready &= (c >= n) | (v[j] != 0);
    }
    for (int c = lane + R * kWave; c < n; c += kWave) ready &= slot_load(slots + c) != 0;
    if (__all(ready)) break;
    if (spins >= kSpinLimit || ((spins & 255) == 255 && atomic_load_relaxed(abort) != 0)) {
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (lane + j * kWave < n) m = fmaxf(m, unpack_stats(v[j]).x);
  for (int c = lane + R * kWave; c < n; c += kWave) m = fmaxf(m, unpack_stats(slot_load(slots + c)).x);
  MX = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const float2 st = unpack_stats(v[j]);
    if (lane + j * kWave < n && st.x != -INFINITY) s += st.y * exp2f((st.x - MX) * c1);
  }
  for (int c = lane + R * kWave; c < n; c += kWave) {
    const float2 st = unpack_stats(slot_load(slots + c));
    if (st.x != -INFINITY) s += st.y * exp2f((st.x - MX) * c1);
  }
  S = wave_sum(s);
  return ok;
}

// ------------------------------------------------------------------ finalisation -----
// The finalisation is latency-bound (a few dependent memory round trips, nothing else in
// flight for its workgroup), so it overlaps them: each position's decision inputs load while
// the waves poll the rows' slots, and one poll covers both slot sets of a row.
struct FinalizeSmem {
  int tok[kMaxSpecLen];
  float M[kMaxSpecLen];
  float S[kMaxSpecLen];
  int out_tok[kMaxSpecLen];
  int first[2];
};

constexpr int kKeep = 2;  // slots per lane kept from the last poll (rows of up to 128 slots)

// One wave: wait until verify row `row`'s slots are written (its na arg slots when the row
// needs an argmax, its nc stats slots when it is random), then reduce and clear them.  tok:
// the argmax (greedy rows and in-kernel recovered ids; untouched otherwise); M, S: the
// statistics (random rows).
__device__ inline void finalize_row(const VerifyParams& p, int r, int64_t row, bool greedy,
                                    bool full, int na, int& tok, float& M, float& S) {
  const int lane = lane_id();
  const int nc = p.nc;
  uint64_t* aslots = p.arg_slots + row * p.arg_stride;
  uint64_t* sslots = p.stat_slots + row * nc;
  const int nA = (greedy || full) ? na : 0;
  const int nS = greedy ? 0 : nc;
  uint64_t av[kKeep], sv[kKeep];
  for (int spins = 0;; ++spins) {
    int ready = 1;
#pragma unroll
    for (int j = 0; j < kKeep; ++j) {
      const int c = lane + j * kWave;
      av[j] = c < nA ? slot_load(aslots + c) : 0;
      sv[j] = c < nS ? slot_load(sslots + c) : 0;
      ready &= (c >= nA || av[j] != 0) & (c >= nS || sv[j] != 0);
    }
    for (int c = lane + kKeep * kWave; c < nA; c += kWave) ready &= slot_load(aslots + c) != 0;
    for (int c = lane + kKeep * kWave; c < nS; c += kWave) ready &= slot_load(sslots + c) != 0;
    if (__all(ready)) break;
    if (spins >= kSpinLimit || ((spins & 255) == 255 && atomic_load_relaxed(&p.ctrl[1]) != 0)) {
      if (lane == 0) atomic_store_relaxed(&p.ctrl[1], 1);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (nA > 0) {
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < kKeep; ++j) best = av[j] > best ? av[j] : best;
    for (int c = lane + kKeep * kWave; c < nA; c += kWave) {
      const uint64_t k = slot_load(aslots + c);
      best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    tok = min(max(key_index(best), 0), p.V - 1);
    for (int c = lane; c < nA; c += kWave) slot_store(aslots + c, 0);
  }
  M = 0.f;
  S = 1.f;
  if (nS > 0) {
    // (raw max MX, S = sum_c s_c * 2^((mx_c - MX) * c1)), as in wave_row_stats
    const float c1 = exp2_scale(req_temperature(p, r));
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kKeep; ++j)
      if (lane + j * kWave < nS) m = fmaxf(m, unpack_stats(sv[j]).x);
    for (int c = lane + kKeep * kWave; c < nS; c += kWave) m = fmaxf(m, unpack_stats(slot_load(sslots + c)).x);
    M = wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < kKeep; ++j) {
      const float2 st = unpack_stats(sv[j]);
      if (lane + j * kWave < nS && st.x != -INFINITY) sum += st.y * exp2f((st.x - M) * c1);
    }
    for (int c = lane + kKeep * kWave; c < nS; c += kWave) {
      const float2 st = unpack_stats(slot_load(sslots + c));
      if (st.x != -INFINITY) sum += st.y * exp2f((st.x - M) * c1);
    }
    S = wave_sum(sum);
    for (int c = lane; c < nS; c += kWave) slot_store(sslots + c, 0);
  }
}

// Arg slots of a verify row: 2 * nc (4 * nc) for rows of groups scored in half (quarter)
// chunks.
__device__ inline int row_arg_slots(const VerifyParams& p, const int* goff, bool full, int gfirst,
                                    int k) {
  if (!(p.split && full)) return p.nc;
  const int li = gfirst + k / p.G;
  if (li >= goff[p.B] - p.quarter) return 4 * p.nc;
  return li >= goff[p.B] - p.lag ? 2 * p.nc : p.nc;
}

// Inputs of one position's decision: the draft id and uniform, and for a random row q[d],
// the target logit x[d], the row mask and the supplied recovered id.
struct PosInputs {
  int d;
  double u;
  float q;
  float x;
  float4 mk;
  int rec;
};

__device__ inline PosInputs load_position(const VerifyParams& p, bool greedy, int64_t row) {
  PosInputs in;
  in.d = p.draft_ids[row];
  in.u = 0.0;
  in.q = 1.f;
  in.x = 0.f;
  in.mk = make_float4(-INFINITY, -INFINITY, __int_as_float(-1), 0.f);
  in.rec = 0;
  const bool synthetic = p.synth != nullptr;
  if (!greedy || synthetic) in.u = p.uniforms[row];
  if (!greedy && !synthetic && in.d >= 0 && in.d < p.V) {
    if (p.draft) in.q = p.draft[row * p.draft_stride + in.d];
    const int64_t trow = target_row(p, (int)row);
    if (p.target_dtype == MVSD_F32) {
      in.x = static_cast<const float*>(p.target)[trow * p.target_stride + in.d];
    } else if (p.target_dtype == MVSD_BF16) {
      in.x = Elem<MVSD_BF16>::cvt(static_cast<const uint16_t*>(p.target)[trow * p.target_stride + in.d]);
    } else {
      in.x = Elem<MVSD_F16>::cvt(static_cast<const _Float16*>(p.target)[trow * p.target_stride + in.d]);
    }
    if (p.masks) in.mk = p.masks[row];
  }
  if (!greedy && p.recovered) in.rec = p.recovered[row];
  return in;
}

// Accept / reject decision at position pos of request r, given the row's argmax or recovered
// id tok and statistics (M, S).
__device__ inline void decide_position(const VerifyParams& p, int r, bool greedy, int pos,
                                       const PosInputs& in, int tok, float M, float S,
                                       bool& accepted, int& token) {
  const bool synthetic = p.synth != nullptr;
  const int d = in.d;
  if (greedy) {
    // rejection_sampler.py:715-732
    if (synthetic) {
      accepted = in.u < (double)p.synth[pos] && d >= 0;
      token = accepted ? d : tok;
    } else {
      token = tok;
      accepted = d == token;
    }
    return;
  }
  // rejection_sampler.py:782-814
  if (d < 0) {
    accepted = false;
  } else if (synthetic) {
    accepted = in.u < (double)p.synth[pos];
  } else if (d >= p.V) {
    accepted = false;  // the reference would index out of bounds here
  } else {
    const float temp = req_temperature(p, r);
    float pd = expf(in.x / temp - M / temp) / S;
    if (p.masks && row_masked(in.mk, in.x, d)) pd = 0.f;  // -inf after the constraints
    accepted = in.q > 0.f && (double)(pd / in.q) >= in.u;
  }
  token = accepted ? d : tok;
}

// Executed by the whole block that completed request r's last task.  goff: the requests'
// first group indices (global or LDS).  Writes the request's whole output row.
__device__ void finalize_request(const VerifyParams& p, const int* goff, int r, bool greedy,
                                 bool full, FinalizeSmem& sm) {
  int begin, K;
  req_range(p, r, begin, K);
  const int gfirst = goff[r];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  // thread pos < K (K <= kMaxSpecLen <= kVThreads) owns position pos; its inputs load while
  // the waves reduce the rows' slots
  PosInputs in;
  if (tid < K) in = load_position(p, greedy, begin + tid);
  for (int k = wave_id(); k < K; k += kVWaves) {
    int tok = 0;
    float M, S;
    finalize_row(p, r, begin + k, greedy, full, row_arg_slots(p, goff, full, gfirst, k), tok, M, S);
    if (lane == 0) {
      sm.tok[k] = tok;
      sm.M[k] = M;
      sm.S[k] = S;
    }
  }
  if (tid == 0) atomic_store_relaxed(&p.req_cnt[r], 0);
  __syncthreads();

  // every position's decision in parallel; the chain keeps the prefix up to the first reject
  bool accepted = true;
  if (tid < K) {
    int token;
    const int tok = (greedy || full) ? sm.tok[tid] : in.rec;
    decide_position(p, r, greedy, tid, in, tok, sm.M[tid], sm.S[tid], accepted, token);
    sm.out_tok[tid] = token;
  }
  static_assert(kMaxSpecLen <= 2 * kWave && kVWaves >= 2, "positions live in waves 0 and 1");
  if (wave_id() < 2) {
    const unsigned long long rej = __ballot(tid < K && !accepted);
    if (lane == 0) sm.first[wave_id()] = rej ? wave_id() * kWave + __builtin_ctzll(rej) : K;
  }
  __syncthreads();
  const int first = min(sm.first[0], sm.first[1]);
  int32_t* out = p.out + (int64_t)r * p.out_stride;
  for (int pos = tid; pos <= p.max_spec_len; pos += kVThreads) {
    int v = -1;
    if (pos < K && pos <= first) v = sm.out_tok[pos];
    else if (pos == K && first == K) v = p.bonus[r];
    out[pos] = v;
  }
}

// ------------------------------------------------------------------ tasks ------------

// A task covers rows [row0, row0 + nrows) of one group and columns [v0, vend), walked in
// sub-chunks of kVThreads * EPT columns.  Full, aligned sub-chunks are double-buffered: the
// loads of sub-chunk j + 1 are issued before sub-chunk j is reduced, so a workgroup keeps HBM
// requests in flight for the whole task.  Buffers hold the raw 16-byte vectors; elements are
// converted to fp32 only when they are consumed.

template <bool F>
using Fast = std::integral_constant<bool, F>;

// Element k (0 <= k < EPT) of a DT row buffer, as fp32.
template <int DT>
__device__ inline float raw_elem(const u32x4* raw, int k) {
  using S = typename Elem<DT>::storage;
  constexpr int VEC = Elem<DT>::kVec;
  const S* s = reinterpret_cast<const S*>(&raw[k / VEC]);
  return Elem<DT>::cvt(s[k % VEC]);
}

// Element k of an fp32 buffer laid out like a DT row (the 4-element vector k / 4 holds
// elements 4 (k / 4) .. 4 (k / 4) + 3 for every DT, since kVec is a multiple of 4).
__device__ inline float raw_f32(const u32x4* raw, int k) { return __uint_as_float(raw[k / 4][k % 4]); }

// Column of the first element of 16-byte vector i of this thread (DT layout).
template <int DT>
__device__ inline int64_t vec_col(int64_t s0, int i) {
  constexpr int VEC = Elem<DT>::kVec;
  return s0 + ((int64_t)i * kVThreads + threadIdx.x) * VEC;
}

// Target loads.  The stats tasks' loads are temporal so that the lines stay cached for the
// score tasks' re-read of the same chunk (MVSD_VERIFY_NT_STATS=1 makes them non-temporal);
// the score tasks' loads (MVSD_VERIFY_NT_SCORES) and the single-read kernel's are the last
// use and stream non-temporally.
#ifndef MVSD_VERIFY_NT_STATS
#define MVSD_VERIFY_NT_STATS 0
#endif
#ifndef MVSD_VERIFY_NT_SCORES
#define MVSD_VERIFY_NT_SCORES 1
#endif
template <bool NT>
__device__ inline u32x4 load_target16(const void* p) {
  const u32x4* q = static_cast<const u32x4*>(p);
  if constexpr (NT) return __builtin_nontemporal_load(q);
  else return *q;
}

// DT row sub-chunk, full and aligned.
__device__ inline uint32_t bits16(uint16_t v) { return v; }
__device__ inline uint32_t bits16(_Float16 v) { return __builtin_bit_cast(uint16_t, v); }

// The 16-byte vector of DT entries at col, entries at or past vend replaced by fill; packed in
// registers (no local array).
template <int DT>
__device__ inline u32x4 load_vec_checked(const typename Elem<DT>::storage* __restrict__ base,
                                         int64_t col, int64_t vend,
                                         typename Elem<DT>::storage fill) {
  u32x4 v;
  if constexpr (Elem<DT>::kVec == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = __float_as_uint(col + j < vend ? base[col + j] : fill);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = bits16(col + 2 * j < vend ? base[col + 2 * j] : fill);
      const uint32_t hi = bits16(col + 2 * j + 1 < vend ? base[col + 2 * j + 1] : fill);
      v[j] = lo | hi << 16;
    }
  }
  return v;
}

template <int DT, int EPT, bool NT>
__device__ inline void load_raw(const typename Elem<DT>::storage* __restrict__ base, int64_t s0,
                                u32x4 (&out)[EPT / Elem<DT>::kVec]) {
#pragma unroll
  for (int i = 0; i < EPT / Elem<DT>::kVec; ++i)
    out[i] = load_target16<NT>(base + vec_col<DT>(s0, i));
}

// DT row sub-chunk, bounds-checked: elements at or beyond vend read as `fill`.
template <int DT, int EPT, bool NT>
__device__ inline void load_raw_checked(const typename Elem<DT>::storage* __restrict__ base,
                                        int64_t s0, int64_t vend, bool aligned,
                                        typename Elem<DT>::storage fill,
                                        u32x4 (&out)[EPT / Elem<DT>::kVec]) {
  using S = typename Elem<DT>::storage;
  constexpr int VEC = Elem<DT>::kVec;
#pragma unroll
  for (int i = 0; i < EPT / VEC; ++i) {
    const int64_t col = vec_col<DT>(s0, i);
    if (aligned && col + VEC <= vend) out[i] = load_target16<NT>(base + col);
    else out[i] = load_vec_checked<DT>(base, col, vend, fill);
  }
}

// fp32 row sub-chunk in DT layout; FAST: full and aligned, else bounds-checked with `fill`.
template <int DT, int EPT, bool FAST>
__device__ inline void load_raw_f32(const float* __restrict__ base, int64_t s0, int64_t vend,
                                    bool aligned, float fill, u32x4 (&out)[EPT / 4]) {
  constexpr int VEC = Elem<DT>::kVec;
#pragma unroll
  for (int m = 0; m < EPT / 4; ++m) {
    const int64_t col = vec_col<DT>(s0, m / (VEC / 4)) + (m % (VEC / 4)) * 4;
    if (FAST || (aligned && col + 4 <= vend))
      out[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + col));
    else
      out[m] = load_vec_checked<MVSD_F32>(base, col, vend, fill);
  }
}

// Walk [v0, vend) in SUB-column sub-chunks: load(buf, s0, Fast<bool>) issues a sub-chunk's
// loads, body(buf, s0, Fast<bool>) consumes them.  hook() runs once, after the first loads
// are issued.  Unaligned inputs and the partial last sub-chunk take the checked path.
// The loads of the next MVSD_VERIFY_DEPTH - 1 sub-chunks are issued unconditionally (past the
// end of the run they reload the final sub-chunk, an L2 hit): every path then issues the same
// loads, so the compiler's in-order load counter lets body(j) wait for sub-chunk j alone while
// the following ones are in flight.
#ifndef MVSD_VERIFY_DEPTH
#define MVSD_VERIFY_DEPTH 2
#endif
template <int SUB, typename Buf, typename Load, typename Body, typename Hook>
__device__ inline void pipeline(int64_t v0, int64_t vend, bool aligned, Load&& load, Body&& body,
                                Hook&& hook) {
  const int nfull = aligned ? (int)((vend - v0) / SUB) : 0;
  auto at = [&](int j) { return v0 + (int64_t)min(j, nfull - 1) * SUB; };
  if (nfull > 0) {
    if constexpr (MVSD_VERIFY_DEPTH >= 3) {  // sub-chunks j+1 and j+2 in flight during body(j)
      Buf a, b, c;
      load(a, at(0), Fast<true>());
      load(b, at(1), Fast<true>());
      hook();
      for (int j = 0;;) {
        load(c, at(j + 2), Fast<true>());
        body(a, v0 + (int64_t)j * SUB, Fast<true>());
        if (++j == nfull) break;
        load(a, at(j + 2), Fast<true>());
        body(b, v0 + (int64_t)j * SUB, Fast<true>());
        if (++j == nfull) break;
        load(b, at(j + 2), Fast<true>());
        body(c, v0 + (int64_t)j * SUB, Fast<true>());
        if (++j == nfull) break;
      }
    } else {
      // Sub-chunks 0 and 1 are both in flight before the hook (which may wait for the
      // group's statistics); afterwards a buffer is reloaded with sub-chunk j + 2 as soon as
      // sub-chunk j has been consumed.
      Buf a, b;
      load(a, at(0), Fast<true>());
      hook();
      for (int j = 0;;) {
        load(b, at(j + 1), Fast<true>());
        body(a, v0 + (int64_t)j * SUB, Fast<true>());
        if (++j == nfull) break;
        load(a, at(j + 1), Fast<true>());
        body(b, v0 + (int64_t)j * SUB, Fast<true>());
        if (++j == nfull) break;
      }
    }
  } else {
    hook();
  }
  for (int64_t s0 = v0 + (int64_t)nfull * SUB; s0 < vend; s0 += SUB) {
    Buf t;
    load(t, s0, Fast<false>());
    body(t, s0, Fast<false>());
  }
}

// Base pointers of the group's target rows (rows past nrows repeat the last one).
template <int DT, int G>
__device__ inline void target_bases(const VerifyParams& p, int row0, int nrows,
                                    const typename Elem<DT>::storage* (&tb)[G]) {
  using S = typename Elem<DT>::storage;
#pragma unroll
  for (int g = 0; g < G; ++g)
    tb[g] = static_cast<const S*>(p.target) + target_row(p, row0 + min(g, nrows - 1)) * p.target_stride;
}

template <int DT, int EPT, int G>
struct TargetBuf {
  u32x4 x[G][EPT / Elem<DT>::kVec];
};

template <int DT, int EPT, int G>
struct ScoreBuf {
  u32x4 x[G][EPT / Elem<DT>::kVec];
  u32x4 q[G][EPT / 4];
  u32x4 e[EPT / 4];
};

// Value of a per-row register array for row = this thread's index (threads < G).
template <int G, typename T>
__device__ inline T row_of_thread(const T (&a)[G]) {
  T v = a[0];
#pragma unroll
  for (int g = 1; g < G; ++g) v = (int)threadIdx.x == g ? a[g] : v;
  return v;
}

template <int DT, int EPT, int G>
__device__ inline auto target_loader(const VerifyParams& p, const typename Elem<DT>::storage* (&tb)[G],
                                     int nrows, int64_t vend) {
  // every row slot loads (rows past nrows repeat the last row), so every path issues the
  // same loads
  return [&p, &tb, vend](TargetBuf<DT, EPT, G>& buf, int64_t s0, auto fast) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if constexpr (decltype(fast)::value)
        load_raw<DT, EPT, MVSD_VERIFY_NT_STATS>(tb[g], s0, buf.x[g]);
      else
        load_raw_checked<DT, EPT, MVSD_VERIFY_NT_STATS>(tb[g], s0, vend, p.target_aligned,
                                                        Elem<DT>::ninf(), buf.x[g]);
    }
  };
}

// Row masks of the group's rows (rows past nrows repeat the last row).
template <bool MASKED, int G>
__device__ inline void row_masks(const VerifyParams& p, int row0, int nrows, float4 (&mk)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g)
    mk[g] = MASKED ? p.masks[row0 + min(g, nrows - 1)] : make_float4(0.f, 0.f, 0.f, 0.f);
}

// Greedy task: chunk-local argmax of the raw logits (NaN first, lowest index wins); with
// MASKED, entries masked by the row's sampling constraints count as -inf.
template <int DT, int EPT, int G, bool MASKED, typename Hook>
__device__ inline void task_argmax(const VerifyParams& p, int c, int row0, int nrows, int64_t v0,
                                   int64_t vend, uint64_t* s_key, Hook&& after_loads) {
  using S = typename Elem<DT>::storage;
  const S* tb[G];
  target_bases<DT, G>(p, row0, nrows, tb);
  float4 mk[G];
  row_masks<MASKED, G>(p, row0, nrows, mk);
  float bv[G];
  int bi[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    bv[g] = -INFINITY;
    bi[g] = (int)v0;
  }
  auto body = [&](const TargetBuf<DT, EPT, G>& buf, int64_t s0, auto fast) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g < nrows) {
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          const int idx = elem_index<DT, EPT>(s0, k);
          float v = raw_elem<DT>(buf.x[g], k);
          if constexpr (MASKED) v = row_masked(mk[g], v, idx) ? -INFINITY : v;
          // columns rise with s0 and k: a strict compare keeps the first maximum; NaN wins
          const bool take = ((v > bv[g]) | ((v != v) & (bv[g] == bv[g]))) &
                            (decltype(fast)::value || idx < vend);
          bv[g] = take ? v : bv[g];
          bi[g] = take ? idx : bi[g];
        }
      }
    }
  };
  pipeline<kVThreads * EPT, TargetBuf<DT, EPT, G>>(v0, vend, p.target_aligned,
                                                   target_loader<DT, EPT, G>(p, tb, nrows, vend),
                                                   body, after_loads);
  uint64_t key[G];
#pragma unroll
  for (int g = 0; g < G; ++g) key[g] = argmax_key(bv[g], bi[g]);
  const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_key);
  if ((int)threadIdx.x < nrows) slot_store(p.arg_slots + (int64_t)(row0 + threadIdx.x) * p.arg_stride + c, best);
}

// A-task: per row of the group, the chunk's raw max mx and sum of exp2((x - mx) * c1), kept
// online per thread (the running sum is rescaled when the thread's max grows).  With MASKED,
// entries masked by the row's sampling constraints add nothing to the sum; the maximum still
// runs over every entry, which only moves the reference point of the exponentials (the
// largest value of a row is never masked).
// With PARK, every thread also stores its raw target vectors of sub-chunk j (counted from v0)
// at park[((j * G + g) * NV + i) * kVThreads + thread] in LDS, for the scores of the same task.
template <int DT, int EPT, int G, bool MASKED, bool PARK = false, typename Hook>
__device__ inline void task_stats(const VerifyParams& p, int c, float c1, int row0, int nrows,
                                  int64_t v0, int64_t vend, float* s_red, float* s_M,
                                  Hook&& after_loads, u32x4* park = nullptr) {
  using S = typename Elem<DT>::storage;
  const S* tb[G];
  target_bases<DT, G>(p, row0, nrows, tb);
  float4 mk[G];
  row_masks<MASKED, G>(p, row0, nrows, mk);
  float m[G], s[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    s[g] = 0.f;
  }
  auto body = [&](const TargetBuf<DT, EPT, G>& buf, int64_t s0, auto) {
    if constexpr (PARK) {
      constexpr int NV = EPT / Elem<DT>::kVec;
      const int j = (int)((s0 - v0) / (kVThreads * EPT));
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < NV; ++i) park[((j * G + g) * NV + i) * kVThreads + threadIdx.x] = buf.x[g][i];
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g < nrows) {
        float x[EPT];
        float lm = -INFINITY;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          x[k] = raw_elem<DT>(buf.x[g], k);
          lm = fmaxf(lm, x[k]);
        }
        if (lm > m[g]) {  // m = -inf: the old sum is 0 and exp2(-inf) = 0
          s[g] *= __builtin_amdgcn_exp2f((m[g] - lm) * c1);
          m[g] = lm;
        }
        const float ref = m[g] == -INFINITY ? 0.f : m[g];
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          const float e = __builtin_amdgcn_exp2f((x[k] - ref) * c1);
          if constexpr (MASKED) acc += row_masked(mk[g], x[k], elem_index<DT, EPT>(s0, k)) ? 0.f : e;
          else acc += e;
        }
        s[g] += acc;
      }
    }
  };
  pipeline<kVThreads * EPT, TargetBuf<DT, EPT, G>>(v0, vend, p.target_aligned,
                                                   target_loader<DT, EPT, G>(p, tb, nrows, vend),
                                                   body, after_loads);
  float M[G];
#pragma unroll
  for (int g = 0; g < G; ++g) M[g] = m[g];
  block_max<G, kVWaves>(M, s_red);
#pragma unroll
  for (int g = 0; g < G; ++g)
    s[g] = m[g] == -INFINITY ? 0.f : s[g] * __builtin_amdgcn_exp2f((m[g] - M[g]) * c1);
  // row maxima for the row threads through LDS (ordered by the barrier of the sum below), so
  // that no thread indexes the register array M by its thread index
  if (threadIdx.x == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) s_M[g] = M[g];
  }
  const float srow = block_sum_to_row_thread<G, kVWaves>(s, s_red);
  if ((int)threadIdx.x < nrows) {
    const float mrow = s_M[threadIdx.x];
    slot_store(p.stat_slots + (int64_t)(row0 + threadIdx.x) * p.nc + c,
               pack_stats(mrow, mrow == -INFINITY ? 0.f : srow));
  }
}

// B-task: per row of the group, the chunk-local argmax of max(p - q, 0) * (1 / E).  The
// group's stats were published by A-tasks holding lower tickets; the wait for them overlaps
// with the first sub-chunk's loads.
// With PARKED the target comes from the LDS copy task_stats<..., PARK> made of the same
// chunk (each thread reads back its own vectors), and after_loads runs once the wait for the
// group's statistics is over instead of before it.
template <int DT, int EPT, int G, bool HAS_DRAFT, bool MASKED, bool PARKED = false, typename Hook>
__device__ inline void task_scores(const VerifyParams& p, int c, int r, float c1, int row0,
                                   int nrows, int64_t v0, int64_t vend, uint64_t* s_key,
                                   float* s_M, float* s_L, Hook&& after_loads,
                                   const u32x4* park = nullptr) {
  using S = typename Elem<DT>::storage;
  using Buf = ScoreBuf<DT, EPT, G>;
  const S* tb[G];
  target_bases<DT, G>(p, row0, nrows, tb);
  float4 mk[G];
  row_masks<MASKED, G>(p, row0, nrows, mk);
  const float* qb[G];
  int d[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int row = row0 + min(g, nrows - 1);
    qb[g] = HAS_DRAFT ? p.draft + (int64_t)row * p.draft_stride : nullptr;
    d[g] = HAS_DRAFT ? -1 : p.draft_ids[row];
  }
  const float* eb = p.noise + (int64_t)r * p.noise_stride;
  const bool aligned = p.target_aligned && p.noise_aligned && (p.draft_aligned || !HAS_DRAFT);

  // every row slot loads (rows past nrows repeat the last row): one load sequence on every path
  auto load = [&](Buf& buf, int64_t s0, auto fast) {
    constexpr bool F = decltype(fast)::value;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if constexpr (PARKED)
        ;
      else if constexpr (F)
        load_raw<DT, EPT, MVSD_VERIFY_NT_SCORES>(tb[g], s0, buf.x[g]);
      else
        load_raw_checked<DT, EPT, MVSD_VERIFY_NT_SCORES>(tb[g], s0, vend, p.target_aligned,
                                                         Elem<DT>::ninf(), buf.x[g]);
      if constexpr (HAS_DRAFT)
        load_raw_f32<DT, EPT, F>(qb[g], s0, vend, p.draft_aligned, 0.f, buf.q[g]);
    }
    load_raw_f32<DT, EPT, F>(eb, s0, vend, p.noise_aligned, 1.f, buf.e);
  };

  float MX[G], NL[G];
  auto wait_stats = [&]() {
    if constexpr (!PARKED) after_loads();
    if (wave_id() < nrows) {
      float mx, sum;
      if (!wave_row_stats(p.stat_slots + (int64_t)(row0 + wave_id()) * p.nc, p.nc, c1, &p.ctrl[1], mx, sum) &&
          lane_id() == 0)
        atomic_store_relaxed(&p.ctrl[1], 1);
      if (lane_id() == 0) {
        s_M[wave_id()] = mx;
        s_L[wave_id()] = (float)(-log2((double)sum));
      }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      MX[g] = s_M[g];
      NL[g] = s_L[g];
    }
    if constexpr (PARKED) after_loads();
  };

  // Scores are max(p - q, 0) / E >= 0 and ties keep the lowest index, so starting from
  // (0, v0) and taking only strictly larger scores gives the same argmax without the clamp.
  float bv[G];
  int bi[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    bv[g] = 0.f;
    bi[g] = (int)v0;
  }
  auto body = [&](const Buf& buf, int64_t s0, auto fast) {
    constexpr int NV = EPT / Elem<DT>::kVec;
    u32x4 xp[PARKED ? G : 1][NV];
    if constexpr (PARKED) {
      const int j = (int)((s0 - v0) / (kVThreads * EPT));
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < NV; ++i) xp[g][i] = park[((j * G + g) * NV + i) * kVThreads + threadIdx.x];
    }
    float inv[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) inv[k] = recip_rn(raw_f32(buf.e, k));
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g < nrows) {
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          const int idx = elem_index<DT, EPT>(s0, k);
          const u32x4* xg;
          if constexpr (PARKED) xg = xp[g];
          else xg = buf.x[g];
          const float x = raw_elem<DT>(xg, k);
          float prob = __builtin_amdgcn_exp2f(fmaf(x - MX[g], c1, NL[g]));  // softmax
          if constexpr (MASKED) prob = row_masked(mk[g], x, idx) ? 0.f : prob;
          float w;
          if constexpr (HAS_DRAFT) w = prob - raw_f32(buf.q[g], k);  // clamp folded into bv >= 0
          else w = idx == d[g] ? 0.f : prob;
          const float score = w * inv[k];
          // columns rise with s0 and k, so a strict compare keeps the first maximum
          const bool take = (score > bv[g]) & (decltype(fast)::value || idx < vend);
          bv[g] = take ? score : bv[g];
          bi[g] = take ? idx : bi[g];
        }
      }
    }
  };
  pipeline<kVThreads * EPT, Buf>(v0, vend, aligned, load, body, wait_stats);
  uint64_t key[G];
#pragma unroll
  for (int g = 0; g < G; ++g) key[g] = argmax_key(bv[g], bi[g]);
  const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_key);
  if ((int)threadIdx.x < nrows) slot_store(p.arg_slots + (int64_t)(row0 + threadIdx.x) * p.arg_stride + c, best);
}

// ------------------------------------------------------------------ main kernel ------
// Tunables (compile-time): elements per thread per row (fp32 targets; 16-bit targets), rows
// per group, and an optional cap on waves per SIMD that bounds the register budget (0 = let
// the compiler choose).
#ifndef MVSD_VERIFY_EPT_F32
#define MVSD_VERIFY_EPT_F32 4
#endif
#ifndef MVSD_VERIFY_EPT_16
#define MVSD_VERIFY_EPT_16 8
#endif
#ifndef MVSD_VERIFY_GROUP
#define MVSD_VERIFY_GROUP 4
#endif
#ifndef MVSD_VERIFY_WAVES_PER_EU
#define MVSD_VERIFY_WAVES_PER_EU 0
#endif
#if MVSD_VERIFY_WAVES_PER_EU > 0
#define MVSD_VERIFY_ATTRS __attribute__((amdgpu_waves_per_eu(MVSD_VERIFY_WAVES_PER_EU, 8)))
#else
#define MVSD_VERIFY_ATTRS
#endif
#ifndef MVSD_FUSED_WAVES_PER_EU
#define MVSD_FUSED_WAVES_PER_EU 0
#endif
#if MVSD_FUSED_WAVES_PER_EU > 0
#define MVSD_FUSED_ATTRS __attribute__((amdgpu_waves_per_eu(MVSD_FUSED_WAVES_PER_EU, 8)))
#else
#define MVSD_FUSED_ATTRS
#endif

// Ticket t -> step s = t / step_size: the first nc tickets of step s are the A-chunks (stats,
// or the argmax for greedy groups) of group s; when the batch has random requests the next nc
// are the B-chunks (scores) of group s - lag.  Slots of absent groups are claimed and skipped.
struct TaskDecode {
  int total, step_size, nc, lag, groups, two_phase, split, quarter;
  const int* qgi;  // queue position -> group index (nullptr: identity)
  const int* goff;  // requests' group offsets in LDS (descriptors derived), or nullptr
  RequestMeta meta;  // request metadata in LDS (with goff)
  int B, G;
};

// Descriptor of group li (the layout of grp_desc) from the requests' group offsets and
// metadata in LDS.
__device__ inline int4 group_desc(const int* goff, const RequestMeta& m, int B, int G, int li) {
  int lo = 0, hi = B - 1;  // the last request whose first group is <= li owns it
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (goff[mid] <= li) lo = mid;
    else hi = mid - 1;
  }
  const int r = lo;
  const int kf = m.kflags[r];
  const int k = kf & 0xffff;
  const int g = li - goff[r];
  const int ng = goff[r + 1] - goff[r];
  return make_int4(r, m.begin[r] + g * G, min(G, k - g * G) | ng << 8 | (kf >> 16) << 16 | g << 24,
                   __float_as_int(m.c1[r]));
}

// Thread 0: decode ticket t and fetch its group descriptor into dst[0..7]
// = {t, arg slot, valid | phase_b << 1 | half << 2 | quarter << 3, request, first row,
// rows | groups << 8 | flags << 16 | index in request << 24, bits of c1, the request's groups
// scored in half chunks | in quarter chunks << 16}.  The arg slot is the chunk, or for a
// half-chunk (quarter-chunk) task of the epilogue split 2 * chunk + half (4 * chunk + quarter).
//
// With the split, tickets past the regular steps (groups * step_size of them) hold only score
// tasks: lag - quarter steps of 2 * nc half-chunk tasks (one group each), then quarter steps
// of 4 * nc quarter-chunk tasks (one group each).
__device__ inline void fetch_task(const VerifyParams& p, const TaskDecode& td, int t, int* dst) {
  int c = 0, flags = 0, nsplit = 0;
  int4 d = make_int4(0, 0, 0, 0);
  if (t < td.total) {
    const int t_reg = td.groups * td.step_size;
    const int t_half = (td.lag - td.quarter) * td.step_size;
    int li, kind = 0;  // kind: 0 regular step, 1 half chunk, 2 quarter chunk
    bool phase_b = true;
    if (!td.split || t < t_reg) {
      const int step = t / td.step_size;
      const int w = t - step * td.step_size;
      phase_b = w >= td.nc;
      c = phase_b ? w - td.nc : w;
      li = phase_b ? step - td.lag : step;
    } else if (t < t_reg + t_half) {
      const int u = t - t_reg;
      const int s = u / td.step_size;
      c = u - s * td.step_size;
      li = td.groups + s - td.lag;
      kind = 1;
    } else {
      const int u = t - t_reg - t_half;
      const int s = u / (2 * td.step_size);
      c = u - s * 2 * td.step_size;
      li = td.groups - td.quarter + s;
      kind = 2;
    }
    if (li >= 0 && li < td.groups) {
      d = td.goff ? group_desc(td.goff, td.meta, td.B, td.G, li) : p.grp_desc[td.qgi ? td.qgi[li] : li];
      const bool full = (d.z >> 16) & kFull;
      flags = (!phase_b || full ? 1 : 0) | (phase_b ? 2 : 0) | (kind == 1 ? 4 : 0) | (kind == 2 ? 8 : 0);
      if (td.split && full) {
        // the request's groups in [groups - lag, groups - quarter) score in half chunks,
        // those in [groups - quarter, groups) in quarter chunks
        const int first = li - ((d.z >> 24) & 0xff);
        const int end = first + ((d.z >> 8) & 0xff);
        const int qlo = td.groups - td.quarter, hlo = td.groups - td.lag;
        const int nq = max(0, end - max(first, qlo));
        const int nh = max(0, min(end, qlo) - max(first, hlo));
        nsplit = nh | nq << 16;
      }
    }
  }
  dst[0] = t;
  dst[1] = c;
  dst[2] = flags;
  dst[3] = d.x;
  dst[4] = d.y;
  dst[5] = d.z;
  dst[6] = d.w;
  dst[7] = nsplit;
}

// Group offsets of the requests (groups of ceil(K / G) rows) into goff[0..B] in LDS, and the
// request metadata, built by every workgroup: each thread reads the metadata of a run of
// consecutive requests once (the group counts wait in goff for the scan).  Requests without
// drafts get their output row here (bonus, then -1), from workgroup r mod grid; every other
// row is written by its finalisation.
// Exclusive scan of one value per thread over the kVThreads-thread block: shuffle scans within
// the waves, then one barrier for the wave totals.  Returns this thread's exclusive prefix;
// total receives the block's sum.
__device__ inline int block_exclusive_scan(int v, int& total) {
  __shared__ int s_wave[kVWaves];
  const int lane = lane_id(), w = wave_id();
  int x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(x, d, kWave);
    x += lane >= d ? y : 0;
  }
  if (lane == kWave - 1) s_wave[w] = x;
  __syncthreads();
  int before = 0, sum = 0;
#pragma unroll
  for (int i = 0; i < kVWaves; ++i) {
    const int t = s_wave[i];
    before += i < w ? t : 0;
    sum += t;
  }
  total = sum;
  return before + x - v;
}

__device__ inline void build_lds_tables(const VerifyParams& p, int* goff, const RequestMeta& m) {
  const int tid = threadIdx.x;
  const int per = (p.B + kVThreads - 1) / kVThreads;
  const int r0 = tid * per, r1 = min(p.B, r0 + per);
  int run = 0;
  for (int r = r0; r < r1; ++r) {
    int b, k;
    req_range(p, r, b, k);
    const int ng = (k + p.G - 1) / p.G;
    goff[r] = ng;
    run += ng;
    const bool greedy = req_is_greedy(p, r);
    m.begin[r] = b;
    m.kflags[r] = k | ((greedy ? kGreedy : 0) | (!greedy && !p.recovered ? kFull : 0)) << 16;
    m.c1[r] = exp2_scale(req_temperature(p, r));
  }
  int total;
  int acc = block_exclusive_scan(run, total);
  for (int r = r0; r < r1; ++r) {
    const int ng = goff[r];
    goff[r] = acc;
    acc += ng;
    if (ng == 0 && (r % (int)gridDim.x) == (int)blockIdx.x) {
      int32_t* out = p.out + (int64_t)r * p.out_stride;
      for (int c = 0; c <= p.max_spec_len; ++c) out[c] = c == 0 ? p.bonus[r] : -1;
    }
  }
  if (tid == 0) goff[p.B] = total;
  __syncthreads();
}

// The row masks of the sampling constraints live in the workspace; the last workgroup out
// (every task and finalisation has read them) returns them to zero, like everything else the
// call used, so that a later call whose slot arrays overlap them finds zeros.
__device__ inline void clear_masks(const VerifyParams& p) {
  if (p.masks)
    for (int i = threadIdx.x; i < p.P; i += kVThreads) p.masks[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int DT, int EPT, int G, bool HAS_DRAFT, bool MASKED>
__global__ __launch_bounds__(kVThreads) MVSD_VERIFY_ATTRS void verify_kernel(VerifyParams p) {
  static_assert(EPT % Elem<DT>::kVec == 0, "EPT must be a multiple of the vector width");
  __shared__ float s_red[G * kVWaves];
  __shared__ uint64_t s_key[G * kVWaves];
  __shared__ float s_M[G];
  __shared__ float s_L[G];
  __shared__ int s_info[2][8];  // double-buffered decoded ticket (current, next)
  __shared__ int s_last;
  __shared__ FinalizeSmem fsm;

  __shared__ int s_goff[kMaxLdsRequests + 1];
  __shared__ int s_rbegin[kMaxLdsRequests], s_rkf[kMaxLdsRequests];
  __shared__ float s_rc1[kMaxLdsRequests];

  const int tid = threadIdx.x;
  const int queue = blockIdx.x % p.nq;
  int* ticket = &p.qticket[queue];
  // the first ticket is claimed before the tables are built, so its round trip overlaps them
  int tfirst = 0;
  if (tid == 0) tfirst = atomic_add_relaxed(ticket, 1);
  const int* goff = p.grp_off;
  const RequestMeta meta{s_rbegin, s_rkf, s_rc1};
  if (p.lds_groups) {
    build_lds_tables(p, s_goff, meta);
    goff = s_goff;
  }
  const int groups = goff[p.B];
  TaskDecode td;
  td.nc = p.nc;
  td.lag = p.lag;
  td.groups = p.lds_groups ? groups : p.qcount[queue];
  td.qgi = p.nq > 1 ? p.qgi + p.qoff[queue] : nullptr;
  td.goff = p.lds_groups ? s_goff : nullptr;
  td.meta = meta;
  td.B = p.B;
  td.G = p.G;
  td.two_phase = p.two_phase;
  td.split = p.split;
  td.quarter = p.split ? p.quarter : 0;
  td.step_size = p.two_phase ? 2 * td.nc : td.nc;
  td.total = (td.groups + (p.two_phase ? td.lag : 0) + td.quarter) * td.step_size;

  // Deferred request-completion count (see below).
  int pend_cnt = 0, pend_r = -1, pend_target = 0;
  bool pend_greedy = false, pend_full = false;
  auto settle = [&]() {
    if (pend_r >= 0) {
      if (tid == 0) s_last = pend_cnt == pend_target - 1;
      __syncthreads();
      if (s_last) finalize_request(p, goff, pend_r, pend_greedy, pend_full, fsm);
      __syncthreads();
      pend_r = -1;
    }
  };

  // The next ticket is claimed when a task starts and decoded once the task's loads are in
  // flight, so the atomic and the descriptor fetch overlap with HBM traffic.
  if (tid == 0) fetch_task(p, td, tfirst, s_info[0]);
  __syncthreads();
  for (int par = 0;; par ^= 1) {
    const int* info = s_info[par];
    const int t = info[0];
    if (t >= td.total) break;
    int tnext = 0;
    if (tid == 0) tnext = atomic_add_relaxed(ticket, 1);
    auto prefetch = [&]() {
      if (tid == 0) fetch_task(p, td, tnext, s_info[par ^ 1]);
    };
    const int tflags = info[2];
    if (!(tflags & 1)) {
      prefetch();
      __syncthreads();
      continue;
    }
    const bool phase_b = tflags & 2;
    const int c = info[1];
    const int r = info[3];
    const int row0 = info[4];
    const int nrows = info[5] & 0xff;
    const int ngr = (info[5] >> 8) & 0xff;
    const int gflags = (info[5] >> 16) & 0xff;
    const float c1 = __int_as_float(info[6]);
    const int nsplit = info[7];
    const bool greedy = gflags & kGreedy;
    const bool full = gflags & kFull;
    int64_t v0, vend;
    if (tflags & 12) {
      // part c % n (n = 2 halves or 4 quarters) of chunk c / n, split at sub-chunk boundaries
      const int n = (tflags & 4) ? 2 : 4;
      const int part = c & (n - 1);
      const int64_t cs = (int64_t)(c / n) * p.chunk;
      const int64_t ce = min((int64_t)p.V, cs + p.chunk);
      constexpr int64_t SUB = (int64_t)kVThreads * EPT;
      const int64_t nsc = (ce - cs + SUB - 1) / SUB;
      v0 = min(ce, cs + (nsc * part + n - 1) / n * SUB);
      vend = min(ce, cs + (nsc * (part + 1) + n - 1) / n * SUB);
    } else {
      v0 = (int64_t)c * p.chunk;
      vend = min((int64_t)p.V, v0 + p.chunk);
    }
    if (greedy) {
      task_argmax<DT, EPT, G, MASKED>(p, c, row0, nrows, v0, vend, s_key, prefetch);
    } else if (!phase_b) {
      task_stats<DT, EPT, G, MASKED>(p, c, c1, row0, nrows, v0, vend, s_red, s_M, prefetch);
    } else {
      task_scores<DT, EPT, G, HAS_DRAFT, MASKED>(p, c, r, c1, row0, nrows, v0, vend, s_key, s_M,
                                                 s_L, prefetch);
    }
    // ---- request completion: the last counted task runs the accept/reject chain ----
    // (counted: B-tasks of full random requests, A-tasks otherwise).  The counter's result
    // is examined after the next task, so the atomic's round trip is never waited for.
    settle();
    if (full == phase_b) {
      if (tid == 0) pend_cnt = atomic_add_relaxed(&p.req_cnt[r], 1);
      pend_r = r;
      // half-chunk groups count 2 * nc tasks, quarter-chunk groups 4 * nc
      pend_target = (ngr + (nsplit & 0xffff) + 3 * (nsplit >> 16)) * td.nc;
      pend_greedy = greedy;
      pend_full = full;
    }
    __syncthreads();
  }
  settle();

  // The last workgroup out (every other one has made its final claim and finished reading
  // grp_off / grp_desc) returns the group tables, ticket and exit counter to zero, so the
  // whole workspace is zero again whatever layout the next call uses.
  if (tid == 0) s_last = atomic_add_relaxed(&p.ctrl[2], 1) == (int)gridDim.x - 1;
  __syncthreads();
  if (s_last) {
    clear_masks(p);
    if (!p.lds_groups) {
      for (int i = tid; i <= p.B; i += kVThreads) p.grp_off[i] = 0;
      for (int i = tid; i < groups; i += kVThreads) {
        p.grp_desc[i] = make_int4(0, 0, 0, 0);
        p.qgi[i] = 0;
      }
    }
    for (int q = tid; q < p.nq; q += kVThreads) {
      atomic_store_relaxed(&p.qticket[q], 0);
      p.qcount[q] = 0;
      p.qoff[q] = 0;
    }
    if (tid == 0) atomic_store_relaxed(&p.ctrl[2], 0);
  }
}

// ------------------------------------------------------------------ fused kernel -----
// Single-read kernel.  A task is one sub-chunk (kVThreads * EPT columns) of a row group;
// tickets go out in group-major order, so the nc sub-chunks of a group hold consecutive
// tickets.  In each iteration a workgroup
//   * issues the draft / noise loads (and the stats-slot polls of its group) of the oldest
//     task of its FIFO when that task is due, then the target loads of its next task;
//   * reduces the current task's target sub-chunk, loaded during the previous iteration:
//     per-row chunk stats (greedy groups: the chunk argmax) are published, and for random
//     rows the sub-chunk is parked in LDS and the task joins the FIFO;
//   * once the FIFO holds kDepth tasks, retires the oldest: the group's stats are combined
//     and the parked sub-chunk is scored against the draft and noise sub-chunks, publishing
//     the chunk-local recovered candidate.
// Every input byte is read once; a task that finds no free parking slot (only when the FIFO
// has grown past kDepth, see below) re-reads its target sub-chunk when it is scored.
//
// One ticket atomic per iteration, issued after the stage-1 reduction by thread 0, is read
// and decoded one iteration later (group descriptors come from the LDS group offsets and
// scalar loads), and the ticket's target loads go out in the iteration after that: no wave
// waits on an atomic it has just issued, and every vector load is unconditional (absent
// tasks load one line), so the in-order load counters wait for exactly the data needed.
//
// Progress.  A workgroup waits for a group's stats only when retiring its oldest task, of
// group g, and only if every ticket it holds without having published its stats lies past
// g.  Those tickets are all newer than the one whose loads are in flight, so checking that
// one suffices; otherwise the retirement is postponed and the FIFO grows.  Take the lowest
// group g* that some workgroup waits for: a workgroup holding an unpublished ticket of g* is
// not waiting (it could only wait for a group below g*), so it publishes it.  If every
// resident workgroup waits, one of them holds a ticket past g*, so every ticket of g* has been
// claimed, hence published, and the workgroups waiting for g* proceed.  Workgroups not yet
// resident hold no tickets.  The waits are bounded all the same (kSpinLimit, flag ctrl[1]).
// While the FIFO holds tasks of one group only, it holds fewer than nc of them, so kFifo >
// nc + kDepth + 4 bounds it (checked by the host).

#ifndef MVSD_FUSED_DEPTH
#define MVSD_FUSED_DEPTH 3
#endif
constexpr int kDepth = MVSD_FUSED_DEPTH;  // parking slots (target sub-chunks) per workgroup
static_assert(kDepth >= 2 && kDepth <= 8, "parking depth");
constexpr int kFifo = 128;     // FIFO records (a power of two)
constexpr int kTaskInts = 16;  // LDS words of a task record

// Load of a read-only kernel input at a wave-uniform index through the constant address
// space: a scalar load, which leaves the vector-memory counters alone.
template <typename T>
__device__ inline T ld_const(const T* base, int64_t i) {
  return ((const __attribute__((address_space(4))) T*)base)[i];
}
__device__ inline float4 ld_const(const float4* base, int64_t i) {
  const float* f = reinterpret_cast<const float*>(base) + 4 * i;
  return make_float4(ld_const(f, 0), ld_const(f, 1), ld_const(f, 2), ld_const(f, 3));
}

template <int G>
struct FusedTask {
  int t;        // ticket, < 0: none
  int c;        // sub-chunk of the row
  int r;        // request
  int row0;     // first verify row of the group
  int nrows;    // rows in the group
  int ngr;      // groups of the request
  int flags;    // kGreedy | kFull
  int slot;     // parking slot of a FIFO record, -1: not parked
  float c1;     // log2(e) / T
  int trow[G];  // target rows of the group's rows (the last one repeated)
};

template <int G>
__device__ inline FusedTask<G> no_task() {
  FusedTask<G> d;
  d.t = -1;
  d.c = 0;
  d.r = 0;
  d.row0 = 0;
  d.nrows = 1;
  d.ngr = 1;
  d.flags = 0;
  d.slot = -1;
  d.c1 = 1.f;
#pragma unroll
  for (int g = 0; g < G; ++g) d.trow[g] = 0;
  return d;
}

template <int G>
__device__ inline void task_put(int* d, const FusedTask<G>& t) {
  d[0] = t.t;
  d[1] = t.c;
  d[2] = t.r;
  d[3] = t.row0;
  d[4] = t.nrows;
  d[5] = t.ngr;
  d[6] = t.flags;
  d[7] = t.slot;
  d[8] = __float_as_int(t.c1);
#pragma unroll
  for (int g = 0; g < G; ++g) d[9 + g] = t.trow[g];
}

// A task record in LDS, read by every thread into wave-uniform (scalar) registers.
template <int G>
__device__ inline FusedTask<G> task_get(const int* d) {
  FusedTask<G> t;
  t.t = __builtin_amdgcn_readfirstlane(d[0]);
  t.c = __builtin_amdgcn_readfirstlane(d[1]);
  t.r = __builtin_amdgcn_readfirstlane(d[2]);
  t.row0 = __builtin_amdgcn_readfirstlane(d[3]);
  t.nrows = __builtin_amdgcn_readfirstlane(d[4]);
  t.ngr = __builtin_amdgcn_readfirstlane(d[5]);
  t.flags = __builtin_amdgcn_readfirstlane(d[6]);
  t.slot = __builtin_amdgcn_readfirstlane(d[7]);
  t.c1 = __int_as_float(__builtin_amdgcn_readfirstlane(d[8]));
#pragma unroll
  for (int g = 0; g < G; ++g) t.trow[g] = __builtin_amdgcn_readfirstlane(d[9 + g]);
  return t;
}

// Ticket t -> task, run by a whole wave with t wave-uniform: the request comes from the LDS
// group offsets (scanning forward from this workgroup's previous decode, `scan`, since its
// tickets only rise), its metadata from LDS; target rows from scalar loads.  The fields
// follow group_desc.
template <int G>
__device__ inline FusedTask<G> fused_decode(const VerifyParams& p, const int* goff,
                                            const RequestMeta& m, int total, int t, int& scan) {
  FusedTask<G> d = no_task<G>();
  if (t < 0 || t >= total) return d;
  const int li = t / p.nc;
  int r = goff[scan] <= li ? scan : 0;
  while (goff[r + 1] <= li) ++r;  // goff[B] = groups > li ends the scan
  r = __builtin_amdgcn_readfirstlane(r);
  scan = r;
  const int b = __builtin_amdgcn_readfirstlane(m.begin[r]);
  const int kf = __builtin_amdgcn_readfirstlane(m.kflags[r]);
  const int g0 = __builtin_amdgcn_readfirstlane(goff[r]);
  const int g1 = __builtin_amdgcn_readfirstlane(goff[r + 1]);
  const int k = kf & 0xffff;
  const int g = li - g0;
  d.t = t;
  d.c = t - li * p.nc;
  d.r = r;
  d.row0 = b + g * G;
  d.nrows = min(G, k - g * G);
  d.ngr = g1 - g0;
  d.flags = kf >> 16;
  d.c1 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(m.c1[r])));
  int tr[G];
#pragma unroll
  for (int gg = 0; gg < G; ++gg) tr[gg] = d.row0 + min(gg, d.nrows - 1);
  if (p.target_rows) {
#pragma unroll
    for (int gg = 0; gg < G; ++gg) tr[gg] = ld_const(p.target_rows, tr[gg]);
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
      tr[gg] = tr[gg] < 0 ? 0 : (tr[gg] >= p.target_num_rows ? (int)p.target_num_rows - 1 : tr[gg]);
  }
#pragma unroll
  for (int gg = 0; gg < G; ++gg) d.trow[gg] = tr[gg];
  return d;
}

template <int DT, int EPT, int G>
struct FusedX {
  u32x4 x[G][EPT / Elem<DT>::kVec];  // target sub-chunk of a task
};

template <int DT, int EPT, int G>
struct FusedQ {
  u32x4 q[G][EPT / 4];  // draft sub-chunk
  u32x4 e[EPT / 4];     // noise sub-chunk
};

template <int DT, int EPT, int G, bool HAS_DRAFT, bool MASKED>
__global__ __launch_bounds__(kVThreads) MVSD_FUSED_ATTRS void verify_fused_kernel(VerifyParams p) {
  static_assert(EPT % Elem<DT>::kVec == 0, "EPT must be a multiple of the vector width");
  static_assert(9 + G <= kTaskInts, "task record size");
  static_assert(kVWaves % G == 0, "the stats polls give every row whole waves");
  static_assert(G <= kWave, "one lane per row combines the row statistics");
  using S = typename Elem<DT>::storage;
  using Task = FusedTask<G>;
  using XBuf = FusedX<DT, EPT, G>;
  using QBuf = FusedQ<DT, EPT, G>;
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int NV = EPT / VEC;
  constexpr int N32 = EPT / 4;
  constexpr int SUB = kVThreads * EPT;
  constexpr int PR = kVThreads / G;  // poll threads per row: a row's nc <= PR stats slots
  constexpr int WPR = kVWaves / G;   // waves per row
  __shared__ u32x4 s_park[kDepth][G][NV][kVThreads];
  __shared__ int s_fifo[kFifo][kTaskInts];
  __shared__ int s_dec[2][kTaskInts];
  __shared__ int s_fin[2][2][2];
  __shared__ float s_pm[kVWaves], s_ps[kVWaves];
  __shared__ int s_rdy[kVWaves];
  __shared__ float s_wm[G * kVWaves], s_ws[G * kVWaves];
  __shared__ uint64_t s_keyD[G * kVWaves], s_keyF[G * kVWaves];
  __shared__ int s_last;
  __shared__ FinalizeSmem fsm;
  __shared__ int s_goff[kMaxFusedRequests + 1];
  __shared__ int s_rbegin[kMaxFusedRequests], s_rkf[kMaxFusedRequests];
  __shared__ float s_rc1[kMaxFusedRequests];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wid = wave_id();
  const int nc = p.nc;
  const S* target = static_cast<const S*>(p.target);
  const float* dummy = reinterpret_cast<const float*>(p.stat_slots);  // 16-byte aligned, valid
  int* ticket = &p.qticket[0];
  const RequestMeta meta{s_rbegin, s_rkf, s_rc1};

  build_lds_tables(p, s_goff, meta);
  const int total = s_goff[p.B] * nc;

  // ---- loads (unconditional; a task that is absent loads one line with every lane) ----
  auto issue_x = [&](XBuf& b, const Task& t) {
    const bool live = t.t >= 0;
    const int64_t v0 = (int64_t)t.c * SUB;
    const int64_t vlast = min((int64_t)p.V, v0 + SUB) - VEC;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const S* base = target + (int64_t)t.trow[g] * p.target_stride;
#pragma unroll
      for (int n = 0; n < NV; ++n)
        b.x[g][n] = load_target16<true>(base + (live ? min(vec_col<DT>(v0, n), vlast) : 0));
    }
  };
  // Draft / noise sub-chunks of task o.
  auto issue_q = [&](QBuf& b, const Task& o, bool live) {
    const int64_t v0 = (int64_t)o.c * SUB;
    const int64_t vlast4 = min((int64_t)p.V, v0 + SUB) - 4;
    auto col32 = [&](int m) -> int64_t {
      return live ? min(vec_col<DT>(v0, m / (VEC / 4)) + (m % (VEC / 4)) * 4, vlast4) : 0;
    };
    if constexpr (HAS_DRAFT) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float* base = live ? p.draft + (int64_t)(o.row0 + min(g, o.nrows - 1)) * p.draft_stride : dummy;
#pragma unroll
        for (int m = 0; m < N32; ++m)
          b.q[g][m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + col32(m)));
      }
    }
    const float* eb = live ? p.noise + (int64_t)o.r * p.noise_stride : dummy;
#pragma unroll
    for (int m = 0; m < N32; ++m)
      b.e[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(eb + col32(m)));
  };
  // Stats polls of task o's group: thread tid covers slot tid % PR of row tid / PR (rows past
  // the group's end, and no task, poll one line).
  auto issue_poll = [&](const Task& o, bool live) -> uint64_t {
    const int g = tid / PR, c = tid % PR;
    const uint64_t* sl = p.stat_slots;
    if (live) sl += (int64_t)(o.row0 + min(g, o.nrows - 1)) * nc + (g < o.nrows ? min(c, nc - 1) : 0);
    return slot_load(sl);
  };

  // ---- stage 1 of task t (target sub-chunk in xb): stats or greedy argmax; park ----
  auto stage_one = [&](const XBuf& xb, const Task& t, int slot) {
    const int64_t v0 = (int64_t)t.c * SUB;
    const int64_t vend = min((int64_t)p.V, v0 + SUB);
    float4 mk[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      mk[g] = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (MASKED) mk[g] = ld_const(p.masks, t.row0 + min(g, t.nrows - 1));
    }
    if (slot >= 0) {
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (g < t.nrows) {
#pragma unroll
          for (int n = 0; n < NV; ++n) s_park[slot][g][n][tid] = xb.x[g][n];
        }
    }
    if (t.flags & kGreedy) {
      uint64_t key[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float bv = -INFINITY;
        int bi = (int)v0;
        if (g < t.nrows) {
#pragma unroll
          for (int k = 0; k < EPT; ++k) {
            const int idx = elem_index<DT, EPT>(v0, k);
            float v = raw_elem<DT>(xb.x[g], k);
            if constexpr (MASKED) v = row_masked(mk[g], v, idx) ? -INFINITY : v;
            // columns rise with k: a strict compare keeps the first maximum; NaN wins
            const bool take = ((v > bv) | ((v != v) & (bv == bv))) & (idx < vend);
            bv = take ? v : bv;
            bi = take ? idx : bi;
          }
        }
        key[g] = argmax_key(bv, bi);
      }
      const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_keyD);
      if (tid < t.nrows) slot_store(p.arg_slots + (int64_t)(t.row0 + tid) * p.arg_stride + t.c, best);
      return;
    }
    // per wave and row: the raw max m and sum of exp2((x - m) c1) (masked entries add
    // nothing; the max runs over every entry, which only moves the reference point), then
    // the row threads combine the waves' pairs
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g < t.nrows) {
        float x[EPT];
        float m = -INFINITY;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          x[k] = elem_index<DT, EPT>(v0, k) < vend ? raw_elem<DT>(xb.x[g], k) : -INFINITY;
          m = fmaxf(m, x[k]);
        }
        m = wave_max(m);
        const float ref = m == -INFINITY ? 0.f : m;
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          const float e = __builtin_amdgcn_exp2f((x[k] - ref) * t.c1);
          if constexpr (MASKED) acc += row_masked(mk[g], x[k], elem_index<DT, EPT>(v0, k)) ? 0.f : e;
          else acc += e;
        }
        acc = wave_sum(acc);
        if (lane == 0) {
          s_wm[g * kVWaves + wid] = m;
          s_ws[g * kVWaves + wid] = acc;
        }
      }
    }
    __syncthreads();
    if (tid < t.nrows) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kVWaves; ++w) M = fmaxf(M, s_wm[tid * kVWaves + w]);
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kVWaves; ++w) {
        const float mw = s_wm[tid * kVWaves + w];
        if (mw != -INFINITY) sum += s_ws[tid * kVWaves + w] * __builtin_amdgcn_exp2f((mw - M) * t.c1);
      }
      slot_store(p.stat_slots + (int64_t)(t.row0 + tid) * nc + t.c,
                 pack_stats(M, M == -INFINITY ? 0.f : sum));
    }
  };

  // ---- stage 2 of task o: combine its group's stats, score, publish ----
  auto partial = [&](uint64_t v, bool live, float c1) {
    float m = live ? unpack_stats(v).x : -INFINITY;
    m = wave_max(m);
    const float2 st = unpack_stats(v);
    float a = (live && st.x != -INFINITY) ? st.y * exp2f((st.x - m) * c1) : 0.f;
    a = wave_sum(a);
    if (lane == 0) {
      s_pm[wid] = m;
      s_ps[wid] = a;
    }
  };
  // qb: o's draft / noise sub-chunks (loaded for ticket qtag: reloaded here when that is not o,
  // after a postponed retirement); poll: this iteration's stats-slot poll of o's group.
  auto stage_two = [&](QBuf& qb, int qtag, uint64_t poll, const Task& o) {
    const int g = wid / WPR, c = tid % PR;
    const bool live = g < o.nrows && c < nc;
    partial(poll, live, o.c1);
    const int rdy = __all(!live || poll != 0);  // the vote needs every lane active
    if (lane == 0) s_rdy[wid] = rdy;
    if (qtag != o.t) issue_q(qb, o, true);
    XBuf xr;  // the target sub-chunk of a task that was not parked
    if (o.slot < 0) issue_x(xr, o);
    __syncthreads();
    bool ready = true;
#pragma unroll
    for (int w = 0; w < kVWaves; ++w) ready &= s_rdy[w] != 0;
    if (!ready) {  // some chunk of the group has not published yet: each wave waits for its slots
      if (g < o.nrows) {
        const uint64_t* sl = p.stat_slots + (int64_t)(o.row0 + g) * nc + min(c, nc - 1);
        uint64_t v = 0;
        for (int spins = 0;; ++spins) {
          v = slot_load(sl);
          if (__all(c >= nc || v != 0)) break;
          if (spins >= kSpinLimit || ((spins & 255) == 255 && atomic_load_relaxed(&p.ctrl[1]) != 0)) {
            if (lane == 0) atomic_store_relaxed(&p.ctrl[1], 1);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        partial(v, c < nc, o.c1);
      }
      __syncthreads();
    }
    // lane gg < nrows of every wave combines row gg's partials; the values are broadcast
    float myM = 0.f, myL = 0.f;
    if (lane < o.nrows) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < WPR; ++w) M = fmaxf(M, s_pm[lane * WPR + w]);
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < WPR; ++w) {
        const float mw = s_pm[lane * WPR + w];
        if (mw != -INFINITY) sum += s_ps[lane * WPR + w] * exp2f((mw - M) * o.c1);
      }
      myM = M;
      myL = (float)(-log2((double)sum));
    }
    const int64_t v0 = (int64_t)o.c * SUB;
    const int64_t vend = min((int64_t)p.V, v0 + SUB);
    float inv[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) inv[k] = recip_rn(raw_f32(qb.e, k));
    uint64_t key[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      float bv = 0.f;  // scores are >= 0: the clamp is folded into the strict compare
      int bi = (int)v0;
      if (gg < o.nrows) {
        const int row = o.row0 + gg;
        const float MX = readlane_f32(myM, gg);
        const float NL = readlane_f32(myL, gg);
        float4 mk = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (MASKED) mk = ld_const(p.masks, row);
        int d = -1;
        if constexpr (!HAS_DRAFT) d = ld_const(p.draft_ids, row);
        u32x4 xv[NV];
        if (o.slot >= 0) {
#pragma unroll
          for (int n = 0; n < NV; ++n) xv[n] = s_park[o.slot][gg][n][tid];
        } else {
#pragma unroll
          for (int n = 0; n < NV; ++n) xv[n] = xr.x[gg][n];
        }
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          const int idx = elem_index<DT, EPT>(v0, k);
          const float x = raw_elem<DT>(xv, k);
          float prob = __builtin_amdgcn_exp2f(fmaf(x - MX, o.c1, NL));  // softmax
          if constexpr (MASKED) prob = row_masked(mk, x, idx) ? 0.f : prob;
          float w;
          if constexpr (HAS_DRAFT) w = prob - raw_f32(qb.q[gg], k);
          else w = idx == d ? 0.f : prob;
          const float score = w * inv[k];
          // columns rise with k, so a strict compare keeps the first maximum
          const bool take = (score > bv) & (idx < vend);
          bv = take ? score : bv;
          bi = take ? idx : bi;
        }
      }
      key[gg] = argmax_key(bv, bi);
    }
    const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_keyF);
    if (tid < o.nrows) slot_store(p.arg_slots + (int64_t)(o.row0 + tid) * p.arg_stride + o.c, best);
  };

  // ---- uniform pipeline state ----
  int head = 0, size = 0, free_mask = (1 << kDepth) - 1;
  bool claims_done = false;
  bool x_claim = false;               // a claim issued at the last mid point
  int x_r0 = -1, x_t0 = 0, x_f0 = 0;  // counts issued at the last mid point: request, tasks
  int x_r1 = -1, x_t1 = 0, x_f1 = 0;  // of the request, greedy | full << 1
  int pd_r = -1, pd_t = 0, pd_f = 0;  // count of this iteration's stage 1
  int pf_r = -1, pf_t = 0;            // count of the last retirement (full tasks)
  int res_claim = 0, res_c0 = 0, res_c1 = 0;  // thread 0: results of the mid-point atomics
  int scan = 0;                               // wave 0: request cursor of the decodes
  int qtag_a = -1, qtag_b = -1;               // tickets whose draft / noise are in qa / qb

  // first two tickets, decoded before the loop; the third claim is in flight
  if (wid == 0) {
    int ta = 0, tb = 0;
    if (lane == 0) {
      ta = atomic_add_relaxed(ticket, 1);
      tb = atomic_add_relaxed(ticket, 1);
    }
    ta = __builtin_amdgcn_readfirstlane(ta);
    tb = __builtin_amdgcn_readfirstlane(tb);
    const Task a = fused_decode<G>(p, s_goff, meta, total, ta, scan);
    const Task b = fused_decode<G>(p, s_goff, meta, total, tb, scan);
    if (lane == 0) {
      task_put<G>(s_fifo[0], a);
      task_put<G>(s_fifo[1], b);
    }
  }
  __syncthreads();
  Task cur = task_get<G>(s_fifo[0]);
  Task nxt = task_get<G>(s_fifo[1]);
  __syncthreads();
  claims_done = nxt.t < 0;
  x_claim = !claims_done;
  if (tid == 0 && x_claim) res_claim = atomic_add_relaxed(ticket, 1);

  XBuf xa, xb;
  QBuf qa, qb;
  issue_x(xa, cur);

  // xc: the current task's target (loaded last iteration), xn: receives the next task's;
  // qc: draft / noise of the task due now (tag qtc), qn: receives those of the next due task.
  auto iteration = [&](XBuf& xc, XBuf& xn, QBuf& qc, int& qtc, QBuf& qn, int& qtn,
                       const int par) -> bool {
    if (cur.t < 0 && nxt.t < 0 && size == 0 && !x_claim && x_r0 < 0 && x_r1 < 0 && pf_r < 0)
      return false;
    // ---- plan: retire the FIFO's oldest task once it holds kDepth (or when draining) ----
    const bool push = cur.t >= 0 && (cur.flags & kFull);
    const bool due = size + (push ? 1 : 0) >= kDepth || (cur.t < 0 && size > 0);
    const Task o = due ? task_get<G>(s_fifo[head]) : no_task<G>();
    // the task due next iteration, assuming this retirement goes ahead: prefetch its draft /
    // noise now (a postponed retirement makes stage 2 reload them)
    const int size_next = size + (push ? 1 : 0) - (due ? 1 : 0);
    const bool push_next = nxt.t >= 0 && (nxt.flags & kFull);
    const bool due_next = size_next + (push_next ? 1 : 0) >= kDepth || (nxt.t < 0 && size_next > 0);
    Task on = no_task<G>();
    if (due_next) {
      const int k = due ? 1 : 0;  // position of the next oldest task
      if (k < size) on = task_get<G>(s_fifo[(head + k) & (kFifo - 1)]);
      else on = cur;  // the task pushed by this iteration
    }

    // ---- loads: o's stats polls, the next due task's draft / noise, the next task's target ----
    const uint64_t poll = issue_poll(o, due);
    issue_q(qn, on, due_next);
    qtn = due_next ? on.t : -1;
    issue_x(xn, nxt);

    // ---- stage 1 of the current task ----
    if (cur.t >= 0) {
      int slot = -1;
      if (push && free_mask) {
        slot = __builtin_ctz(free_mask);
        free_mask &= ~(1 << slot);
      }
      stage_one(xc, cur, slot);
      if (push) {
        if (tid == 0) {
          Task e = cur;
          e.slot = slot;
          task_put<G>(s_fifo[(head + size) & (kFifo - 1)], e);
        }
        ++size;
      } else {
        pd_r = cur.r;
        pd_t = cur.ngr * nc;
        pd_f = (cur.flags & kGreedy) ? 1 : 0;
      }
    }

    // ---- mid point (wave 0): read the last mid point's atomics, issue this one's ----
    const bool claim = !claims_done && size + 4 < kFifo;
    if (wid == 0) {
      const int rc = __builtin_amdgcn_readfirstlane(res_claim);
      const int r0v = __builtin_amdgcn_readfirstlane(res_c0);
      const int r1v = __builtin_amdgcn_readfirstlane(res_c1);
      if (lane == 0) {
        if (claim) res_claim = atomic_add_relaxed(ticket, 1);
        if (pd_r >= 0) res_c0 = atomic_add_relaxed(&p.req_cnt[pd_r], 1);
        if (pf_r >= 0) res_c1 = atomic_add_relaxed(&p.req_cnt[pf_r], 1);
      }
      const Task d = x_claim ? fused_decode<G>(p, s_goff, meta, total, rc, scan) : no_task<G>();
      if (lane == 0) {
        task_put<G>(s_dec[par], d);
        s_fin[par][0][0] = x_r0 >= 0 && r0v == x_t0 - 1 ? x_r0 : -1;
        s_fin[par][0][1] = x_f0;
        s_fin[par][1][0] = x_r1 >= 0 && r1v == x_t1 - 1 ? x_r1 : -1;
        s_fin[par][1][1] = x_f1;
        if (!claims_done && !claim) atomic_store_relaxed(&p.ctrl[1], 1);  // FIFO bound broken
      }
    }
    const bool had_claim = x_claim;
    x_claim = claim;
    x_r0 = pd_r;
    x_t0 = pd_t;
    x_f0 = pd_f;
    x_r1 = pf_r;
    x_t1 = pf_t;
    x_f1 = 2;
    pd_r = -1;
    pf_r = -1;
    if (!claim) claims_done = true;

    // ---- stage 2 of the due task, unless this workgroup holds an unpublished ticket of its
    // group (the next task's, whose loads are in flight; later ones are newer) ----
    if (due && (nxt.t < 0 || nxt.t >= (o.t / nc + 1) * nc)) {
      stage_two(qc, qtc, poll, o);
      head = (head + 1) & (kFifo - 1);
      --size;
      if (o.slot >= 0) free_mask |= 1 << o.slot;
      pf_r = o.r;
      pf_t = o.ngr * nc;
    } else if (due) {
      qtn = -1;  // postponed: the next iteration retires o again and reloads its data
    }

    // ---- end: completions found at the mid point, the decoded claim becomes the next task ----
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int fr = __builtin_amdgcn_readfirstlane(s_fin[par][k][0]);
      if (fr >= 0) {
        const int ff = __builtin_amdgcn_readfirstlane(s_fin[par][k][1]);
        finalize_request(p, s_goff, fr, ff & 1, ff & 2, fsm);
        __syncthreads();
      }
    }
    const Task d = task_get<G>(s_dec[par]);
    if (had_claim && d.t < 0) claims_done = true;
    cur = nxt;
    nxt = had_claim ? d : no_task<G>();
    return true;
  };

  for (;;) {
    if (!iteration(xa, xb, qa, qtag_a, qb, qtag_b, 0)) break;
    if (!iteration(xb, xa, qb, qtag_b, qa, qtag_a, 1)) break;
  }

  // The last workgroup out (every other one has made its final claim) returns the ticket and
  // the exit counter to zero.
  if (tid == 0) s_last = atomic_add_relaxed(&p.ctrl[2], 1) == (int)gridDim.x - 1;
  __syncthreads();
  if (s_last) clear_masks(p);
  if (s_last && tid == 0) {
    atomic_store_relaxed(ticket, 0);
    atomic_store_relaxed(&p.ctrl[2], 0);
  }
}

// ------------------------------------------------------------------ resident kernel --
// Single-read kernel with register-resident tasks.  A task is one (row group, chunk) pair
// holding both phases: the workgroup loads the group's target chunk into registers, publishes
// the rows' chunk statistics (greedy groups: the chunk argmax), and, once the group's other
// chunks have published theirs, scores the chunk from the same registers.  Each thread holds
// kRVecs 16-byte vectors of each of the G rows, so a chunk is at most kVThreads * kRVecs
// vectors wide.  A workgroup holds two tasks: the current one, whose statistics are
// published, and the next one, whose target loads are in flight.  Per iteration:
//   A. the first poll of the current group's statistics slots, then the draft, noise (and
//      mask) loads of the current task;
//   B. the next task's statistics from its target registers, published per row;
//   C. the end of the wait for the current group's statistics (the poll was issued before
//      A's side loads, so the in-order load counter does not hold it behind them);
//   D. the claim of a new ticket, whose round trip overlaps E;
//   E. the scores of the current task, its argmax published per row, its request counted;
//   F. the decode of the new ticket, the previous task's completion check, and the new
//      ticket's target loads into the freed registers.
//
// Progress.  A workgroup waits (C) only while both tickets it holds are published, and a
// workgroup that has claimed a ticket publishes it before its next wait (F, A and B hold no
// wait).  Take the lowest group g* anybody waits for.  If every ticket of g* is claimed, each
// is published or about to be, so the waits for g* end.  Otherwise every claimed ticket lies
// below g*'s unclaimed ones, so a workgroup holds tickets of g* or lower groups only, and those
// holding a ticket of a lower group are not waiting; they finish and claim on.  Only if every
// resident workgroup held two tickets of g* and nothing else could the claims stop; the host
// keeps nc at most twice the resident workgroups, so then all of g* is claimed.  The waits are
// bounded all the same (kSpinLimit, flag ctrl[1]).
#ifndef MVSD_RESIDENT_VECS
#define MVSD_RESIDENT_VECS 2
#endif
constexpr int kRVecs = MVSD_RESIDENT_VECS;  // 16-byte target vectors per thread and row
template <int DT>
constexpr int rcols() {  // columns per thread and row of a task
  return kRVecs * Elem<DT>::kVec;
}
#ifndef MVSD_RESIDENT_WAVES_PER_EU
#define MVSD_RESIDENT_WAVES_PER_EU 2
#endif
#if MVSD_RESIDENT_WAVES_PER_EU > 0
#define MVSD_RESIDENT_ATTRS __attribute__((amdgpu_waves_per_eu(MVSD_RESIDENT_WAVES_PER_EU, 8)))
#else
#define MVSD_RESIDENT_ATTRS
#endif

// A decoded ticket, uniform over the workgroup: t < 0 for no task.  Absent tasks load row 0's
// first columns so that every path issues the same loads.
struct RTask {
  int t, c, r, row0, nrows, flags;
  float c1;
};

__device__ inline void resident_decode(const int* goff, const RequestMeta& m, int B, int G,
                                       int nc, int total, int t, int* dst) {
  int4 d = make_int4(0, 0, 1, 0);
  int c = 0;
  if (t >= 0 && t < total) {
    const int li = t / nc;
    c = t - li * nc;
    d = group_desc(goff, m, B, G, li);
  } else {
    t = -1;
  }
  dst[0] = t;
  dst[1] = c;
  dst[2] = d.x;
  dst[3] = d.y;
  dst[4] = d.z;
  dst[5] = d.w;
}

__device__ inline RTask resident_read(const int* s) {
  RTask k;
  k.t = __builtin_amdgcn_readfirstlane(s[0]);
  k.c = __builtin_amdgcn_readfirstlane(s[1]);
  k.r = __builtin_amdgcn_readfirstlane(s[2]);
  k.row0 = __builtin_amdgcn_readfirstlane(s[3]);
  const int z = __builtin_amdgcn_readfirstlane(s[4]);
  k.nrows = max(z & 0xff, 1);
  k.flags = k.t < 0 ? 0 : (z >> 16) & 0xff;
  k.c1 = __int_as_float(__builtin_amdgcn_readfirstlane(s[5]));
  return k;
}

template <int DT, int G>
struct RBuf {
  u32x4 x[G][kRVecs];
};

template <int DT, int G, bool HAS_DRAFT, bool MASKED>
struct RSide {  // draft, noise and masks of a task
  u32x4 q[HAS_DRAFT ? G : 1][rcols<DT>() / 4];
  u32x4 e[rcols<DT>() / 4];
  float4 mk[MASKED ? G : 1];
  int d[HAS_DRAFT ? 1 : G];
};

// Column of the first element of this thread's target vector i in the chunk starting at v0.
template <int DT>
__device__ inline int64_t rcol(int64_t v0, int i) {
  return v0 + ((int64_t)i * kVThreads + threadIdx.x) * Elem<DT>::kVec;
}

template <int DT, int G>
__device__ inline void resident_load_x(const VerifyParams& p, const RTask& k, int64_t v0,
                                       int64_t vend, RBuf<DT, G>& b) {
  using S = typename Elem<DT>::storage;
  constexpr int VEC = Elem<DT>::kVec;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const S* base = static_cast<const S*>(p.target) +
                    target_row(p, k.row0 + min(g, k.nrows - 1)) * p.target_stride;
#pragma unroll
    for (int i = 0; i < kRVecs; ++i) {
      const int64_t col = min(rcol<DT>(v0, i), vend - VEC);
      b.x[g][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + col));
    }
  }
}

// fp32 vectors laid out like the target's: fp32 vector m holds the 4 columns starting at
// column 4 (m % (VEC / 4)) of target vector m / (VEC / 4).
template <int DT>
__device__ inline void resident_load_f32(const float* base, int64_t v0, int64_t vend,
                                         u32x4 (&out)[rcols<DT>() / 4]) {
  constexpr int VEC = Elem<DT>::kVec;
#pragma unroll
  for (int m = 0; m < rcols<DT>() / 4; ++m) {
    const int64_t col = min(rcol<DT>(v0, m / (VEC / 4)), vend - VEC) + (m % (VEC / 4)) * 4;
    out[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + col));
  }
}

template <int DT, int G, bool HAS_DRAFT, bool MASKED>
__device__ inline void resident_load_side(const VerifyParams& p, const RTask& k, int64_t v0,
                                          int64_t vend, RSide<DT, G, HAS_DRAFT, MASKED>& s) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int row = k.row0 + min(g, k.nrows - 1);
    if constexpr (MASKED) s.mk[g] = p.masks[row];
    if constexpr (HAS_DRAFT) resident_load_f32<DT>(p.draft + (int64_t)row * p.draft_stride, v0, vend, s.q[g]);
    else s.d[g] = p.draft_ids[row];
  }
  resident_load_f32<DT>(p.noise + (int64_t)k.r * p.noise_stride, v0, vend, s.e);
}

// Row masks alone (the first read of a masked batch's tasks).
template <bool MASKED, int G>
__device__ inline void resident_masks(const VerifyParams& p, const RTask& k, float4 (&mk)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g)
    mk[g] = MASKED ? p.masks[k.row0 + min(g, k.nrows - 1)] : make_float4(0.f, 0.f, 0.f, 0.f);
}

// Element j (0 <= j < rcols) of row g: value and column.
template <int DT, int G>
__device__ inline float rx(const RBuf<DT, G>& b, int g, int j) {
  return raw_elem<DT>(b.x[g], j);
}
template <int DT>
__device__ inline int ridx(int64_t v0, int j) {
  constexpr int VEC = Elem<DT>::kVec;
  return (int)(rcol<DT>(v0, j / VEC) + j % VEC);
}

// Row statistics (max, sum of 2^((x - max) * c1)) of N rows over a block of NW waves,
// combined for row thread g (< N), which receives them; other threads get (-inf, 0).  Each
// wave rescales its lanes' sums to the wave maximum, so one barrier suffices.
template <int N, int NW>
__device__ inline float2 block_stats_to_row_thread(const float (&m)[N], const float (&s)[N],
                                                   float c1, float2* scratch) {
#pragma unroll
  for (int g = 0; g < N; ++g) {
    const float wm = wave_max(m[g]);
    const float sc = m[g] == -INFINITY ? 0.f : s[g] * __builtin_amdgcn_exp2f((m[g] - wm) * c1);
    const float ws = wave_sum(sc);
    if (lane_id() == 0) scratch[g * NW + wave_id()] = make_float2(wm, ws);
  }
  __syncthreads();
  float2 r = make_float2(-INFINITY, 0.f);
  const int t = threadIdx.x;
  if (t < N) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, scratch[t * NW + w].x);
    float S = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float2 q = scratch[t * NW + w];
      if (q.x != -INFINITY) S += q.y * exp2f((q.x - M) * c1);
    }
    r = make_float2(M, S);
  }
  return r;
}

// Chunk statistics of each row, published into the rows' stats slots.
template <int DT, int G, bool MASKED>
__device__ inline void resident_stats(const VerifyParams& p, const RTask& k, int64_t v0,
                                      int64_t vend, const RBuf<DT, G>& b, const float4 (&mk)[G],
                                      float2* s_pair) {
  constexpr int VEC = Elem<DT>::kVec;
  float m[G], s[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float lm = -INFINITY;
#pragma unroll
    for (int j = 0; j < rcols<DT>(); ++j) {
      const bool valid = rcol<DT>(v0, j / VEC) < vend;
      lm = valid ? fmaxf(lm, rx<DT, G>(b, g, j)) : lm;
    }
    const float ref = lm == -INFINITY ? 0.f : lm;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < rcols<DT>(); ++j) {
      const float x = rx<DT, G>(b, g, j);
      bool keep = rcol<DT>(v0, j / VEC) < vend;
      if constexpr (MASKED) keep = keep & !row_masked(mk[g], x, ridx<DT>(v0, j));
      const float e = __builtin_amdgcn_exp2f((x - ref) * k.c1);
      acc += keep ? e : 0.f;
    }
    m[g] = lm;
    s[g] = acc;
  }
  const float2 st = block_stats_to_row_thread<G, kVWaves>(m, s, k.c1, s_pair);
  if ((int)threadIdx.x < k.nrows)
    slot_store(p.stat_slots + (int64_t)(k.row0 + threadIdx.x) * p.nc + k.c,
               pack_stats(st.x, st.x == -INFINITY ? 0.f : st.y));
}

// Chunk argmax of each row (NaN first, lowest index), published into the rows' arg slots.
template <int DT, int G, bool MASKED>
__device__ inline void resident_argmax(const VerifyParams& p, const RTask& k, int64_t v0,
                                       int64_t vend, const RBuf<DT, G>& b, const float4 (&mk)[G],
                                       uint64_t* s_key) {
  constexpr int VEC = Elem<DT>::kVec;
  uint64_t key[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float bv = -INFINITY;
    int bi = (int)v0;
#pragma unroll
    for (int j = 0; j < rcols<DT>(); ++j) {
      const int idx = ridx<DT>(v0, j);
      float v = rx<DT, G>(b, g, j);
      if constexpr (MASKED) v = row_masked(mk[g], v, idx) ? -INFINITY : v;
      // columns rise with j: a strict compare keeps the first maximum; NaN wins
      const bool take = ((v > bv) | ((v != v) & (bv == bv))) & (rcol<DT>(v0, j / VEC) < vend);
      bv = take ? v : bv;
      bi = take ? idx : bi;
    }
    key[g] = argmax_key(bv, bi);
  }
  const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_key);
  if ((int)threadIdx.x < k.nrows)
    slot_store(p.arg_slots + (int64_t)(k.row0 + threadIdx.x) * p.arg_stride + k.c, best);
}

// Scores max(p - q, 0) * (1 / E) of the chunk from the registers (MX, NL: the rows' raw max
// and -log2 of the softmax sum); the chunk argmax of each row goes into its arg slot.
template <int DT, int G, bool HAS_DRAFT, bool MASKED>
__device__ inline void resident_scores(const VerifyParams& p, const RTask& k, int64_t v0,
                                       int64_t vend, const RBuf<DT, G>& b,
                                       const RSide<DT, G, HAS_DRAFT, MASKED>& sd,
                                       const float (&MX)[G], const float (&NL)[G],
                                       uint64_t* s_key) {
  constexpr int VEC = Elem<DT>::kVec;
  float inv[rcols<DT>()];
#pragma unroll
  for (int j = 0; j < rcols<DT>(); ++j) inv[j] = recip_rn(raw_f32(sd.e, j));
  uint64_t key[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    // scores are >= 0 after the clamp and ties keep the lowest index, so starting from
    // (0, v0) and taking only strictly larger scores folds the clamp into the argmax
    float bv = 0.f;
    int bi = (int)v0;
    if (g < k.nrows) {
#pragma unroll
      for (int j = 0; j < rcols<DT>(); ++j) {
        const int idx = ridx<DT>(v0, j);
        const float x = rx<DT, G>(b, g, j);
        float prob = __builtin_amdgcn_exp2f(fmaf(x - MX[g], k.c1, NL[g]));  // softmax
        if constexpr (MASKED) prob = row_masked(sd.mk[g], x, idx) ? 0.f : prob;
        float w;
        if constexpr (HAS_DRAFT) w = prob - raw_f32(sd.q[g], j);
        else w = idx == sd.d[g] ? 0.f : prob;
        const float score = w * inv[j];
        const bool take = (score > bv) & (rcol<DT>(v0, j / VEC) < vend);
        bv = take ? score : bv;
        bi = take ? idx : bi;
      }
    }
    key[g] = argmax_key(bv, bi);
  }
  const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_key);
  if ((int)threadIdx.x < k.nrows)
    slot_store(p.arg_slots + (int64_t)(k.row0 + threadIdx.x) * p.arg_stride + k.c, best);
}

// The first poll of one row's nc stats slots (one wave; kPollKeep slots per lane kept).
// Every lane loads kPollKeep slots (clamped), so every path issues the same loads.
constexpr int kPollKeep = 2;
__device__ inline void poll_issue(const uint64_t* slots, int n, uint64_t (&v)[kPollKeep]) {
#pragma unroll
  for (int j = 0; j < kPollKeep; ++j) v[j] = slot_load(slots + min(lane_id() + j * kWave, n - 1));
}

// The rest of the wait for the row's slots (polls again until all are written), then their
// combination into the row's raw max MX and S = sum_c s_c * 2^((mx_c - MX) * c1), as
// wave_row_stats.  Returns false when the bounded wait ran out.
__device__ inline bool poll_finish(const uint64_t* slots, int n, float c1, const int* abort,
                                   uint64_t (&v)[kPollKeep], float& MX, float& S) {
  const int lane = lane_id();
  bool ok = true;
  for (int spins = 0;; ++spins) {
    int ready = 1;
#pragma unroll
    for (int j = 0; j < kPollKeep; ++j) ready &= (lane + j * kWave >= n) | (v[j] != 0);
    for (int c = lane + kPollKeep * kWave; c < n; c += kWave) ready &= slot_load(slots + c) != 0;
    if (__all(ready)) break;
    if (spins >= kSpinLimit || ((spins & 255) == 255 && atomic_load_relaxed(abort) != 0)) {
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    poll_issue(slots, n, v);
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kPollKeep; ++j)
    if (lane + j * kWave < n) m = fmaxf(m, unpack_stats(v[j]).x);
  for (int c = lane + kPollKeep * kWave; c < n; c += kWave) m = fmaxf(m, unpack_stats(slot_load(slots + c)).x);
  MX = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kPollKeep; ++j) {
    const float2 st = unpack_stats(v[j]);
    if (lane + j * kWave < n && st.x != -INFINITY) s += st.y * exp2f((st.x - MX) * c1);
  }
  for (int c = lane + kPollKeep * kWave; c < n; c += kWave) {
    const float2 st = unpack_stats(slot_load(slots + c));
    if (st.x != -INFINITY) s += st.y * exp2f((st.x - MX) * c1);
  }
  S = wave_sum(s);
  return ok;
}

template <int DT, int G, bool HAS_DRAFT, bool MASKED>
__global__ __launch_bounds__(kVThreads) MVSD_RESIDENT_ATTRS void verify_resident_kernel(VerifyParams p) {
  __shared__ float2 s_pair[G * kVWaves];
  __shared__ uint64_t s_key[G * kVWaves];
  __shared__ float s_MX[G];  // the group's statistics (raw max, -log2 sum) from the wait
  __shared__ float s_L[G];
  __shared__ int s_info[3][8];
  __shared__ int s_last;
  __shared__ FinalizeSmem fsm;
  __shared__ int s_goff[kMaxLdsRequests + 1];
  __shared__ int s_rbegin[kMaxLdsRequests], s_rkf[kMaxLdsRequests];
  __shared__ float s_rc1[kMaxLdsRequests];

  const int tid = threadIdx.x;
  int* ticket = &p.qticket[0];
  int t0 = 0, t1 = 0;
  if (tid == 0) {
    t0 = atomic_add_relaxed(ticket, 1);
    t1 = atomic_add_relaxed(ticket, 1);
  }
  const RequestMeta meta{s_rbegin, s_rkf, s_rc1};
  build_lds_tables(p, s_goff, meta);
  const int nc = p.nc;
  const int total = s_goff[p.B] * nc;
  if (tid == 0) {
    resident_decode(s_goff, meta, p.B, p.G, nc, total, t0, s_info[0]);
    resident_decode(s_goff, meta, p.B, p.G, nc, total, t1, s_info[1]);
  }
  __syncthreads();
  auto span = [&](const RTask& k, int64_t& v0, int64_t& vend) {
    v0 = (int64_t)k.c * p.chunk;
    vend = min((int64_t)p.V, v0 + p.chunk);
  };

  // Request completion: a task's count is examined one iteration later (F), so the counter's
  // round trip is never waited for on the task path; the last task of a request finalises it.
  int pend_cnt = 0, pend_r = -1, pend_target = 0;
  bool pend_greedy = false, pend_full = false;

  RTask cur = resident_read(s_info[0]);
  RTask nxt = resident_read(s_info[1]);
  int slot = 2;  // s_info slot of the next decode
  RBuf<DT, G> xa, xb;
  // The first-read step of a task: its statistics (greedy: its argmax), published per row.
  auto first_read = [&](const RTask& k, const RBuf<DT, G>& b) {
    if (k.t < 0) return;
    int64_t v0, vend;
    span(k, v0, vend);
    float4 mk[G];
    resident_masks<MASKED, G>(p, k, mk);
    if (k.flags & kGreedy) resident_argmax<DT, G, MASKED>(p, k, v0, vend, b, mk, s_key);
    else resident_stats<DT, G, MASKED>(p, k, v0, vend, b, mk, s_pair);
  };
  {
    int64_t v0, vend;
    span(cur, v0, vend);
    resident_load_x<DT, G>(p, cur, v0, vend, xa);
    first_read(cur, xa);
    span(nxt, v0, vend);
    resident_load_x<DT, G>(p, nxt, v0, vend, xb);
    __syncthreads();  // the row threads have read s_pair / s_key
  }

  // X holds the current task (statistics published), Y the next task's target (loads in
  // flight).
  auto iteration = [&](RBuf<DT, G>& X, RBuf<DT, G>& Y) -> bool {
    if (cur.t < 0) return false;
    const bool full = cur.flags & kFull;
    const bool poller = full && wave_id() < cur.nrows;
    const uint64_t* row_slots = p.stat_slots + (int64_t)(cur.row0 + min(wave_id(), cur.nrows - 1)) * nc;
    int64_t v0, vend;
    span(cur, v0, vend);
    // A: the first poll of the group's statistics, then the side loads of the current task
    uint64_t pv[kPollKeep];
    if (poller) poll_issue(row_slots, nc, pv);
    RSide<DT, G, HAS_DRAFT, MASKED> sd;
    if (full) resident_load_side<DT, G, HAS_DRAFT, MASKED>(p, cur, v0, vend, sd);
    // B: the next task's statistics (its target loads were issued one iteration ago)
    first_read(nxt, Y);
    // C: the rest of the wait for the current group's statistics
    float MX[G], NL[G];
    if (full) {
      if (poller) {
        float mx, sum;
        if (!poll_finish(row_slots, nc, cur.c1, &p.ctrl[1], pv, mx, sum) && lane_id() == 0)
          atomic_store_relaxed(&p.ctrl[1], 1);
        if (lane_id() == 0) {
          s_MX[wave_id()] = mx;
          s_L[wave_id()] = (float)(-log2((double)sum));
        }
      }
      __syncthreads();
#pragma unroll
      for (int g = 0; g < G; ++g) {
        MX[g] = s_MX[g];
        NL[g] = s_L[g];
      }
    }
    // D: claim a new ticket; its round trip overlaps the scores
    int tk = 0;
    if (tid == 0) tk = atomic_add_relaxed(ticket, 1);
    // E: scores of the current task, and its count
    if (full) resident_scores<DT, G, HAS_DRAFT, MASKED>(p, cur, v0, vend, X, sd, MX, NL, s_key);
    int cnt = 0;
    if (tid == 0) cnt = atomic_add_relaxed(&p.req_cnt[cur.r], 1);
    // F: decode the new ticket and check the previous task's count (the flag rides in the
    // decode slot, which no wave rewrites before every wave has read it)
    if (tid == 0) {
      resident_decode(s_goff, meta, p.B, p.G, nc, total, tk, s_info[slot]);
      s_info[slot][6] = pend_r >= 0 && pend_cnt == pend_target - 1 ? 1 : 0;
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(s_info[slot][6])) {
      finalize_request(p, s_goff, pend_r, pend_greedy, pend_full, fsm);
      __syncthreads();
    }
    pend_cnt = cnt;
    pend_r = cur.r;
    pend_target = (s_goff[cur.r + 1] - s_goff[cur.r]) * nc;  // every task of the request
    pend_greedy = cur.flags & kGreedy;
    pend_full = full;
    cur = nxt;
    nxt = resident_read(s_info[slot]);
    slot = slot == 2 ? 0 : slot + 1;
    int64_t n0, nend;
    span(nxt, n0, nend);
    resident_load_x<DT, G>(p, nxt, n0, nend, X);
    return true;
  };
  for (;;) {
    if (!iteration(xa, xb)) break;
    if (!iteration(xb, xa)) break;
  }
  if (pend_r >= 0) {
    if (tid == 0) s_last = pend_cnt == pend_target - 1;
    __syncthreads();
    if (s_last) finalize_request(p, s_goff, pend_r, pend_greedy, pend_full, fsm);
  }

  // The last workgroup out (every other one has made its final claim) returns the ticket and
  // the exit counter to zero.
  __syncthreads();
  if (tid == 0) s_last = atomic_add_relaxed(&p.ctrl[2], 1) == (int)gridDim.x - 1;
  __syncthreads();
  if (s_last) clear_masks(p);
  if (s_last && tid == 0) {
    atomic_store_relaxed(ticket, 0);
    atomic_store_relaxed(&p.ctrl[2], 0);
  }
}

// ------------------------------------------------------------------ parked kernel ----
// Single-read kernel with long streaming tasks (MVSD_VERIFY_MODE=lds).  A task is one (row
// group, chunk of kLdsSubs sub-chunks) pair holding both phases:
//   1. the group's target chunk streams through the split kernel's two-deep sub-chunk
//      pipeline into per-row statistics, and every thread parks its raw target vectors in
//      LDS; the statistics are published;
//   2. the chunk's draft and noise stream through the same pipeline; behind the first
//      sub-chunk's loads the workgroup waits for the group's statistics, then scores the
//      parked target against them.
// Each thread reads back only the vectors it parked, so the parking needs no barrier.
// Greedy tasks and tasks of requests with supplied recovered ids have phase 1 only.
//
// Progress.  The next ticket is claimed once the task's wait is over (tasks without a wait
// claim it behind their first loads) and decoded at the end of the task, so a workgroup never
// waits while it holds an unpublished ticket.  Take the lowest group g* anybody waits for:
// every workgroup holding an unpublished ticket of g* is in its phase 1, which has no wait,
// and publishes; if some ticket of g* is unclaimed, the workgroups not waiting for g* (those
// in other groups' tasks below g*, or between tasks) go on claiming, and a workgroup waiting
// for g* holds one ticket, so the claims of g* stop only if fewer workgroups are resident than
// g* has chunks (nc); the host keeps nc below the resident workgroups.  The waits are bounded
// all the same (kSpinLimit, flag ctrl[1]).
#ifndef MVSD_LDS_SUBS
#define MVSD_LDS_SUBS 4
#endif
constexpr int kLdsSubs = MVSD_LDS_SUBS;  // sub-chunks per task, all parked in LDS
constexpr int kLdsRequests = 1024;       // requests whose metadata fit beside the parked target

template <int DT, int EPT, int G, bool HAS_DRAFT, bool MASKED>
__global__ __launch_bounds__(kVThreads) void verify_lds_kernel(VerifyParams p) {
  constexpr int NV = EPT / Elem<DT>::kVec;
  __shared__ float s_red[G * kVWaves];
  __shared__ uint64_t s_key[G * kVWaves];
  __shared__ float s_M[G];
  __shared__ float s_L[G];
  __shared__ int s_info[2][8];
  __shared__ int s_last;
  __shared__ FinalizeSmem fsm;
  __shared__ int s_goff[kLdsRequests + 1];
  __shared__ int s_rbegin[kLdsRequests], s_rkf[kLdsRequests];
  __shared__ float s_rc1[kLdsRequests];
  __shared__ u32x4 s_park[kLdsSubs * G * NV * kVThreads];

  const int tid = threadIdx.x;
  int* ticket = &p.qticket[0];
  // the first ticket is claimed before the tables are built, so its round trip overlaps them
  int tfirst = 0;
  if (tid == 0) tfirst = atomic_add_relaxed(ticket, 1);
  const RequestMeta meta{s_rbegin, s_rkf, s_rc1};
  build_lds_tables(p, s_goff, meta);
  const int nc = p.nc;
  const int total = s_goff[p.B] * nc;
  if (tid == 0) resident_decode(s_goff, meta, p.B, p.G, nc, total, tfirst, s_info[0]);
  __syncthreads();

  // Deferred request-completion count: the counter's result is examined after the next task,
  // so its round trip is never waited for on the task path.
  int pend_cnt = 0, pend_r = -1, pend_target = 0;
  bool pend_greedy = false, pend_full = false;
  auto settle = [&]() {
    if (pend_r >= 0) {
      if (tid == 0) s_last = pend_cnt == pend_target - 1;
      __syncthreads();
      if (s_last) finalize_request(p, s_goff, pend_r, pend_greedy, pend_full, fsm);
      __syncthreads();
      pend_r = -1;
    }
  };

  for (int par = 0;; par ^= 1) {
    const RTask k = resident_read(s_info[par]);
    if (k.t < 0) break;
    int tn = 0;
    auto claim = [&]() {
      if (tid == 0) tn = atomic_add_relaxed(ticket, 1);
    };
    const bool greedy = k.flags & kGreedy;
    const bool full = k.flags & kFull;
    const int64_t v0 = (int64_t)k.c * p.chunk;
    const int64_t vend = min((int64_t)p.V, v0 + p.chunk);
    if (greedy) {
      task_argmax<DT, EPT, G, MASKED>(p, k.c, k.row0, k.nrows, v0, vend, s_key, claim);
    } else if (!full) {
      task_stats<DT, EPT, G, MASKED>(p, k.c, k.c1, k.row0, k.nrows, v0, vend, s_red, s_M, claim);
    } else {
      task_stats<DT, EPT, G, MASKED, true>(p, k.c, k.c1, k.row0, k.nrows, v0, vend, s_red, s_M,
                                           [] {}, s_park);
      task_scores<DT, EPT, G, HAS_DRAFT, MASKED, true>(p, k.c, k.r, k.c1, k.row0, k.nrows, v0,
                                                       vend, s_key, s_M, s_L, claim, s_park);
    }
    settle();
    if (tid == 0) pend_cnt = atomic_add_relaxed(&p.req_cnt[k.r], 1);
    pend_r = k.r;
    pend_target = (s_goff[k.r + 1] - s_goff[k.r]) * nc;  // every task of the request
    pend_greedy = greedy;
    pend_full = full;
    if (tid == 0) resident_decode(s_goff, meta, p.B, p.G, nc, total, tn, s_info[par ^ 1]);
    __syncthreads();
  }
  settle();

  // The last workgroup out (every other one has made its final claim) returns the ticket and
  // the exit counter to zero.
  if (tid == 0) s_last = atomic_add_relaxed(&p.ctrl[2], 1) == (int)gridDim.x - 1;
  __syncthreads();
  if (s_last) clear_masks(p);
  if (s_last && tid == 0) {
    atomic_store_relaxed(ticket, 0);
    atomic_store_relaxed(&p.ctrl[2], 0);
  }
}

// ------------------------------------------------------------------ workspace init ---
__global__ __launch_bounds__(256) void zero_fill_kernel(uint64_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = 0;
}

hipError_t launch_zero_fill(void* p, int64_t bytes, hipStream_t stream) {
  const int64_t n = bytes / 8;
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256),
                     0, stream, static_cast<uint64_t*>(p), n);
  return hipGetLastError();
}

// ------------------------------------------------------------------ dispatch ---------
constexpr int kGroup = MVSD_VERIFY_GROUP;
template <int DT>
constexpr int ept_of() {
  return DT == MVSD_F32 ? MVSD_VERIFY_EPT_F32 : MVSD_VERIFY_EPT_16;
}
#ifndef MVSD_VERIFY_MIN_SUBS
#define MVSD_VERIFY_MIN_SUBS 8
#endif
#ifndef MVSD_VERIFY_TASKS_PER_WG
#define MVSD_VERIFY_TASKS_PER_WG 10
#endif

VerifyPlan verify_plan(int target_dtype, int64_t vocab_size, int64_t groups, int phases, int cap) {
  VerifyPlan plan;
  plan.ept = target_dtype == MVSD_F32 ? ept_of<MVSD_F32>() : ept_of<MVSD_BF16>();
  plan.g = kGroup;
  plan.sub = kVThreads * plan.ept;
  plan.nsub = (int)((vocab_size + plan.sub - 1) / plan.sub);
  // Chunks per row: enough tasks for about MVSD_VERIFY_TASKS_PER_WG per resident workgroup,
  // each task as long as possible (fewer ticket claims, longer load pipelines), and at least
  // MVSD_VERIFY_MIN_SUBS sub-chunks per task so that small batches do not shred the rows into
  // tasks too short to amortise their start and end.
  int64_t nc = plan.nsub;
  if (groups > 0 && cap > 0) {
    nc = ((int64_t)MVSD_VERIFY_TASKS_PER_WG * cap + phases * groups - 1) / (phases * groups);
    const int64_t nc_max = plan.nsub / MVSD_VERIFY_MIN_SUBS;
    if (nc > nc_max) nc = nc_max;
    if (const char* env = getenv("MVSD_VERIFY_NC")) nc = atoi(env);
    nc = nc < 1 ? 1 : (nc > plan.nsub ? plan.nsub : nc);
  }
  const int64_t subs_per_chunk = (plan.nsub + nc - 1) / nc;
  plan.chunk = (int)(subs_per_chunk * plan.sub);
  plan.nc = (int)((vocab_size + plan.chunk - 1) / plan.chunk);
  return plan;
}

VerifyPlan verify_lds_plan(int target_dtype, int64_t vocab_size) {
  VerifyPlan plan;
  plan.ept = target_dtype == MVSD_F32 ? ept_of<MVSD_F32>() : ept_of<MVSD_BF16>();
  plan.g = kGroup;
  plan.sub = kVThreads * plan.ept;
  plan.chunk = kLdsSubs * plan.sub;
  plan.nc = (int)((vocab_size + plan.chunk - 1) / plan.chunk);
  plan.nsub = plan.nc;
  return plan;
}

int lds_max_requests() { return kLdsRequests; }

VerifyPlan verify_resident_plan(int target_dtype, int64_t vocab_size) {
  VerifyPlan plan;
  plan.ept = kRVecs * (target_dtype == MVSD_F32 ? 4 : 8);
  plan.g = kGroup;
  plan.sub = kVThreads * plan.ept;
  const int64_t nc = (vocab_size + plan.sub - 1) / plan.sub;
  const int64_t per = (vocab_size + nc - 1) / nc;
  plan.chunk = (int)((per + 63) / 64 * 64);
  plan.nc = (int)((vocab_size + plan.chunk - 1) / plan.chunk);
  plan.nsub = plan.nc;
  return plan;
}

template <int DT>
const void* kernel_for(int mode, bool has_draft, bool masked) {
  constexpr int E = ept_of<DT>();
  if (mode == kModeSplit) {
    if (masked)
      return has_draft ? reinterpret_cast<const void*>(&verify_kernel<DT, E, kGroup, true, true>)
                       : reinterpret_cast<const void*>(&verify_kernel<DT, E, kGroup, false, true>);
    return has_draft ? reinterpret_cast<const void*>(&verify_kernel<DT, E, kGroup, true, false>)
                     : reinterpret_cast<const void*>(&verify_kernel<DT, E, kGroup, false, false>);
  }
  if (mode == kModeLds) {
    if (masked)
      return has_draft ? reinterpret_cast<const void*>(&verify_lds_kernel<DT, E, kGroup, true, true>)
                       : reinterpret_cast<const void*>(&verify_lds_kernel<DT, E, kGroup, false, true>);
    return has_draft ? reinterpret_cast<const void*>(&verify_lds_kernel<DT, E, kGroup, true, false>)
                     : reinterpret_cast<const void*>(&verify_lds_kernel<DT, E, kGroup, false, false>);
  }
  if (mode == kModeResident) {
    if (masked)
      return has_draft ? reinterpret_cast<const void*>(&verify_resident_kernel<DT, kGroup, true, true>)
                       : reinterpret_cast<const void*>(&verify_resident_kernel<DT, kGroup, false, true>);
    return has_draft ? reinterpret_cast<const void*>(&verify_resident_kernel<DT, kGroup, true, false>)
                     : reinterpret_cast<const void*>(&verify_resident_kernel<DT, kGroup, false, false>);
  }
  if (masked)
    return has_draft ? reinterpret_cast<const void*>(&verify_fused_kernel<DT, E, kGroup, true, true>)
                     : reinterpret_cast<const void*>(&verify_fused_kernel<DT, E, kGroup, false, true>);
  return has_draft ? reinterpret_cast<const void*>(&verify_fused_kernel<DT, E, kGroup, true, false>)
                   : reinterpret_cast<const void*>(&verify_fused_kernel<DT, E, kGroup, false, false>);
}

int fused_max_chunks() {
  const int by_poll = kVThreads / kGroup;
  const int by_fifo = kFifo - kDepth - 5;
  return by_poll < by_fifo ? by_poll : by_fifo;
}

const void* verify_kernel_ptr(int target_dtype, int mode, bool has_draft, bool masked) {
  switch (target_dtype) {
    case MVSD_F32: return kernel_for<MVSD_F32>(mode, has_draft, masked);
    case MVSD_BF16: return kernel_for<MVSD_BF16>(mode, has_draft, masked);
    case MVSD_F16: return kernel_for<MVSD_F16>(mode, has_draft, masked);
    default: return nullptr;
  }
}

hipError_t launch_verify(const VerifyParams& params, int target_dtype, int mode, int grid,
                         hipStream_t stream) {
  hipError_t err = hipSuccess;
  if (!params.lds_groups) {
    hipLaunchKernelGGL(verify_init_kernel, dim3(1), dim3(1024), 0, stream, params);
    err = hipGetLastError();
  }
  if (err != hipSuccess || params.P == 0) return err;
  if (params.masks) {
    err = launch_constraints(params, target_dtype, stream);
    if (err != hipSuccess) return err;
  }
  const void* fn = verify_kernel_ptr(target_dtype, mode, params.draft != nullptr,
                                     params.masks != nullptr);
  if (!fn) return hipErrorInvalidValue;
  void* args[] = {const_cast<VerifyParams*>(&params)};
  err = hipLaunchKernel(fn, dim3(grid), dim3(kVThreads), args, 0, stream);
  if (err != hipSuccess) return err;
  return hipGetLastError();
}

}  // namespace mvsd
