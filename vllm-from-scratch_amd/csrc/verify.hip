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

#include "mvsd_device.h"
#include "verify.h"

namespace mvsd {

constexpr int kSpinLimit = 1 << 21;

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

__device__ inline int64_t target_row(const VerifyParams& p, int row) {
  if (!p.target_rows) return row;
  const int64_t t = p.target_rows[row];
  return t < 0 ? 0 : (t >= p.target_num_rows ? p.target_num_rows - 1 : t);
}

__device__ inline bool req_is_greedy(const VerifyParams& p, int r) {
  return p.all_greedy || p.temperature[r] == 0.f;
}

// Temperature applied to request r's rows: 1 unless apply_temperature; 0 (greedy) -> 1
// as expand_batch_to_tokens(replace_from=0, replace_to=1) does (rejection_sampler.py:553-559).
__device__ inline float req_temperature(const VerifyParams& p, int r) {
  if (!p.apply_temperature || p.all_greedy) return 1.f;
  const float t = p.temperature[r];
  return t == 0.f ? 1.f : t;
}

// x / t, correctly rounded, given rt = 1 / t correctly rounded (Markstein's correction:
// q0 = x * rt is within an ulp, the FMA residual x - q0 * t is exact, and q0 + residual * rt
// rounds to the IEEE quotient).  Three VALU ops instead of the ten of the IEEE sequence.
__device__ inline float div_by(float x, float t, float rt) {
  const float q0 = x * rt;
  return fmaf(fmaf(-q0, t, x), rt, q0);
}

// exp(d) for d <= 0 (or -inf): 2^(d log2 e) with the product split into a rounded head and
// an FMA-recovered tail so large |d| keeps full accuracy; ~1.5 ulp.
__device__ inline float exp_le0(float d) {
  constexpr float kLog2e = 1.44269502925872802734375f;      // RN(log2 e)
  constexpr float kLog2eLo = 1.925963033500011079e-08f;     // log2 e - kLog2e
  constexpr float kLn2 = 0.693147180559945309f;
  d = fmaxf(d, -200.f);  // exp(-200) underflows to 0; keeps the tail finite for -inf
  const float t = d * kLog2e;
  const float lo = fmaf(d, kLog2eLo, fmaf(d, kLog2e, -t));
  const float e = __builtin_amdgcn_exp2f(t);
  return fmaf(e, lo * kLn2, e);
}

// ------------------------------------------------------------------ loads ------------
// EPT consecutive-by-lane elements of one row chunk into fp32 registers.  FAST: full,
// aligned chunk, unconditional 16-byte loads.  Otherwise bounds-checked, `fill` beyond vend.
template <int DT, int EPT, bool FAST>
__device__ inline void load_chunk(const typename Elem<DT>::storage* __restrict__ base, int64_t v0,
                                  int64_t vend, bool aligned, float fill, float (&out)[EPT]) {
  using S = typename Elem<DT>::storage;
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int NV = EPT / VEC;
  const int tid = threadIdx.x;
  if constexpr (FAST) {
    u32x4 raw[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
      raw[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(base + v0 + ((int64_t)i * kVThreads + tid) * VEC));
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const S* s = reinterpret_cast<const S*>(&raw[i]);
#pragma unroll
      for (int j = 0; j < VEC; ++j) out[i * VEC + j] = Elem<DT>::cvt(s[j]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float tmp[VEC];
      load_vec<DT>(base, v0 + ((int64_t)i * kVThreads + tid) * VEC, vend, aligned, fill, tmp);
#pragma unroll
      for (int j = 0; j < VEC; ++j) out[i * VEC + j] = tmp[j];
    }
  }
}

// fp32 chunk whose lane layout follows a DT row (VEC elements of DT per 16-byte group).
template <int DT, int EPT, bool FAST>
__device__ inline void load_chunk_f32(const float* __restrict__ base, int64_t v0, int64_t vend,
                                      bool aligned, float fill, float (&out)[EPT]) {
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int NV = EPT / VEC;
  const int tid = threadIdx.x;
  if constexpr (FAST) {
    u32x4 raw[EPT / 4];
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int h = 0; h < VEC / 4; ++h)
        raw[i * (VEC / 4) + h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            base + v0 + ((int64_t)i * kVThreads + tid) * VEC + h * 4));
#pragma unroll
    for (int k = 0; k < EPT / 4; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) out[k * 4 + j] = __uint_as_float(raw[k][j]);
  } else {
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int h = 0; h < VEC; h += 4) {
        float tmp[4];
        load_vec<MVSD_F32>(base, v0 + ((int64_t)i * kVThreads + tid) * VEC + h, vend, aligned,
                           fill, tmp);
#pragma unroll
        for (int j = 0; j < 4; ++j) out[i * VEC + h + j] = tmp[j];
      }
  }
}

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
      for (int g = 0; g < ng; ++g) p.grp_req[first + g] = r;
    }
    __syncthreads();
    if (tid == 1023) s_carry = carry + s_scan[1023];
    __syncthreads();
  }
  if (tid == 0) p.grp_off[p.B] = s_carry;
}

// ------------------------------------------------------------------ row statistics ---
// Softmax statistics travel as (raw chunk max mx, sum of exp2((x - mx) * c1)) with
// c1 = log2(e) / T: for T > 0 the max of x / T is the max of x divided by T, so no per-element
// division is needed, and p = exp((x - MX) / T) / S = exp2(fma(x - MX, c1, -log2 S)).

// log2(e) / T rounded once from double.
__device__ inline float exp2_scale(float temp) {
  return (float)(1.4426950408889634074 / (double)temp);
}

// One wavefront: wait until the n stats slots of a row are written, then combine them into
// the row's raw max MX and S = sum_c s_c * 2^((mx_c - MX) * c1).  Up to 4 * 64 slots are kept
// in registers from the last poll.
__device__ inline bool wave_row_stats(const uint64_t* slots, int n, float c1, float& MX, float& S) {
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
    if (spins >= kSpinLimit) {
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
struct FinalizeSmem {
  int tok[kMaxSpecLen];
  float M[kMaxSpecLen];
  float S[kMaxSpecLen];
  int out_tok[kMaxSpecLen];
  int accepted[kMaxSpecLen];
  int first_reject;
};

// Executed by the whole block that completed request r's last task.
__device__ void finalize_request(const VerifyParams& p, int r, bool greedy, bool full,
                                 FinalizeSmem& sm) {
  int begin, K;
  req_range(p, r, begin, K);
  const int lane = lane_id();
  const int nc = p.nc;
  for (int k = wave_id(); k < K; k += kVWaves) {
    const int64_t row = begin + k;
    uint64_t* aslots = p.arg_slots + row * nc;
    uint64_t* sslots = p.stat_slots + row * nc;
    if (greedy || full) {
      if (!wave_wait_slots(aslots, nc, kSpinLimit) && lane == 0) atomic_store_relaxed(&p.ctrl[1], 1);
      uint64_t best = 0;
      for (int c = lane; c < nc; c += kWave) {
        const uint64_t k = slot_load(aslots + c);
        best = k > best ? k : best;
      }
      best = wave_max_u64(best);
      if (lane == 0) sm.tok[k] = min(max(key_index(best), 0), p.V - 1);
      for (int c = lane; c < nc; c += kWave) slot_store(aslots + c, 0);
    } else if (lane == 0) {
      sm.tok[k] = p.recovered[row];
    }
    if (!greedy) {
      const float c1 = exp2_scale(req_temperature(p, r));
      float MX, S;
      if (!wave_row_stats(sslots, nc, c1, MX, S) && lane == 0) atomic_store_relaxed(&p.ctrl[1], 1);
      if (lane == 0) {
        sm.M[k] = MX;
        sm.S[k] = S;
      }
      for (int c = lane; c < nc; c += kWave) slot_store(sslots + c, 0);
    }
  }
  if (threadIdx.x == 0) atomic_store_relaxed(&p.req_cnt[r], 0);
  __syncthreads();

  // every position's decision in parallel; the chain keeps the prefix up to the first reject
  const int tid = threadIdx.x;
  const bool synthetic = p.synth != nullptr;
  for (int pos = tid; pos < K; pos += kVThreads) {
    const int64_t row = begin + pos;
    const int d = p.draft_ids[row];
    bool accepted;
    int token;
    if (greedy) {
      // rejection_sampler.py:715-732
      if (synthetic) {
        accepted = p.uniforms[row] < (double)p.synth[pos] && d >= 0;
        token = accepted ? d : sm.tok[pos];
      } else {
        token = sm.tok[pos];
        accepted = d == token;
      }
    } else {
      // rejection_sampler.py:782-814
      const double u = p.uniforms[row];
      if (d < 0) {
        accepted = false;
      } else if (synthetic) {
        accepted = u < (double)p.synth[pos];
      } else if (d >= p.V) {
        accepted = false;  // the reference would index out of bounds here
      } else {
        const float q = p.draft ? p.draft[row * p.draft_stride + d] : 1.f;
        const int64_t trow = target_row(p, (int)row);
        float x;
        if (p.target_dtype == MVSD_F32) {
          x = static_cast<const float*>(p.target)[trow * p.target_stride + d];
        } else if (p.target_dtype == MVSD_BF16) {
          x = Elem<MVSD_BF16>::cvt(static_cast<const uint16_t*>(p.target)[trow * p.target_stride + d]);
        } else {
          x = Elem<MVSD_F16>::cvt(static_cast<const _Float16*>(p.target)[trow * p.target_stride + d]);
        }
        const float temp = req_temperature(p, r);
        const float pd = expf(x / temp - sm.M[pos] / temp) / sm.S[pos];
        accepted = q > 0.f && (double)(pd / q) >= u;
      }
      token = accepted ? d : sm.tok[pos];
    }
    sm.accepted[pos] = accepted;
    sm.out_tok[pos] = token;
  }
  __syncthreads();
  if (tid == 0) {
    int first = K;
    for (int pos = 0; pos < K; ++pos) {
      if (!sm.accepted[pos]) {
        first = pos;
        break;
      }
    }
    sm.first_reject = first;
  }
  __syncthreads();
  const int first = sm.first_reject;
  int32_t* out = p.out + (int64_t)r * p.out_stride;
  for (int pos = tid; pos <= K; pos += kVThreads) {
    if (pos < K && pos <= first) out[pos] = sm.out_tok[pos];
    else if (pos == K && first == K) out[K] = p.bonus[r];
  }
}

// ------------------------------------------------------------------ tasks ------------

// The group's target slice into registers (-inf beyond V and for rows >= nrows).
template <int DT, int EPT, int G, bool FAST>
__device__ inline void load_rows(const VerifyParams& p, int row0, int nrows, int64_t v0,
                                 int64_t vend, float (&x)[G][EPT]) {
  using S = typename Elem<DT>::storage;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (g < nrows) {
      const S* base = static_cast<const S*>(p.target) + target_row(p, row0 + g) * p.target_stride;
      load_chunk<DT, EPT, FAST>(base, v0, vend, p.target_aligned, -INFINITY, x[g]);
    } else {
#pragma unroll
      for (int k = 0; k < EPT; ++k) x[g][k] = -INFINITY;
    }
  }
}

// Value of a per-row register array for row = this thread's index (threads < G).
template <int G, typename T>
__device__ inline T row_of_thread(const T (&a)[G]) {
  T v = a[0];
#pragma unroll
  for (int g = 1; g < G; ++g) v = (int)threadIdx.x == g ? a[g] : v;
  return v;
}

// Greedy task: chunk-local argmax of the raw logits (NaN first, lowest index wins).
template <int DT, int EPT, int G, bool FAST>
__device__ inline void task_argmax(const VerifyParams& p, int c, int row0, int nrows, int64_t v0,
                                   int64_t vend, uint64_t* s_key) {
  float x[G][EPT];
  load_rows<DT, EPT, G, FAST>(p, row0, nrows, v0, vend, x);
  uint64_t key[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float bv = -INFINITY;
    int bi = (int)v0;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int idx = elem_index<DT, EPT>(v0, k);
      const float v = x[g][k];
      // indices rise along k: a strict compare keeps the first maximum; a NaN beats numbers
      const bool take = ((v > bv) | ((v != v) & (bv == bv))) & (FAST || idx < vend);
      bv = take ? v : bv;
      bi = take ? idx : bi;
    }
    key[g] = argmax_key(bv, bi);
  }
  const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_key);
  if ((int)threadIdx.x < nrows) slot_store(p.arg_slots + (int64_t)(row0 + threadIdx.x) * p.nc + c, best);
}

// A-task: per row of the group, the chunk's raw max and sum of exp2((x - mx) * c1).
template <int DT, int EPT, int G, bool FAST>
__device__ inline void task_stats(const VerifyParams& p, int c, int r, int row0, int nrows,
                                  int64_t v0, int64_t vend, float* s_red) {
  float x[G][EPT];
  load_rows<DT, EPT, G, FAST>(p, row0, nrows, v0, vend, x);
  const float c1 = exp2_scale(req_temperature(p, r));
  float m[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mm = -INFINITY;
#pragma unroll
    for (int k = 0; k < EPT; ++k) mm = fmaxf(mm, x[g][k]);
    m[g] = mm;
  }
  block_max<G, kVWaves>(m, s_red);
  float s[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mg = m[g] == -INFINITY ? 0.f : m[g];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < EPT; ++k) ss += __builtin_amdgcn_exp2f((x[g][k] - mg) * c1);
    s[g] = ss;
  }
  const float srow = block_sum_to_row_thread<G, kVWaves>(s, s_red);
  if ((int)threadIdx.x < nrows) {
    const float mrow = row_of_thread<G>(m);
    slot_store(p.stat_slots + (int64_t)(row0 + threadIdx.x) * p.nc + c,
               pack_stats(mrow, mrow == -INFINITY ? 0.f : srow));
  }
}

// B-task: per row of the group, the chunk-local argmax of max(p - q, 0) * (1 / E).  All of
// the task's loads (the target slice again, noise chunk, draft chunks) are issued up front;
// the group's stats were published by A-tasks holding lower tickets.
template <int DT, int EPT, int G, bool FAST>
__device__ inline void task_scores(const VerifyParams& p, int c, int r, int row0, int nrows,
                                   int64_t v0, int64_t vend, uint64_t* s_key, float* s_M,
                                   float* s_L) {
  float x[G][EPT];
  load_rows<DT, EPT, G, FAST>(p, row0, nrows, v0, vend, x);
  float inv[EPT];
  load_chunk_f32<DT, EPT, FAST>(p.noise + (int64_t)r * p.noise_stride, v0, vend, p.noise_aligned,
                                1.f, inv);
  float q[G][EPT];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (p.draft && g < nrows) {
      load_chunk_f32<DT, EPT, FAST>(p.draft + (int64_t)(row0 + g) * p.draft_stride, v0, vend,
                                    p.draft_aligned, 0.f, q[g]);
    } else {
#pragma unroll
      for (int k = 0; k < EPT; ++k) q[g][k] = 0.f;
    }
  }
  const float c1 = exp2_scale(req_temperature(p, r));
  if (wave_id() < nrows) {
    float MX, S;
    if (!wave_row_stats(p.stat_slots + (int64_t)(row0 + wave_id()) * p.nc, p.nc, c1, MX, S) &&
        lane_id() == 0)
      atomic_store_relaxed(&p.ctrl[1], 1);
    if (lane_id() == 0) {
      s_M[wave_id()] = MX;
      s_L[wave_id()] = (float)(-log2((double)S));
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < EPT; ++k) inv[k] = 1.0f / inv[k];
  uint64_t key[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float bv = -INFINITY;
    int bi = (int)v0;
    if (g < nrows) {
      const float MX = s_M[g];
      const float nl = s_L[g];
      const int d = p.draft ? -1 : p.draft_ids[row0 + g];
#pragma unroll
      for (int k = 0; k < EPT; ++k) {
        const int idx = elem_index<DT, EPT>(v0, k);
        const float prob = __builtin_amdgcn_exp2f(fmaf(x[g][k] - MX, c1, nl));  // softmax
        const float w = p.draft ? fmaxf(prob - q[g][k], 0.f) : (idx == d ? 0.f : prob);
        const float score = w * inv[k];
        // indices rise along k, so a strict compare keeps the first maximum
        const bool take = (score > bv) & (FAST || idx < vend);
        bv = take ? score : bv;
        bi = take ? idx : bi;
      }
    }
    key[g] = argmax_key(bv, bi);
  }
  const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_key);
  if ((int)threadIdx.x < nrows) slot_store(p.arg_slots + (int64_t)(row0 + threadIdx.x) * p.nc + c, best);
}

// ------------------------------------------------------------------ main kernel ------
// Tunables (compile-time): elements per thread per row, and an optional cap on waves per SIMD
// that bounds the register budget (0 = let the compiler choose).
#ifndef MVSD_VERIFY_EPT
#define MVSD_VERIFY_EPT 8
#endif
#ifndef MVSD_VERIFY_WAVES_PER_EU
#define MVSD_VERIFY_WAVES_PER_EU 0
#endif
#if MVSD_VERIFY_WAVES_PER_EU > 0
#define MVSD_VERIFY_ATTRS __attribute__((amdgpu_waves_per_eu(MVSD_VERIFY_WAVES_PER_EU, 8)))
#else
#define MVSD_VERIFY_ATTRS
#endif

// Ticket t -> step s = t / steps_size: the first nc tickets of step s are the A-chunks (stats,
// or the argmax for greedy groups) of group s; when the batch has random requests the next nc
// are the B-chunks (scores) of group s - lag.  Slots of absent groups are claimed and skipped.
template <int DT, int EPT, int G>
__global__ __launch_bounds__(kVThreads) MVSD_VERIFY_ATTRS void verify_kernel(VerifyParams p) {
  static_assert(EPT % Elem<DT>::kVec == 0, "EPT must be a multiple of the vector width");
  __shared__ float s_red[G * kVWaves];
  __shared__ uint64_t s_key[G * kVWaves];
  __shared__ float s_M[G];
  __shared__ float s_L[G];
  __shared__ int s_task;
  __shared__ int s_last;
  __shared__ FinalizeSmem fsm;

  const int tid = threadIdx.x;
  const int nc = p.nc;
  const int lag = p.lag;
  const int groups = p.grp_off[p.B];
  const int step_size = p.two_phase ? 2 * nc : nc;
  const int total = (groups + (p.two_phase ? lag : 0)) * step_size;

  for (;;) {
    if (tid == 0) s_task = atomic_add_relaxed(&p.ctrl[0], 1);
    __syncthreads();
    const int t = s_task;
    __syncthreads();
    if (t >= total) break;

    const int step = t / step_size;
    const int w = t - step * step_size;
    const bool phase_b = w >= nc;
    const int c = phase_b ? w - nc : w;
    const int gi = phase_b ? step - lag : step;
    if (gi < 0 || gi >= groups) continue;
    const int r = p.grp_req[gi];
    int begin, K;
    req_range(p, r, begin, K);
    const int g0 = gi - p.grp_off[r];
    const int row0 = begin + g0 * G;
    const int nrows = min(G, K - g0 * G);
    const int ngr = (K + G - 1) / G;
    const bool greedy = req_is_greedy(p, r);
    const bool full = !greedy && p.recovered == nullptr;
    if (phase_b && !full) continue;
    const int64_t v0 = (int64_t)c * p.chunk;
    const int64_t vend = min((int64_t)p.V, v0 + p.chunk);
    const bool fast = p.target_aligned && vend - v0 == p.chunk &&
                      (!phase_b || (p.noise_aligned && (p.draft_aligned || !p.draft)));
    if (greedy) {
      if (fast) task_argmax<DT, EPT, G, true>(p, c, row0, nrows, v0, vend, s_key);
      else task_argmax<DT, EPT, G, false>(p, c, row0, nrows, v0, vend, s_key);
    } else if (!phase_b) {
      if (fast) task_stats<DT, EPT, G, true>(p, c, r, row0, nrows, v0, vend, s_red);
      else task_stats<DT, EPT, G, false>(p, c, r, row0, nrows, v0, vend, s_red);
    } else {
      if (fast) task_scores<DT, EPT, G, true>(p, c, r, row0, nrows, v0, vend, s_key, s_M, s_L);
      else task_scores<DT, EPT, G, false>(p, c, r, row0, nrows, v0, vend, s_key, s_M, s_L);
    }
    // ---- request completion: the last counted task runs the accept/reject chain ----
    // (counted: B-tasks of full random requests, A-tasks otherwise)
    if (full == phase_b) {
      if (tid == 0) s_last = atomic_add_relaxed(&p.req_cnt[r], 1) == ngr * nc - 1;
      __syncthreads();
      if (s_last) finalize_request(p, r, greedy, full, fsm);
    }
    __syncthreads();
  }

  // The last workgroup out (every other one has made its final claim and finished reading
  // grp_off / grp_req) returns the group tables, ticket and exit counter to zero, so the whole
  // workspace is zero again whatever layout the next call uses.
  if (tid == 0) s_last = atomic_add_relaxed(&p.ctrl[2], 1) == (int)gridDim.x - 1;
  __syncthreads();
  if (s_last) {
    for (int i = tid; i <= p.B; i += kVThreads) p.grp_off[i] = 0;
    for (int i = tid; i < groups; i += kVThreads) p.grp_req[i] = 0;
    if (tid == 0) {
      atomic_store_relaxed(&p.ctrl[0], 0);
      atomic_store_relaxed(&p.ctrl[2], 0);
    }
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
constexpr int kEpt = MVSD_VERIFY_EPT;
constexpr int kGroup = 4;

VerifyPlan verify_plan(int target_dtype, int64_t vocab_size) {
  VerifyPlan plan;
  plan.ept = kEpt;
  plan.g = kGroup;
  plan.chunk = kVThreads * plan.ept;
  plan.nc = (int)((vocab_size + plan.chunk - 1) / plan.chunk);
  (void)target_dtype;
  return plan;
}

const void* verify_kernel_ptr(int target_dtype) {
  switch (target_dtype) {
    case MVSD_F32: return reinterpret_cast<const void*>(&verify_kernel<MVSD_F32, kEpt, kGroup>);
    case MVSD_BF16: return reinterpret_cast<const void*>(&verify_kernel<MVSD_BF16, kEpt, kGroup>);
    case MVSD_F16: return reinterpret_cast<const void*>(&verify_kernel<MVSD_F16, kEpt, kGroup>);
    default: return nullptr;
  }
}

hipError_t launch_verify(const VerifyParams& params, int target_dtype, int grid,
                         hipStream_t stream) {
  hipLaunchKernelGGL(verify_init_kernel, dim3(1), dim3(1024), 0, stream, params);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || params.P == 0) return err;
  switch (target_dtype) {
    case MVSD_F32:
      hipLaunchKernelGGL((verify_kernel<MVSD_F32, kEpt, kGroup>), dim3(grid), dim3(kVThreads), 0,
                         stream, params);
      break;
    case MVSD_BF16:
      hipLaunchKernelGGL((verify_kernel<MVSD_BF16, kEpt, kGroup>), dim3(grid), dim3(kVThreads), 0,
                         stream, params);
      break;
    case MVSD_F16:
      hipLaunchKernelGGL((verify_kernel<MVSD_F16, kEpt, kGroup>), dim3(grid), dim3(kVThreads), 0,
                         stream, params);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mvsd
