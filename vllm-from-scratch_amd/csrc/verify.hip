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
// The reference scores a recovered id for every verify row (:627-670) and keeps only the one
// at the first rejection (:806-814).  This kernel decides each request's chain first and then
// scores only that row, so it reads every target row once, plus, for each random request with
// a rejection, that one row's target, draft and noise once more.  The outputs are the same.
//
// One persistent launch over a ticket counter:
//   * Stats units: a group of up to G rows of one request, as NC tasks of one column chunk
//     each.  Random rows publish, per chunk, a slot with (raw max, sum of
//     exp2((x - max) * log2(e) / T)); greedy rows publish the chunk's argmax key.
//   * The last stats task of a request to start (relaxed atomic count) decides it: per row
//     it combines the row's slots into (max, sum) or the argmax, reads the draft id, q[d],
//     x[d] and the uniform, and finds the first rejection.  Greedy requests and random
//     requests whose recovered ids are supplied get their output row right there.  Other
//     random requests publish the decision (first rejected position, or none) in the
//     request's decision slot.
//   * Score units: one per such random request (NC tasks), placed LAG stats units after the
//     request's last stats unit, so that the decision is normally there when they start.  A
//     score task reads the decision; with a rejection at row j it streams chunk c of target
//     row j, draft row j and the request's noise row and publishes the chunk's argmax of
//     max(p - q, 0) * (1 / E).  The last of them to start writes the request's output row.
//     Every output row therefore has exactly one writer.
//   * Tasks are counted when they start.  The last stats task of a request to start decides the
//     request right after its own work, waiting only for the slots of the request's other stats
//     tasks, which have started and never wait; likewise the last score task to start finishes
//     the request.  A score task waits for its request's decision, which depends only on stats
//     tasks holding lower tickets.  So no wait can deadlock.  Every wait is still
//     bounded: a wait that gives up sets the failure flag, after which the other waits give up
//     quickly; the writer of each request whose inputs are incomplete fills its output row
//     with kPoison, and the last workgroup out clears the workspace.
//   * Slots are 64-bit values exchanged with relaxed agent-scope atomics; 0 means empty and
//     no written slot is 0, so readers poll the data itself and no fence (no L2 write-back or
//     invalidation) is needed.  Every call leaves the workspace zeroed for the next one.
#include <float.h>
#include <stdint.h>
#include <stdlib.h>

#include <type_traits>

#include "mvsd_device.h"
#include "verify.h"

namespace mvsd {

// Request r's verify rows [begin, begin + K), clamped so that inconsistent metadata can
// produce wrong tokens but never an out-of-bounds access: 0 <= begin <= begin + K <= P and
// K <= max_spec_len.
__device__ inline void req_range(const VerifyParams& p, int r, int& begin, int& K) {
  int b = r == 0 ? (p.cu_prev ? p.cu_prev[0] : 0) : p.cu[r - 1];
  int e = p.cu[r];
  b = min(max(b, 0), p.P);
  e = min(max(e, b), p.P);
  begin = b;
  K = min(e - b, p.max_spec_len);
}

// Slots per verify row (and per request for the scores): one per task of a row, up to two per
// chunk (tasks at the end of a launch cover half chunks).
__device__ inline int64_t slot_stride(const VerifyParams& p) { return 2 * (int64_t)p.nc; }

// log2(e) / T rounded once from double.
__device__ inline float exp2_scale(float temp) {
  return (float)(1.4426950408889634074 / (double)temp);
}

// Request flags.
constexpr int kGreedy = 1;
constexpr int kFull = 2;  // random request whose recovered id comes from in-kernel scores

// Per-request tables in LDS, built by every workgroup at start: first group, first verify
// row, rows (clamped as by req_range) with the flags above bit 16, log2(e) / T, and the
// score units (position in the unit order << 12 | request) of the kFull requests.
struct Tables {
  int* gpos;    // [B + 1] by position: first group << 12 | request; gpos[B] = groups << 12
  int* gstart;  // [B] first group of request r
  int* begin;  // [B]
  int* kflags;  // [B]
  float* c1;   // [B]
  int* fpos;   // [F]
  int groups;
  int nfull;
  // The launch's tail, run in half-chunk tasks: stats units of groups >= gt, score units of
  // ordinal >= kt; u0 = the first tail unit's position.
  int gt, kt, u0;
};

// ------------------------------------------------------------------ loads ------------
// Column of element k of this thread in the sub-chunk starting at v0: 16-byte vectors of kVec
// elements, consecutive lanes on consecutive vectors.
template <int DT, int EPT>
__device__ inline int elem_index(int64_t v0, int k) {
  constexpr int VEC = Elem<DT>::kVec;
  return (int)(v0 + ((int64_t)(k / VEC) * kVThreads + threadIdx.x) * VEC + (k % VEC));
}

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

// Target loads.  The stats tasks' loads are temporal, so that a row a score task reads again
// shortly afterwards is still in the Infinity Cache; the score tasks' loads are the last use
// and stream non-temporally.
template <bool NT>
__device__ inline u32x4 load16(const void* p) {
  const u32x4* q = static_cast<const u32x4*>(p);
  if constexpr (NT) return __builtin_nontemporal_load(q);
  else return *q;
}

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

// DT row sub-chunk, full and aligned.
template <int DT, int EPT, bool NT>
__device__ inline void load_raw(const typename Elem<DT>::storage* __restrict__ base, int64_t s0,
                                u32x4 (&out)[EPT / Elem<DT>::kVec]) {
#pragma unroll
  for (int i = 0; i < EPT / Elem<DT>::kVec; ++i) out[i] = load16<NT>(base + vec_col<DT>(s0, i));
}

// DT row sub-chunk, bounds-checked: elements at or beyond vend read as `fill`.
template <int DT, int EPT, bool NT>
__device__ inline void load_raw_checked(const typename Elem<DT>::storage* __restrict__ base,
                                        int64_t s0, int64_t vend, bool aligned,
                                        typename Elem<DT>::storage fill,
                                        u32x4 (&out)[EPT / Elem<DT>::kVec]) {
  constexpr int VEC = Elem<DT>::kVec;
#pragma unroll
  for (int i = 0; i < EPT / VEC; ++i) {
    const int64_t col = vec_col<DT>(s0, i);
    if (aligned && col + VEC <= vend) out[i] = load16<NT>(base + col);
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

// Draft probabilities of a thread's EPT elements in one sub-chunk, in the target's column
// layout: fp32 (one word per element) or bf16 / fp16 (two per word), upcast when consumed.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int DD, int EPT>
struct DraftBuf {
  static constexpr int kWords = DD == MVSD_F32 ? EPT : EPT / 2;
  uint32_t w[kWords];
};

template <int DD>
__device__ inline float draft_elem(const uint32_t* w, int k) {
  if constexpr (DD == MVSD_F32) {
    return __uint_as_float(w[k]);
  } else {
    const uint16_t h = (uint16_t)(w[k / 2] >> (16 * (k % 2)));
    return Elem<DD>::cvt(__builtin_bit_cast(typename Elem<DD>::storage, h));
  }
}

// Draft sub-chunk for the columns of the DT layout; FAST: full and aligned, else
// bounds-checked (columns at or past vend read as 0).
template <int DT, int DD, int EPT, bool FAST>
__device__ inline void load_draft(const void* base_v, int64_t s0, int64_t vend, bool aligned,
                                  DraftBuf<DD, EPT>& q) {
  constexpr int VEC = Elem<DT>::kVec;
  if constexpr (DD == MVSD_F32) {
    u32x4 raw[EPT / 4];
    load_raw_f32<DT, EPT, FAST>(static_cast<const float*>(base_v), s0, vend, aligned, 0.f, raw);
#pragma unroll
    for (int m = 0; m < EPT / 4; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) q.w[4 * m + j] = raw[m][j];
  } else {
    using S = typename Elem<DD>::storage;
    const S* base = static_cast<const S*>(base_v);
#pragma unroll
    for (int i = 0; i < EPT / VEC; ++i) {
      const int64_t col = vec_col<DT>(s0, i);
      if (FAST || (aligned && col + VEC <= vend)) {
        if constexpr (VEC == 4) {
          const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(base + col));
          q.w[2 * i] = v[0];
          q.w[2 * i + 1] = v[1];
        } else {
          const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + col));
#pragma unroll
          for (int j = 0; j < 4; ++j) q.w[4 * i + j] = v[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < VEC / 2; ++j) {
          const uint32_t lo = col + 2 * j < vend ? bits16(base[col + 2 * j]) : 0u;
          const uint32_t hi = col + 2 * j + 1 < vend ? bits16(base[col + 2 * j + 1]) : 0u;
          q.w[i * (VEC / 2) + j] = lo | hi << 16;
        }
      }
    }
  }
}

// Walk [v0, vend) in SUB-column sub-chunks: load(buf, s0, Fast<bool>) issues a sub-chunk's
// loads, body(buf, s0, Fast<bool>) consumes them.  hook() runs once, after the first loads
// are issued.  Unaligned inputs and the partial last sub-chunk take the checked path.
// The loads of sub-chunk j + 1 are issued before body(j), unconditionally (past the end of
// the run they reload the final sub-chunk, a cache hit): every path then issues the same
// loads, so the compiler's in-order load counter lets body(j) wait for sub-chunk j alone
// while the next one is in flight.
template <int SUB, typename Buf, typename Load, typename Body, typename Hook>
__device__ inline void pipeline(int64_t v0, int64_t vend, bool aligned, Load&& load, Body&& body,
                                Hook&& hook) {
  const int nfull = aligned ? (int)((vend - v0) / SUB) : 0;
  auto at = [&](int j) { return v0 + (int64_t)min(j, nfull - 1) * SUB; };
  if (nfull > 0) {
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
  } else {
    hook();
  }
  for (int64_t s0 = v0 + (int64_t)nfull * SUB; s0 < vend; s0 += SUB) {
    Buf t;
    load(t, s0, Fast<false>());
    body(t, s0, Fast<false>());
  }
}

// ------------------------------------------------------------------ waits ------------
// One wavefront polls the n slots at `slots` until every one is written, keeping the first
// kKeep * 64 of them in registers (v[j] holds slot lane + 64 j).  Gives up after
// p.spin_limit polls, or sooner once the failure flag ctrl[kCtrlFlag] is set (so one wait that
// cannot complete ends every other wait quickly); giving up sets the flag and returns false.
// first_read: v already holds a first read of those slots (wave_read_slots), issued ahead of
// other loads so that the in-order load counter does not hold the poll behind them.
constexpr int kKeep = 2;

__device__ inline void wave_read_slots(const uint64_t* slots, int n, uint64_t (&v)[kKeep]) {
#pragma unroll
  for (int j = 0; j < kKeep; ++j) {
    const int c = lane_id() + j * kWave;
    v[j] = c < n ? slot_load(slots + c) : 0;
  }
}

__device__ inline bool wave_poll(const VerifyParams& p, const uint64_t* slots, int n,
                                 uint64_t (&v)[kKeep], bool first_read = false) {
  const int lane = lane_id();
  if (!first_read) {
#pragma unroll
    for (int j = 0; j < kKeep; ++j) v[j] = 0;
  }
  for (int spins = 0;; ++spins) {
    if (spins >= p.spin_limit) break;
    int ready = 1;
#pragma unroll
    for (int j = 0; j < kKeep; ++j) {
      const int c = lane + j * kWave;
      if (!first_read || spins > 0) v[j] = c < n ? slot_load(slots + c) : 0;
      ready &= (c >= n) | (v[j] != 0);
    }
    for (int c = lane + kKeep * kWave; c < n; c += kWave) ready &= slot_load(slots + c) != 0;
    if (__all(ready)) return true;
    if ((spins & 255) == 255 && atomic_load_relaxed(&p.ctrl[kCtrlFlag]) != 0) break;
    __builtin_amdgcn_s_sleep(1);
  }
  if (lane == 0) atomic_store_relaxed(&p.ctrl[kCtrlFlag], 1);
  return false;
}

// Row statistics from its n polled stats slots: raw max MX and S = sum_c s_c * 2^((mx_c - MX)
// * c1).  Every lane receives the same values.
__device__ inline void combine_stats(const uint64_t* slots, int n, const uint64_t (&v)[kKeep],
                                     float c1, float& MX, float& S) {
  const int lane = lane_id();
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kKeep; ++j)
    if (lane + j * kWave < n) m = fmaxf(m, unpack_stats(v[j]).x);
  for (int c = lane + kKeep * kWave; c < n; c += kWave) m = fmaxf(m, unpack_stats(slot_load(slots + c)).x);
  MX = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kKeep; ++j) {
    const float2 st = unpack_stats(v[j]);
    if (lane + j * kWave < n && st.x != -INFINITY) s += st.y * exp2f((st.x - MX) * c1);
  }
  for (int c = lane + kKeep * kWave; c < n; c += kWave) {
    const float2 st = unpack_stats(slot_load(slots + c));
    if (st.x != -INFINITY) s += st.y * exp2f((st.x - MX) * c1);
  }
  S = wave_sum(s);
}

// Largest of n polled argmax keys (every lane receives it).
__device__ inline uint64_t combine_keys(const uint64_t* slots, int n, const uint64_t (&v)[kKeep]) {
  uint64_t best = 0;
#pragma unroll
  for (int j = 0; j < kKeep; ++j) best = v[j] > best ? v[j] : best;
  for (int c = lane_id() + kKeep * kWave; c < n; c += kWave) {
    const uint64_t k = slot_load(slots + c);
    best = k > best ? k : best;
  }
  return wave_max_u64(best);
}

__device__ inline void wave_clear(uint64_t* slots, int n) {
  for (int c = lane_id(); c < n; c += kWave) slot_store(slots + c, 0);
}

// ------------------------------------------------------------------ stats tasks ------
// A stats task covers rows [row0, row0 + nrows) of one group and columns [v0, vend), walked
// in sub-chunks of kVThreads * EPT columns, double-buffered by pipeline().  Buffers hold the
// raw 16-byte vectors; elements are converted to fp32 only when they are consumed.

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
__device__ inline auto target_loader(const VerifyParams& p, const typename Elem<DT>::storage* (&tb)[G],
                                     int64_t vend) {
  // every row slot loads (rows past nrows repeat the last row), so every path issues the
  // same loads
  return [&p, &tb, vend](TargetBuf<DT, EPT, G>& buf, int64_t s0, auto fast) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if constexpr (decltype(fast)::value)
        load_raw<DT, EPT, false>(tb[g], s0, buf.x[g]);
      else
        load_raw_checked<DT, EPT, false>(tb[g], s0, vend, p.target_aligned, Elem<DT>::ninf(),
                                         buf.x[g]);
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

// Greedy rows: chunk-local argmax of the raw logits (NaN first, lowest index wins); with
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
  if constexpr (Elem<DT>::kVec == 8) {
    // 16-bit targets, 8 consecutive columns per thread and sub-chunk.  Per row the sub-chunk's
    // maximum comes from a tree of max operations and its NaN test from a tree of sums (a NaN
    // entry, or +inf beside -inf, makes the sum NaN); only a lane whose maximum exceeds its
    // best so far then looks for the first column holding it.  Sub-chunks whose sum is NaN,
    // and rows with a mask, take the per-entry rule below (NaN first, lowest column).  Entries
    // past vend hold -inf (the checked loads' fill) at higher columns than every entry of the
    // chunk, so they never win: ties keep the lower column.
    static_assert(EPT == 8, "one 16-byte vector per row and sub-chunk");
    bool has_mask[G];
#pragma unroll
    for (int g = 0; g < G; ++g)  // a neutral mask (A = B = -inf) masks nothing
      has_mask[g] = MASKED && (mk[g].x != -INFINITY || mk[g].y != -INFINITY);
    auto body = [&](const TargetBuf<DT, EPT, G>& buf, int64_t s0, auto) {
      const int col0 = elem_index<DT, EPT>(s0, 0);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (g < nrows) {
          float x[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) x[k] = raw_elem<DT>(buf.x[g], k);
          const float sum = ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
          if (has_mask[g] || sum != sum) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              float v = x[k];
              if constexpr (MASKED) v = row_masked(mk[g], v, col0 + k) ? -INFINITY : v;
              const bool take = (v > bv[g]) | ((v != v) & (bv[g] == bv[g]));
              bv[g] = take ? v : bv[g];
              bi[g] = take ? col0 + k : bi[g];
            }
          } else {
            const float lm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                                   fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
            if (lm > bv[g]) {
              int kk = 7;
#pragma unroll
              for (int k = 6; k >= 0; --k) kk = x[k] == lm ? k : kk;
              bv[g] = lm;
              bi[g] = col0 + kk;
            }
          }
        }
      }
    };
    pipeline<kVThreads * EPT, TargetBuf<DT, EPT, G>>(v0, vend, p.target_aligned,
                                                     target_loader<DT, EPT, G>(p, tb, vend), body,
                                                     after_loads);
  } else {
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
                                                   target_loader<DT, EPT, G>(p, tb, vend), body,
                                                   after_loads);
  }
  uint64_t key[G];
#pragma unroll
  for (int g = 0; g < G; ++g) key[g] = argmax_key(bv[g], bi[g]);
  const uint64_t best = block_max_key_to_row_thread<G, kVWaves>(key, s_key);
  if ((int)threadIdx.x < nrows) slot_store(p.stat_slots + (row0 + threadIdx.x) * slot_stride(p) + c, best);
}

// Random rows: per row, the chunk's raw max mx and sum of exp2((x - mx) * c1), kept online per
// thread (the running sum is rescaled when the thread's max grows).  With MASKED, entries
// masked by the row's sampling constraints add nothing to the sum; the maximum still runs over
// every entry, which only moves the reference point of the exponentials (the largest value of
// a row is never masked).
template <int DT, int EPT, int G, bool MASKED, typename Hook>
__device__ inline void task_stats(const VerifyParams& p, int c, float c1, int row0, int nrows,
                                  int64_t v0, int64_t vend, float* s_red, float* s_M,
                                  Hook&& after_loads) {
  using S = typename Elem<DT>::storage;
  const S* tb[G];
  target_bases<DT, G>(p, row0, nrows, tb);
  float4 mk[G];
  row_masks<MASKED, G>(p, row0, nrows, mk);
  float m[G], s[G];
  bool has_mask[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    s[g] = 0.f;
    // a neutral mask (A = B = -inf) masks nothing: such rows skip the per-entry test
    has_mask[g] = MASKED && (mk[g].x != -INFINITY || mk[g].y != -INFINITY);
  }
  auto body = [&](const TargetBuf<DT, EPT, G>& buf, int64_t s0, auto) {
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
        auto sum = [&](auto with_mask) {
          float acc = 0.f;
          // entries below A are masked: a lane whose entries are all below it adds nothing
          // (a wave skips the exponentials when all its lanes do, as on most of a top-k row)
          if constexpr (decltype(with_mask)::value) {
            if (lm < mk[g].x) return acc;
          }
#pragma unroll
          for (int k = 0; k < EPT; ++k) {
            const float e = __builtin_amdgcn_exp2f((x[k] - ref) * c1);
            if constexpr (decltype(with_mask)::value)
              acc += row_masked(mk[g], x[k], elem_index<DT, EPT>(s0, k)) ? 0.f : e;
            else
              acc += e;
          }
          return acc;
        };
        s[g] += has_mask[g] ? sum(std::true_type()) : sum(std::false_type());
      }
    }
  };
  pipeline<kVThreads * EPT, TargetBuf<DT, EPT, G>>(v0, vend, p.target_aligned,
                                                   target_loader<DT, EPT, G>(p, tb, vend), body,
                                                   after_loads);
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
    slot_store(p.stat_slots + (row0 + threadIdx.x) * slot_stride(p) + c,
               pack_stats(mrow, mrow == -INFINITY ? 0.f : srow));
  }
}

// ------------------------------------------------------------------ score tasks ------
// Score tasks read three rows per column (target, draft, noise) and lay all three out in
// quads: 4 consecutive columns per lane and load, consecutive lanes on consecutive quads (the
// fp32 layout, elem_index<MVSD_F32>, whatever the target type).  Every load instruction of a
// wave then covers one contiguous span of each row: 512 bytes of a 2-byte target, 1 KB of fp32
// noise.  In the 16-byte-vector layout of a 2-byte target a lane owns 8 columns, and its two
// fp32 noise (and draft) loads of one sub-chunk lie 16 bytes apart with the next lane's 32 bytes
// on: each instruction would cover every other 16 bytes of a 2 KB span.
template <int DT>
using TargetQuad = std::conditional_t<Elem<DT>::kVec == 4, u32x4, u32x2>;

// Target row sub-chunk in quads; FAST: full and aligned, else bounds-checked with `fill`.
template <int DT, int EPT, bool FAST>
__device__ inline void load_target_quads(const typename Elem<DT>::storage* __restrict__ base,
                                         int64_t s0, int64_t vend, bool aligned,
                                         typename Elem<DT>::storage fill,
                                         TargetQuad<DT> (&out)[EPT / 4]) {
  if constexpr (Elem<DT>::kVec == 4) {
    if constexpr (FAST) load_raw<DT, EPT, true>(base, s0, out);
    else load_raw_checked<DT, EPT, true>(base, s0, vend, aligned, fill, out);
  } else {
#pragma unroll
    for (int m = 0; m < EPT / 4; ++m) {
      const int64_t col = vec_col<MVSD_F32>(s0, m);
      if (FAST || (aligned && col + 4 <= vend)) {
        out[m] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(base + col));
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t lo = bits16(col + 2 * j < vend ? base[col + 2 * j] : fill);
          const uint32_t hi = bits16(col + 2 * j + 1 < vend ? base[col + 2 * j + 1] : fill);
          out[m][j] = lo | hi << 16;
        }
      }
    }
  }
}

// Element k (0 <= k < EPT) of a target buffer in quads, as fp32.
template <int DT>
__device__ inline float quad_elem(const TargetQuad<DT>* x, int k) {
  using S = typename Elem<DT>::storage;
  const S* s = reinterpret_cast<const S*>(&x[k / 4]);
  return Elem<DT>::cvt(s[k % 4]);
}

template <int DT, int DD, int EPT>
struct ScoreBuf {
  static_assert(EPT % 4 == 0, "score tasks load whole quads");
  TargetQuad<DT> x[EPT / 4];
  DraftBuf<DD < 0 ? MVSD_F32 : DD, DD < 0 ? 4 : EPT> q;  // unused without draft probs
  u32x4 e[EPT / 4];
};

// The rejected row `row` of random request r: the chunk-local argmax of max(p - q, 0) * (1 / E)
// over [v0, vend) (point-mass drafts: p with the draft id d removed, :891-897).  The row's
// statistics come from its nslots stats slots, polled by wave 1 while the first sub-chunk
// loads.
// Returns the chunk's argmax key in thread 0; ok = false if the statistics wait gave up.
template <int DT, int EPT, int DD, bool MASKED, typename Hook>
__device__ inline uint64_t task_score(const VerifyParams& p, int r, float c1, int row, int nslots,
                                      int d, int64_t v0, int64_t vend, uint64_t* s_key,
                                      float* s_ml, bool& ok, Hook&& after_loads) {
  using S = typename Elem<DT>::storage;
  using Buf = ScoreBuf<DT, DD, EPT>;
  constexpr bool HAS_DRAFT = DD >= 0;
  constexpr int DE = DD == MVSD_F32 ? 4 : 2;  // draft element bytes
  const S* tb = static_cast<const S*>(p.target) + target_row(p, row) * p.target_stride;
  const void* qb = HAS_DRAFT ? static_cast<const char*>(p.draft) + (int64_t)row * p.draft_stride * DE
                             : nullptr;
  const float* eb = p.noise + (int64_t)r * p.noise_stride;
  const float4 mk = MASKED ? p.masks[row] : make_float4(0.f, 0.f, 0.f, 0.f);
  const bool aligned = p.target_aligned && p.noise_aligned && (p.draft_aligned || !HAS_DRAFT);

  auto load = [&](Buf& buf, int64_t s0, auto fast) {
    constexpr bool F = decltype(fast)::value;
    load_target_quads<DT, EPT, F>(tb, s0, vend, p.target_aligned, Elem<DT>::ninf(), buf.x);
    if constexpr (HAS_DRAFT) load_draft<MVSD_F32, DD, EPT, F>(qb, s0, vend, p.draft_aligned, buf.q);
    load_raw_f32<MVSD_F32, EPT, F>(eb, s0, vend, p.noise_aligned, 1.f, buf.e);
  };

  float MX = 0.f, NL = 0.f;
  // Wave 1 polls, so that the poll overlaps the next ticket's decode in thread 0 (after_loads),
  // and its first read of the slots is issued before the first sub-chunk's loads, so that the
  // wave's in-order load counter does not hold the poll behind them (wave 0 polling after its
  // loads measured 1.0 % slower at the headline, 2.2 % at an EAGLE-sized bf16 batch).
  static_assert(kVWaves >= 2, "the statistics poll runs on wave 1");
  const uint64_t* slots = p.stat_slots + row * slot_stride(p);
  uint64_t v[kKeep];
  if (wave_id() == 1) wave_read_slots(slots, nslots, v);
  auto wait_stats = [&]() {
    after_loads();
    if (wave_id() == 1) {
      const bool polled = wave_poll(p, slots, nslots, v, true);
      float mx, sum;
      combine_stats(slots, nslots, v, c1, mx, sum);
      if (lane_id() == 0) {
        s_ml[0] = mx;
        s_ml[1] = (float)(-log2((double)sum));
        s_ml[2] = polled ? 1.f : 0.f;
      }
    }
    __syncthreads();
    MX = s_ml[0];
    NL = s_ml[1];
    ok = s_ml[2] != 0.f;
  };

  // Scores are max(p - q, 0) / E >= 0 and ties keep the lowest index, so starting from
  // (0, v0) and taking only strictly larger scores gives the same argmax without the clamp.
  float bv = 0.f;
  int bi = (int)v0;
  // a neutral mask (A = B = -inf) masks nothing
  const bool has_mask = MASKED && (mk.x != -INFINITY || mk.y != -INFINITY);
  auto body = [&](const Buf& buf, int64_t s0, auto fast) {
    if constexpr (MASKED) {
      // entries below A are masked and score at most 0: a lane whose entries are all below it
      // has nothing to score (a wave skips when all its lanes do, as on most of a top-k row)
      if (has_mask) {
        float xm = -INFINITY;
#pragma unroll
        for (int k = 0; k < EPT; ++k) xm = fmaxf(xm, quad_elem<DT>(buf.x, k));
        if (xm < mk.x) return;
      }
    }
    float sc[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int idx = elem_index<MVSD_F32, EPT>(s0, k);
      const float x = quad_elem<DT>(buf.x, k);
      float prob = __builtin_amdgcn_exp2f(fmaf(x - MX, c1, NL));  // softmax
      if constexpr (MASKED) prob = has_mask && row_masked(mk, x, idx) ? 0.f : prob;
      float w;
      if constexpr (HAS_DRAFT) w = prob - draft_elem<DD>(buf.q.w, k);  // clamp folded into bv >= 0
      else w = idx == d ? 0.f : prob;
      const float score = w * recip_rn(raw_f32(buf.e, k));
      sc[k] = (decltype(fast)::value || idx < vend) ? score : 0.f;
    }
    if constexpr (Elem<DT>::kVec == 4) {
      // fp32 targets: a strict compare per entry keeps the first maximum (columns rise with s0
      // and k); at 8 entries per lane this measured faster than the tree below
#pragma unroll
      for (int k = 0; k < EPT; ++k) {
        const bool take = sc[k] > bv;
        bv = take ? sc[k] : bv;
        bi = take ? elem_index<MVSD_F32, EPT>(s0, k) : bi;
      }
      return;
    }
    // 2-byte targets, 16 entries per lane: the lane's best of this sub-chunk from a tree of
    // maxima; only a lane whose best beats its best so far looks for the first column holding
    // it, so the first maximum is kept (columns rise with s0 and k).  A NaN score never wins
    // (the tree drops it, and NaN > bv is false).
    float t[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) t[k] = sc[k];
#pragma unroll
    for (int w = EPT / 2; w >= 1; w /= 2) {
#pragma unroll
      for (int k = 0; k < w; ++k) t[k] = fmaxf(t[k], t[k + w]);
    }
    const float m = t[0];
    if (m > bv) {
      int kk = EPT - 1;
#pragma unroll
      for (int k = EPT - 2; k >= 0; --k) kk = sc[k] == m ? k : kk;
      bv = m;
      bi = elem_index<MVSD_F32, EPT>(s0, kk);
    }
  };
  pipeline<kVThreads * EPT, Buf>(v0, vend, aligned, load, body, wait_stats);
  const uint64_t key[1] = {argmax_key(bv, bi)};
  return block_max_key_to_row_thread<1, kVWaves>(key, s_key);
}

// ------------------------------------------------------------------ decisions --------
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
    if (p.draft) {
      const int64_t at = row * p.draft_stride + in.d;
      if (p.draft_dtype == MVSD_F32) in.q = static_cast<const float*>(p.draft)[at];
      else if (p.draft_dtype == MVSD_BF16) in.q = Elem<MVSD_BF16>::cvt(static_cast<const uint16_t*>(p.draft)[at]);
      else in.q = Elem<MVSD_F16>::cvt(static_cast<const _Float16*>(p.draft)[at]);
    }
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
                                       bool& accepted, int& token, float& pd_out) {
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
    pd_out = pd;
  }
  token = accepted ? d : tok;
}

// Stats slots of row k of request r: nc, or 2 nc when its group is in the tail.
__device__ inline int row_slot_count(const VerifyParams& p, const Tables& tb, int r, int k) {
  return tb.gstart[r] + k / p.G >= tb.gt ? 2 * p.nc : p.nc;
}

struct DecideSmem {
  int tok[kMaxSpecLen];
  float M[kMaxSpecLen];
  float S[kMaxSpecLen];
  int out_tok[kMaxSpecLen];
  int first[2];
  int wfail[kVWaves];
};

// Decision slot values of a kFull request: first rejected position + 1 in [1, K], K + 1 when
// every draft is accepted, kDecisionFailed when the decider's waits gave up.
constexpr int kDecisionFailed = 0x40000000;
// Score slots of a task that could not score (a wait gave up) and of a task with nothing to
// score (every draft accepted, or the decider gave up); both below every real key.
constexpr uint64_t kFailKey = 1;
constexpr uint64_t kSkipKey = 2;

// Executed by the whole block that ran the last stats task of request r to start, once that
// task is done.  Combines every
// row's slots and decides every position in parallel (the chain keeps the prefix up to the
// first rejection).  Greedy requests and random requests with supplied recovered ids get
// their output row here (kPoison in every entry if a wait gave up), and every slot of the
// request is cleared.  A kFull request publishes its decision instead; the slots of its
// rejected row stay for the score tasks, and its output row is written by finish_scores.
// Always inlined, as is finish_scores: a call makes the kernel copy its parameters to scratch.
__device__ __forceinline__ void decide_request(const VerifyParams& p, const Tables& tb, int r,
                                               DecideSmem& sm) {
  const int begin = tb.begin[r];
  const int kf = tb.kflags[r];
  const int K = kf & 0xffff;
  const bool greedy = (kf >> 16) & kGreedy;
  const bool full = (kf >> 16) & kFull;
  const float c1 = tb.c1[r];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  // thread pos < K (K <= kMaxSpecLen <= kVThreads) owns position pos; its inputs load while
  // the waves combine the rows' slots
  PosInputs in;
  if (tid < K) in = load_position(p, greedy, begin + tid);
  bool ok = true;
  for (int k = wave_id(); k < K; k += kVWaves) {
    const uint64_t* slots = p.stat_slots + (begin + k) * slot_stride(p);
    const int n = row_slot_count(p, tb, r, k);
    uint64_t v[kKeep];
    ok &= wave_poll(p, slots, n, v);
    int tok = 0;
    float M = 0.f, S = 1.f;
    if (greedy) tok = min(max(key_index(combine_keys(slots, n, v)), 0), p.V - 1);
    else combine_stats(slots, n, v, c1, M, S);
    if (lane == 0) {
      sm.tok[k] = tok;
      sm.M[k] = M;
      sm.S[k] = S;
    }
  }
  if (lane == 0) sm.wfail[wave_id()] = !ok;
  __syncthreads();

  bool accepted = true;
  if (tid < K) {
    int token;
    float pd = NAN;
    const int tok = greedy ? sm.tok[tid] : (full ? -1 : in.rec);
    decide_position(p, r, greedy, tid, in, tok, sm.M[tid], sm.S[tid], accepted, token, pd);
    sm.out_tok[tid] = token;
    if (p.debug_row_stats && !greedy) {
      float* o = p.debug_row_stats + 3 * (int64_t)(begin + tid);
      o[0] = sm.M[tid];
      o[1] = sm.S[tid];
      o[2] = pd;
    }
  }
  static_assert(kMaxSpecLen <= 2 * kWave && kVWaves >= 2, "positions live in waves 0 and 1");
  if (wave_id() < 2) {
    const unsigned long long rej = __ballot(tid < K && !accepted);
    if (lane == 0) sm.first[wave_id()] = rej ? wave_id() * kWave + __builtin_ctzll(rej) : K;
  }
  __syncthreads();
  const int first = min(sm.first[0], sm.first[1]);
  bool failed = false;
#pragma unroll
  for (int w = 0; w < kVWaves; ++w) failed |= sm.wfail[w] != 0;
  const bool scored = full && !failed && first < K;
  if (!full) {
    // the accepted prefix, the token at the first rejection (greedy: the argmax; supplied
    // recovered ids: that id), or the bonus after a fully accepted chain, then -1
    int32_t* out = p.out + (int64_t)r * p.out_stride;
    for (int pos = tid; pos <= p.max_spec_len; pos += kVThreads) {
      int v = -1;
      if (failed) v = kPoison;
      else if (pos < K && pos <= first) v = sm.out_tok[pos];
      else if (pos == K && first == K) v = p.bonus[r];
      out[pos] = v;
    }
    if (p.masks)
      for (int k = tid; k < K; k += kVThreads) p.masks[begin + k] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int k = wave_id(); k < K; k += kVWaves)
    if (!(scored && k == first))
      wave_clear(p.stat_slots + (begin + k) * slot_stride(p), row_slot_count(p, tb, r, k));
  if (tid == 0) {
    atomic_store_relaxed(&p.req_cnt[r], 0);
    if (full) atomic_store_relaxed(&p.decision[r], failed ? kDecisionFailed : first + 1);
  }
}

// One wave of the block that ran the last score task of kFull request r to start, which read
// the decision as `dec` (0 if its wait gave up).  Waits for the nslots score slots of the
// request (so
// every score task has read the decision and the rejected row's statistics), then writes the
// request's output row: the accepted drafts, then the recovered id at the rejected position,
// or the bonus after a fully accepted chain; kPoison in every entry if any wait gave up.  Then
// clears everything the request used.
__device__ __forceinline__ void finish_scores(const VerifyParams& p, const Tables& tb, int r,
                                              int dec, int nslots) {
  if (wave_id() != 0) return;
  const int lane = lane_id();
  const int begin = tb.begin[r];
  const int K = tb.kflags[r] & 0xffff;
  uint64_t* slots = p.score_slots + r * slot_stride(p);
  uint64_t v[kKeep];
  bool failed = !wave_poll(p, slots, nslots, v);
  int bad = 0;
#pragma unroll
  for (int j = 0; j < kKeep; ++j) bad |= v[j] == kFailKey;
  for (int c = lane + kKeep * kWave; c < nslots; c += kWave) bad |= slot_load(slots + c) == kFailKey;
  failed |= __any(bad) != 0;
  failed |= dec < 1 || dec > K + 1;
  const int first = failed ? K : dec - 1;
  int tok = -1;
  if (!failed && first < K) tok = min(max(key_index(combine_keys(slots, nslots, v)), 0), p.V - 1);
  int32_t* out = p.out + (int64_t)r * p.out_stride;
  for (int pos = lane; pos <= p.max_spec_len; pos += kWave) {
    int v = -1;
    if (failed) v = kPoison;
    else if (pos < first) v = p.draft_ids[begin + pos];
    else if (pos == first && first < K) v = tok;
    else if (pos == K && first == K) v = p.bonus[r];
    out[pos] = v;
  }
  wave_clear(slots, nslots);
  if (!failed && first < K)
    wave_clear(p.stat_slots + (begin + first) * slot_stride(p), row_slot_count(p, tb, r, first));
  if (p.masks)
    for (int k = lane; k < K; k += kWave) p.masks[begin + k] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (lane == 0) {
    atomic_store_relaxed(&p.decision[r], 0);
    atomic_store_relaxed(&p.score_cnt[r], 0);
  }
}

// ------------------------------------------------------------------ tickets ----------
// Unit order: the stats units of the groups in request order, with the score unit of kFull
// request r inserted right after the stats unit of group (last group of r) + lag, or at the
// end.  Units before the tail (position u < u0) hold nc tickets each, one per chunk; tail
// units hold 2 nc tickets, one per half chunk, so that the launch ends with short tasks.  The
// tail is the stats units of the last tail_groups groups and every score unit after the first
// of them (with tail_groups = 0: the score units after the last stats unit).

// Exclusive scans of three values per thread over the kVThreads-thread block, side by side:
// shuffle scans within the waves, then one barrier for the wave totals.  v[i] becomes this
// thread's exclusive prefix of value i and total[i] the block's sum.  `s_wave` holds
// 3 * kVWaves ints.
__device__ inline void block_exclusive_scan3(int (&v)[3], int (&total)[3], int* s_wave) {
  const int lane = lane_id(), w = wave_id();
  int x[3] = {v[0], v[1], v[2]};
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int y = __shfl_up(x[i], d, kWave);
      x[i] += lane >= d ? y : 0;
    }
  }
  if (lane == kWave - 1)
#pragma unroll
    for (int i = 0; i < 3; ++i) s_wave[i * kVWaves + w] = x[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    int before = 0, sum = 0;
#pragma unroll
    for (int j = 0; j < kVWaves; ++j) {
      const int s = s_wave[i * kVWaves + j];
      before += j < w ? s : 0;
      sum += s;
    }
    total[i] = sum;
    v[i] = before + x[i] - v[i];
  }
}

// Length of the prefix of [0, n) on which pred holds (pred holds on a prefix; n <= 64 * 64),
// found by one wave in two rounds: the first index of each of 64 blocks, then the entries of
// the block holding the end.  Called by every lane of a wave; every lane receives the count.
template <typename Pred>
__device__ inline int wave_prefix_count(int n, Pred&& pred) {
  const int lane = lane_id();
  const int step = (n + kWave - 1) / kWave;
  const int blocks = __popcll(__ballot(lane * step < n && pred(lane * step)));
  if (blocks == 0) return 0;
  const int base = (blocks - 1) * step;
  return base + __popcll(__ballot(lane < step && base + lane < n && pred(base + lane)));
}

// Every workgroup builds the tables: each thread reads the metadata of a run of consecutive
// requests once, then block scans give the group offsets and the kFull ordinals.  Stats
// groups run random requests first, then greedy requests (each in request order): greedy
// requests have no score units, so the launch ends on stats tasks that nothing waits for,
// rather than on score tasks waiting for the last decisions.  Requests without drafts get
// their output row here (bonus, then -1), from workgroup r mod grid.
__device__ inline void build_tables(const VerifyParams& p, Tables& tb, int* s_wave) {
  const int tid = threadIdx.x;
  const int per = (p.B + kVThreads - 1) / kVThreads;
  const int r0 = tid * per, r1 = min(p.B, r0 + per);
  // per class (random, greedy): requests << 18 | groups, which a launch keeps below 2^31
  int run_r = 0, run_g = 0, run_f = 0;
  for (int r = r0; r < r1; ++r) {
    // the temperature is read once, beside the bounds (req_is_greedy and req_temperature each
    // read it, and the compiler kept the two reads, one round trip after the other)
    const float temp = p.all_greedy ? 0.f : p.temperature[r];
    int b, k;
    req_range(p, r, b, k);
    const int ng = (k + p.G - 1) / p.G;
    const bool greedy = temp == 0.f;  // req_is_greedy
    const bool full = !greedy && !p.recovered && k > 0;
    tb.gstart[r] = ng;
    if (greedy) run_g += (1 << 18) + ng;
    else run_r += (1 << 18) + ng;
    run_f += full ? 1 : 0;
    tb.begin[r] = b;
    tb.kflags[r] = k | ((greedy ? kGreedy : 0) | (full ? kFull : 0)) << 16;
    tb.c1[r] = exp2_scale(p.apply_temperature && !greedy ? temp : 1.f);  // req_temperature
  }
  int acc[3] = {run_r, run_g, run_f}, tot[3];
  block_exclusive_scan3(acc, tot, s_wave);
  int acc_r = acc[0], acc_g = acc[1], acc_f = acc[2];
  const int tot_r = tot[0], tot_g = tot[1], nfull = tot[2];
  const int groups_r = tot_r & 0x3ffff, nreq_r = tot_r >> 18;
  const int groups = groups_r + (tot_g & 0x3ffff);
  for (int r = r0; r < r1; ++r) {
    const int ng = tb.gstart[r];
    const int kf = tb.kflags[r];
    int g0, pos;
    if ((kf >> 16) & kGreedy) {
      g0 = groups_r + (acc_g & 0x3ffff);
      pos = nreq_r + (acc_g >> 18);
      acc_g += (1 << 18) + ng;
    } else {
      g0 = acc_r & 0x3ffff;
      pos = acc_r >> 18;
      acc_r += (1 << 18) + ng;
    }
    tb.gstart[r] = g0;
    tb.gpos[pos] = g0 << 12 | r;
    if ((kf >> 16) & kFull) {
      tb.fpos[acc_f] = (acc_f + min(groups, g0 + ng + p.lag)) << 12 | r;
      ++acc_f;
    }
    if (ng == 0 && (r % (int)gridDim.x) == (int)blockIdx.x) {
      int32_t* out = p.out + (int64_t)r * p.out_stride;
      for (int c = 0; c <= p.max_spec_len; ++c) out[c] = c == 0 ? p.bonus[r] : -1;
    }
  }
  if (tid == 0) tb.gpos[p.B] = groups << 12;
  __syncthreads();
  tb.groups = groups;
  tb.nfull = nfull;
  // Score unit k follows S_k = (fpos_k >> 12) - k stats units (non-decreasing in k).  The tail
  // starts at stats unit gt; its score units are those with S_k > tau.
  tb.gt = max(0, groups - p.tail_groups);
  const int tau = p.tail_groups > 0 ? tb.gt : groups - 1;
  tb.kt = wave_prefix_count(nfull, [&](int k) { return (tb.fpos[k] >> 12) - k <= tau; });
  tb.u0 = tb.gt + tb.kt;
}

constexpr int kStatsTask = 1;
constexpr int kScoreTask = 2;

// Wave 0, every lane: decode ticket t (lane 0's value) into dst[0..7] = {t, slot (the chunk,
// or 2 * chunk + half in the tail), kind | tail << 4, request, first row, rows | groups << 8 |
// flags << 16 (stats) or K | flags << 16 (score), bits of c1, the request's decision as read
// now (score units; 0 if not yet published)}, written by lane 0.  kind 0: past the last unit.
// The table searches take two rounds of LDS reads across the wave (a search by one thread
// took about 1.3 us, in the middle of the task whose loads it follows).
__device__ inline void fetch_task(const VerifyParams& p, const Tables& tb, int t, int* dst) {
  t = __builtin_amdgcn_readfirstlane(t);
  const int units = tb.groups + tb.nfull;
  const int reg = tb.u0 * p.nc;
  int u, part, tail;
  if (t < reg) {
    u = t / p.nc;
    part = t - u * p.nc;
    tail = 0;
  } else {
    const int q = (t - reg) / (2 * p.nc);
    u = tb.u0 + q;
    part = t - reg - q * 2 * p.nc;
    tail = 1;
  }
  int kind = 0, r = 0, row0 = 0, info = 0, dec = 0;
  if (u < units) {
    // score units at positions < u
    const int lo = wave_prefix_count(tb.nfull, [&](int k) { return (tb.fpos[k] >> 12) < u; });
    if (lo < tb.nfull && (tb.fpos[lo] >> 12) == u) {
      kind = kScoreTask;
      r = tb.fpos[lo] & 0xfff;
      row0 = tb.begin[r];
      info = tb.kflags[r];
      if (lane_id() == 0) dec = atomic_load_relaxed(&p.decision[r]);
    } else {
      kind = kStatsTask;
      const int li = u - lo;
      // the last position whose first group is <= li owns it (position 0's first group is 0)
      const int a = wave_prefix_count(p.B, [&](int i) { return (tb.gpos[i] >> 12) <= li; }) - 1;
      r = tb.gpos[a] & 0xfff;
      const int kf = tb.kflags[r];
      const int k = kf & 0xffff;
      const int g = li - (tb.gpos[a] >> 12);
      const int ng = (tb.gpos[a + 1] >> 12) - (tb.gpos[a] >> 12);
      row0 = tb.begin[r] + g * p.G;
      info = min(p.G, k - g * p.G) | ng << 8 | (kf >> 16) << 16;
    }
  }
  if (lane_id() == 0) {
    dst[0] = t;
    dst[1] = part;
    dst[2] = kind | tail << 4;
    dst[3] = r;
    dst[4] = row0;
    dst[5] = info;
    dst[6] = __float_as_int(tb.c1[r]);
    dst[7] = dec;
  }
}

// Columns [v0, vend) of task slot `part`: chunk `part` in full, or in the tail half
// part & 1 of chunk part >> 1, split at a score sub-chunk boundary (a half may be empty).
template <int EPT>
__device__ inline void task_columns(const VerifyParams& p, int part, bool tail, int64_t& v0,
                                    int64_t& vend) {
  const int c = tail ? part >> 1 : part;
  const int64_t cs = (int64_t)c * p.chunk;
  const int64_t ce = min((int64_t)p.V, cs + p.chunk);
  if (!tail) {
    v0 = cs;
    vend = ce;
    return;
  }
  constexpr int64_t SS = 2 * (int64_t)kVThreads * EPT;
  const int64_t nsc = (ce - cs + SS - 1) / SS;
  const int64_t mid = min(ce, cs + (nsc + 1) / 2 * SS);
  v0 = (part & 1) ? mid : cs;
  vend = (part & 1) ? ce : mid;
}

// ------------------------------------------------------------------ main kernel ------
// DD: the draft probabilities' dtype (MVSD_F32, MVSD_BF16, MVSD_F16), or -1 for point-mass
// drafts.
template <int DT, int EPT, int G, int DD, bool MASKED>
__global__ __launch_bounds__(kVThreads) void verify_kernel(VerifyParams p) {
  static_assert(EPT % Elem<DT>::kVec == 0, "EPT must be a multiple of the vector width");
  __shared__ float s_red[G * kVWaves];
  __shared__ uint64_t s_key[G * kVWaves];
  __shared__ float s_M[G];
  __shared__ float s_ml[3];
  __shared__ int s_info[2][8];  // double-buffered decoded ticket (current, next)
  __shared__ int s_last;
  __shared__ int s_dec;
  __shared__ int s_wave[3 * kVWaves];
  __shared__ DecideSmem dsm;
  __shared__ int s_gpos[kMaxLaunchRequests + 1], s_gstart[kMaxLaunchRequests];
  __shared__ int s_begin[kMaxLaunchRequests], s_kf[kMaxLaunchRequests], s_fpos[kMaxLaunchRequests];
  __shared__ float s_c1[kMaxLaunchRequests];

  const int tid = threadIdx.x;
  int* ticket = &p.ctrl[kCtrlTicket];
  // the first ticket is claimed before the tables are built, so its round trip overlaps them
  int tfirst = 0;
  if (tid == 0) tfirst = atomic_add_relaxed(ticket, 1);
  Tables tb{s_gpos, s_gstart, s_begin, s_kf, s_c1, s_fpos, 0, 0};
  build_tables(p, tb, s_wave);
  const int total = tb.u0 * p.nc + (tb.groups + tb.nfull - tb.u0) * 2 * p.nc;

  // Every task is counted when it starts, with a relaxed atomic whose result is examined when
  // the task ends (its round trip overlaps the task).  The last task of a request to start
  // finishes the request right after its own work: it waits only for the slots of the request's
  // other tasks, which have all started and never wait themselves.

  // The next ticket is claimed when a task starts and decoded once the task's loads are in
  // flight, so the atomic and the decode overlap with HBM traffic.
  if (wave_id() == 0) fetch_task(p, tb, tfirst, s_info[0]);
  __syncthreads();
  for (int par = 0;; par ^= 1) {
    const int* info = s_info[par];
    const int t = info[0];
    if (t >= total) break;
    int tnext = 0;
    if (tid == 0) tnext = atomic_add_relaxed(ticket, 1);
    auto prefetch = [&]() {
      if (wave_id() == 0) fetch_task(p, tb, tnext, s_info[par ^ 1]);
    };
    const int kind = info[2] & 0xf;
    const bool tail = info[2] >> 4;
    const int c = info[1];
    const int r = info[3];
    const int row0 = info[4];
    const int rinfo = info[5];
    const float c1 = __int_as_float(info[6]);
    int64_t v0, vend;
    task_columns<EPT>(p, c, tail, v0, vend);
    int started = 0;
    if (kind == kStatsTask) {
      const int nrows = rinfo & 0xff;
      const int ngr = (rinfo >> 8) & 0xff;
      if (tid == 0) started = atomic_add_relaxed(&p.req_cnt[r], 1);
      if ((rinfo >> 16) & kGreedy)
        task_argmax<DT, EPT, G, MASKED>(p, c, row0, nrows, v0, vend, s_key, prefetch);
      else
        task_stats<DT, EPT, G, MASKED>(p, c, c1, row0, nrows, v0, vend, s_red, s_M, prefetch);
      // the request's stats tasks: nc per group, 2 nc per tail group
      const int g0 = tb.gstart[r], g1 = g0 + ngr;
      const int ntasks = p.nc * (ngr + max(0, g1 - max(g0, tb.gt)));
      if (tid == 0) s_last = started == ntasks - 1;
      __syncthreads();
      if (s_last) decide_request(p, tb, r, dsm);
    } else if (kind == kScoreTask) {
      // every score task counts, so that exactly one of them finishes the request
      if (tid == 0) {
        started = atomic_add_relaxed(&p.score_cnt[r], 1);
        int d = info[7];
        for (int spins = 0; d == 0; ++spins) {
          if (spins >= p.spin_limit ||
              ((spins & 255) == 255 && atomic_load_relaxed(&p.ctrl[kCtrlFlag]) != 0)) {
            atomic_store_relaxed(&p.ctrl[kCtrlFlag], 1);
            break;
          }
          d = atomic_load_relaxed(&p.decision[r]);
          if (d == 0) __builtin_amdgcn_s_sleep(1);
        }
        s_dec = d;
      }
      __syncthreads();
      const int d = s_dec;
      const int K = rinfo & 0xffff;
      uint64_t key = d == 0 ? kFailKey : kSkipKey;
      if (d >= 1 && d <= K) {
        // rejection at position d - 1: score this chunk of that row
        const int row = row0 + d - 1;
        const int draft = DD >= 0 ? -1 : p.draft_ids[row];
        bool ok;
        const int nslots = tb.gstart[r] + (d - 1) / p.G >= tb.gt ? 2 * p.nc : p.nc;
        key = task_score<DT, 2 * EPT, DD, MASKED>(p, r, c1, row, nslots, draft, v0, vend,
                                                         s_key, s_ml, ok, prefetch);
        if (!ok) key = kFailKey;
      } else {
        // every draft accepted, or no usable decision: nothing to score, but the slot tells
        // the finisher that this task has read the decision
        prefetch();
      }
      const int ntasks = tail ? 2 * p.nc : p.nc;
      if (tid == 0) {
        slot_store(p.score_slots + r * slot_stride(p) + c, key);
        s_last = started == ntasks - 1;
      }
      __syncthreads();
      if (s_last) finish_scores(p, tb, r, d, ntasks);
    } else {
      prefetch();
    }
    __syncthreads();
  }

  // The last workgroup out resets the ticket and the exit counter.  If some wait gave up, the
  // requests concerned already hold kPoison; slots may still have been published after the
  // wait gave up, so the last workgroup then clears every slot, count, decision and mask of
  // the launch.  Workgroups that exit after the failure count with acquire-release, which
  // orders their stores before that clean-up.
  if (tid == 0) {
    const bool failed = atomic_load_relaxed(&p.ctrl[kCtrlFlag]) != 0;
    int* exits = &p.ctrl[kCtrlExit];
    const int n = failed ? atomic_add_acq_rel(exits, 1) : atomic_add_relaxed(exits, 1);
    s_last = n == (int)gridDim.x - 1;
    s_dec = s_last && atomic_load_acquire(&p.ctrl[kCtrlFlag]) != 0;
  }
  __syncthreads();
  if (s_last) {
    if (s_dec) {
      for (int r = tid; r < p.B; r += kVThreads) {
        int b, k;
        req_range(p, r, b, k);
        for (int j = 0; j < k; ++j) {
          for (int c = 0; c < slot_stride(p); ++c) slot_store(p.stat_slots + (b + j) * slot_stride(p) + c, 0);
          if (p.masks) p.masks[b + j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        for (int c = 0; c < slot_stride(p); ++c) slot_store(p.score_slots + r * slot_stride(p) + c, 0);
        atomic_store_relaxed(&p.req_cnt[r], 0);
        atomic_store_relaxed(&p.score_cnt[r], 0);
        atomic_store_relaxed(&p.decision[r], 0);
      }
      __syncthreads();
      if (tid == 0) atomic_store_relaxed(&p.ctrl[kCtrlFlag], 0);
    }
    if (tid == 0) {
      atomic_store_relaxed(&p.ctrl[kCtrlTicket], 0);
      atomic_store_relaxed(&p.ctrl[kCtrlExit], 0);
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
constexpr int kGroup = 4;          // rows per stats group
constexpr int kMinSubs = 8;        // sub-chunks per task at least
constexpr int kMinSubsSmall = 2;   // ... on batches too small to fill the device otherwise
constexpr int64_t kSmallBatchRows = 64;  // verify rows + requests of such a batch at most
// Every task has fixed costs (its first loads' latency, block reductions, publication), so
// tasks are as long as the tail allows: about 7 per resident workgroup measured 1.5 % faster at
// the headline and 1.8 % on a ragged bf16 batch than 10 (with tasks capped at 512 KiB).  On large
// batches the 7 tasks are long (whole 1.2 MB bf16 row groups on an EAGLE-sized batch, 6 %
// faster than 512 KiB tasks); the tail is then a small share of the launch.
constexpr int kTasksPerWg = 7;     // tasks per resident workgroup aimed for
template <int DT>
constexpr int ept_of() {
  return DT == MVSD_F32 ? 4 : 8;  // 16 bytes of target per thread and row per sub-chunk
}

VerifyPlan verify_plan(int target_dtype, int64_t vocab_size, int64_t units, int cap,
                       int64_t batch_rows, bool score_units) {
  VerifyPlan plan;
  plan.ept = target_dtype == MVSD_F32 ? ept_of<MVSD_F32>() : ept_of<MVSD_BF16>();
  plan.g = kGroup;
  plan.sub = kVThreads * plan.ept;
  const int64_t nsub = (vocab_size + plan.sub - 1) / plan.sub;
  // Chunks per row: enough tasks for about kTasksPerWg per resident workgroup, each task as
  // long as possible (fewer ticket claims, longer load pipelines), and at least kMinSubs
  // sub-chunks per task so that batches do not shred the rows into tasks too short to
  // amortise their start and end.  A batch of at most kSmallBatchRows verify rows and requests
  // that cannot give every resident workgroup a task of kMinSubs sub-chunks (a few requests)
  // takes shorter tasks instead, down to kMinSubsSmall sub-chunks, so that its few megabytes
  // are spread over the device.
  // Score tasks walk sub-chunks of twice the columns, so the chunks of a launch with score
  // units hold an even number of sub-chunks.  A launch without score units that can give every
  // resident workgroup a task aims at one task each (no second round, no tail); with score
  // units the count rounds up, the score tasks coming after the decisions anyway.
  const int64_t nc_regular = nsub / kMinSubs > 1 ? nsub / kMinSubs : 1;
  const int64_t nc_small = (nsub + kMinSubsSmall - 1) / kMinSubsSmall;
  // the workspace holds slots for nc_max chunks per row
  const int64_t nc_max = batch_rows <= kSmallBatchRows ? nc_small : nc_regular;
  int64_t nc_hi = nc_regular;
  if (units > 0 && cap > 0 && units * nc_regular < cap) {
    const int64_t want = score_units ? (cap + units - 1) / units : cap / units;
    nc_hi = want < nc_max ? want : nc_max;
    if (nc_hi < nc_regular) nc_hi = nc_regular;
  }
  int64_t nc = nc_hi;
  if (units > 0 && cap > 0) {
    nc = ((int64_t)kTasksPerWg * cap + units - 1) / units;
    nc = nc < 1 ? 1 : (nc > nc_hi ? nc_hi : nc);
  }
  int64_t subs_per_chunk = (nsub + nc - 1) / nc;
  if (subs_per_chunk > 1 && score_units) subs_per_chunk += subs_per_chunk & 1;
  plan.chunk = (int)(subs_per_chunk * plan.sub);
  plan.nc = (int)((vocab_size + plan.chunk - 1) / plan.chunk);
  plan.nc_max = (int)nc_max;
  return plan;
}

template <int DT, bool MASKED>
const void* kernel_for_mask(int draft_dtype) {
  constexpr int E = ept_of<DT>();
  switch (draft_dtype) {
    case -1: return reinterpret_cast<const void*>(&verify_kernel<DT, E, kGroup, -1, MASKED>);
    case MVSD_F32: return reinterpret_cast<const void*>(&verify_kernel<DT, E, kGroup, MVSD_F32, MASKED>);
    case MVSD_BF16: return reinterpret_cast<const void*>(&verify_kernel<DT, E, kGroup, MVSD_BF16, MASKED>);
    case MVSD_F16: return reinterpret_cast<const void*>(&verify_kernel<DT, E, kGroup, MVSD_F16, MASKED>);
    default: return nullptr;
  }
}

template <int DT>
const void* kernel_for(int draft_dtype, bool masked) {
  return masked ? kernel_for_mask<DT, true>(draft_dtype) : kernel_for_mask<DT, false>(draft_dtype);
}

const void* verify_kernel_ptr(int target_dtype, int draft_dtype, bool masked) {
  switch (target_dtype) {
    case MVSD_F32: return kernel_for<MVSD_F32>(draft_dtype, masked);
    case MVSD_BF16: return kernel_for<MVSD_BF16>(draft_dtype, masked);
    case MVSD_F16: return kernel_for<MVSD_F16>(draft_dtype, masked);
    default: return nullptr;
  }
}

hipError_t launch_verify(const VerifyParams& params, int target_dtype, int grid,
                         hipStream_t stream) {
  if (params.B == 0) return hipSuccess;
  const void* fn = verify_kernel_ptr(target_dtype, params.draft ? params.draft_dtype : -1,
                                     params.masks != nullptr);
  if (!fn) return hipErrorInvalidValue;
  void* args[] = {const_cast<VerifyParams*>(&params)};
  hipError_t err = hipLaunchKernel(fn, dim3(grid), dim3(kVThreads), args, 0, stream);
  if (err != hipSuccess) return err;
  return hipGetLastError();
}

}  // namespace mvsd
