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
//     (max, sumexp) for each row and publishes it (release).  Random rows then wait until
//     all NC chunk tasks of the group have published; those tasks were claimed earlier (or
//     are being claimed by running workgroups), never wait themselves before publishing,
//     and therefore finish: the wait cannot deadlock.  A spin bound still ends every wave.
//   * Phase 2 combines the NC partials into the row's (M, S), streams the request's noise
//     chunk once and each row's draft chunk once, and scores p_v = e_v * exp(m_c - M) / S
//     straight from the registers, keeping a chunk-local argmax per row.
//   * The last task to finish a request (acq_rel counter) reduces the chunk argmaxes and
//     runs the sequential accept/reject chain, writing [B, max_spec_len + 1].
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

__device__ inline float2 load_stats(const float2* s) {
  return *s;
}

// ------------------------------------------------------------------ init kernel ------
// One 1024-thread block: zero the ticket / counters, fill the output with -1 (bonus in
// column 0 for requests without drafts), and exclusive-scan the per-request group counts.
__global__ __launch_bounds__(1024) void verify_init_kernel(VerifyParams p) {
  const int tid = threadIdx.x;
  if (tid < 2) p.ctrl[tid] = 0;
  for (int i = tid; i < p.P; i += 1024) p.grp_cnt[i] = 0;
  for (int i = tid; i < p.B; i += 1024) p.req_cnt[i] = 0;
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
    if (r < p.B) p.grp_off[r] = carry + s_scan[tid] - ng;
    __syncthreads();
    if (tid == 1023) s_carry = carry + s_scan[1023];
    __syncthreads();
  }
  if (tid == 0) p.grp_off[p.B] = s_carry;
}

// ------------------------------------------------------------------ finalisation -----
// Executed by the whole block that completed request r's last task.
__device__ void finalize_request(const VerifyParams& p, int r, bool greedy, bool full,
                                 int* s_tok, float* s_M, float* s_S) {
  int begin, K;
  req_range(p, r, begin, K);
  const int lane = lane_id();
  const int nc = p.nc;
  for (int k = wave_id(); k < K; k += kWaves) {
    const int64_t row = begin + k;
    if (greedy || full) {
      float bv = -INFINITY;
      int bi = INT_MAX;
      for (int c = lane; c < nc; c += kWave) {
        argmax_update(bv, bi, p.argv[row * nc + c], p.argi[row * nc + c], true);
      }
      wave_argmax(bv, bi);
      if (lane == 0) s_tok[k] = full ? min(bi, p.V - 1) : bi;
    } else if (lane == 0) {
      s_tok[k] = p.recovered[row];
    }
    if (!greedy) {
      float m = -INFINITY;
      for (int c = lane; c < nc; c += kWave) m = fmaxf(m, load_stats(&p.stats[row * nc + c]).x);
      m = wave_max(m);
      float s = 0.f;
      for (int c = lane; c < nc; c += kWave) {
        const float2 st = load_stats(&p.stats[row * nc + c]);
        if (st.x != -INFINITY) s += st.y * expf(st.x - m);
      }
      s = wave_sum(s);
      if (lane == 0) {
        s_M[k] = m;
        s_S[k] = s;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x != 0) return;

  int32_t* out = p.out + (int64_t)r * p.out_stride;
  const bool synthetic = p.synth != nullptr;
  const float temp = req_temperature(p, r);
  bool rejected = false;
  for (int pos = 0; pos < K; ++pos) {
    const int64_t row = begin + pos;
    const int d = p.draft_ids[row];
    int token;
    bool accepted;
    if (greedy) {
      // rejection_sampler.py:715-732
      if (synthetic) {
        accepted = p.uniforms[row] < (double)p.synth[pos] && d >= 0;
        token = accepted ? d : s_tok[pos];
      } else {
        token = s_tok[pos];
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
        if (temp != 1.f) x = x / temp;
        const float pd = expf(x - s_M[pos]) / s_S[pos];
        accepted = q > 0.f && (double)(pd / q) >= u;
      }
      token = accepted ? d : s_tok[pos];
    }
    out[pos] = token;
    if (!accepted) {
      rejected = true;
      break;
    }
  }
  if (!rejected) out[K] = p.bonus[r];
}

// ------------------------------------------------------------------ main kernel ------
template <int DT, int EPT, int G>
__global__ __launch_bounds__(kThreads) void verify_kernel(VerifyParams p) {
  using S = typename Elem<DT>::storage;
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int NV = EPT / VEC;
  static_assert(EPT % VEC == 0, "EPT must be a multiple of the vector width");

  __shared__ float s_red[G * kWaves];
  __shared__ int s_redi[G * kWaves];
  __shared__ float s_f[G];
  __shared__ int s_task;
  __shared__ int s_last;
  __shared__ int s_tok[kMaxSpecLen];
  __shared__ float s_M[kMaxSpecLen];
  __shared__ float s_S[kMaxSpecLen];

  const int tid = threadIdx.x;
  const int nc = p.nc;
  const int total = p.grp_off[p.B] * nc;

  for (;;) {
    if (tid == 0) s_task = atomic_add_relaxed(&p.ctrl[0], 1);
    __syncthreads();
    const int t = s_task;
    __syncthreads();
    if (t >= total) break;

    const int gi = t / nc;
    const int c = t - gi * nc;
    int lo = 0, hi = p.B;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (p.grp_off[mid] <= gi) lo = mid; else hi = mid;
    }
    const int r = lo;
    int begin, K;
    req_range(p, r, begin, K);
    const int g0 = gi - p.grp_off[r];
    const int row0 = begin + g0 * G;
    const int nrows = min(G, K - g0 * G);
    const int ngr = p.grp_off[r + 1] - p.grp_off[r];
    const bool greedy = req_is_greedy(p, r);
    const bool full = !greedy && p.recovered == nullptr;
    const int64_t v0 = (int64_t)c * p.chunk;
    const int64_t vend = min((int64_t)p.V, v0 + p.chunk);

    // ---- load the group's target slice (fp32 in registers; -inf beyond V) ----
    float x[G][EPT];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g < nrows) {
        const int64_t trow = target_row(p, row0 + g);
        const S* base = static_cast<const S*>(p.target) + trow * p.target_stride;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          float tmp[VEC];
          load_vec<DT>(base, v0 + ((int64_t)i * kThreads + tid) * VEC, vend, p.target_aligned,
                       -INFINITY, tmp);
#pragma unroll
          for (int j = 0; j < VEC; ++j) x[g][i * VEC + j] = tmp[j];
        }
      } else {
#pragma unroll
        for (int k = 0; k < EPT; ++k) x[g][k] = -INFINITY;
      }
    }

    if (greedy) {
      // ---- chunk-local argmax of the raw logits ----
      float bv[G];
      int bi[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        bv[g] = -INFINITY;
        bi[g] = INT_MAX;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            const int idx = (int)(v0 + ((int64_t)i * kThreads + tid) * VEC + j);
            argmax_update(bv[g], bi[g], x[g][i * VEC + j], idx, idx < vend);
          }
        }
      }
      block_argmax<G>(bv, bi, s_red, s_redi);
      if (tid == 0) {
        for (int g = 0; g < nrows; ++g) {
          p.argv[(int64_t)(row0 + g) * nc + c] = bv[g];
          p.argi[(int64_t)(row0 + g) * nc + c] = bi[g];
        }
      }
    } else {
      // ---- phase 1: temperature, chunk max, exp, chunk sum ----
      const float temp = req_temperature(p, r);
      if (temp != 1.f) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int k = 0; k < EPT; ++k) x[g][k] = x[g][k] / temp;
      }
      float m[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mm = -INFINITY;
#pragma unroll
        for (int k = 0; k < EPT; ++k) mm = fmaxf(mm, x[g][k]);
        m[g] = mm;
      }
      block_max<G>(m, s_red);
      float s[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float ss = 0.f;
        const bool dead = m[g] == -INFINITY;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          const float e = dead ? 0.f : expf(x[g][k] - m[g]);
          x[g][k] = e;
          ss += e;
        }
        s[g] = ss;
      }
      block_sum<G>(s, s_red);
      if (tid == 0) {
        for (int g = 0; g < nrows; ++g) p.stats[(int64_t)(row0 + g) * nc + c] = make_float2(m[g], s[g]);
      }

      if (full) {
        // ---- publish, then wait for the group's other chunk tasks ----
        if (tid == 0) {
          atomic_add_release(&p.grp_cnt[gi], 1);
          int spins = 0;
          while (atomic_load_acquire(&p.grp_cnt[gi]) < nc) {
            __builtin_amdgcn_s_sleep(2);
            if (++spins > kSpinLimit) {
              atomic_store_relaxed(&p.ctrl[1], 1);
              break;
            }
          }
        }
        __syncthreads();
        // ---- combine partials: row (M, S) and this chunk's scale exp(m_c - M) / S ----
        const int lane = lane_id();
        for (int g = wave_id(); g < nrows; g += kWaves) {
          const int64_t row = row0 + g;
          float mm = -INFINITY;
          for (int cc = lane; cc < nc; cc += kWave) mm = fmaxf(mm, load_stats(&p.stats[row * nc + cc]).x);
          mm = wave_max(mm);
          float ss = 0.f;
          for (int cc = lane; cc < nc; cc += kWave) {
            const float2 st = load_stats(&p.stats[row * nc + cc]);
            if (st.x != -INFINITY) ss += st.y * expf(st.x - mm);
          }
          ss = wave_sum(ss);
          if (lane == 0) {
            float mine = -INFINITY;
#pragma unroll
            for (int gg = 0; gg < G; ++gg) if (gg == g) mine = m[gg];
            s_f[g] = (mine == -INFINITY) ? 0.f : expf(mine - mm) / ss;
          }
        }
        __syncthreads();

        // ---- phase 2: noise chunk once, then each row's draft chunk ----
        float inv[EPT];
        {
          const float* nbase = p.noise + (int64_t)r * p.noise_stride;
#pragma unroll
          for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int h = 0; h < VEC; h += 4) {
              float tmp[4];
              load_vec<MVSD_F32>(nbase, v0 + ((int64_t)i * kThreads + tid) * VEC + h, vend,
                                 p.noise_aligned, 1.f, tmp);
#pragma unroll
              for (int j = 0; j < 4; ++j) inv[i * VEC + h + j] = 1.0f / tmp[j];
            }
          }
        }
        float bv[G];
        int bi[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          bv[g] = -INFINITY;
          bi[g] = INT_MAX;
          if (g < nrows) {
            const int row = row0 + g;
            const float f = s_f[g];
            const int d = p.draft_ids[row];
            const float* dbase = p.draft ? p.draft + (int64_t)row * p.draft_stride : nullptr;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
#pragma unroll
              for (int h = 0; h < VEC; h += 4) {
                const int64_t idx0 = v0 + ((int64_t)i * kThreads + tid) * VEC + h;
                float q[4] = {0.f, 0.f, 0.f, 0.f};
                if (dbase) load_vec<MVSD_F32>(dbase, idx0, vend, p.draft_aligned, 0.f, q);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                  const int idx = (int)(idx0 + j);
                  const float prob = x[g][i * VEC + h + j] * f;
                  const float w = dbase ? fmaxf(prob - q[j], 0.f) : (idx == d ? 0.f : prob);
                  const float score = w * inv[i * VEC + h + j];
                  argmax_update(bv[g], bi[g], score, idx, idx < vend);
                }
              }
            }
          }
        }
        block_argmax<G>(bv, bi, s_red, s_redi);
        if (tid == 0) {
          for (int g = 0; g < nrows; ++g) {
            p.argv[(int64_t)(row0 + g) * nc + c] = bv[g];
            p.argi[(int64_t)(row0 + g) * nc + c] = bi[g];
          }
        }
      }
    }

    // ---- request completion: the last task runs the accept/reject chain ----
    if (tid == 0) {
      const int old = atomic_add_acq_rel(&p.req_cnt[r], 1);
      s_last = old == ngr * nc - 1;
    }
    __syncthreads();
    if (s_last) {
      finalize_request(p, r, greedy, full, s_tok, s_M, s_S);
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ dispatch ---------

VerifyPlan verify_plan(int target_dtype, int64_t vocab_size) {
  VerifyPlan plan;
  plan.ept = 16;
  plan.g = 4;
  plan.chunk = kThreads * plan.ept;
  plan.nc = (int)((vocab_size + plan.chunk - 1) / plan.chunk);
  (void)target_dtype;
  return plan;
}

template <int DT>
static const void* kernel_for() {
  return reinterpret_cast<const void*>(&verify_kernel<DT, 16, 4>);
}

const void* verify_kernel_ptr(int target_dtype) {
  switch (target_dtype) {
    case MVSD_F32: return kernel_for<MVSD_F32>();
    case MVSD_BF16: return kernel_for<MVSD_BF16>();
    case MVSD_F16: return kernel_for<MVSD_F16>();
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
      hipLaunchKernelGGL((verify_kernel<MVSD_F32, 16, 4>), dim3(grid), dim3(kThreads), 0, stream, params);
      break;
    case MVSD_BF16:
      hipLaunchKernelGGL((verify_kernel<MVSD_BF16, 16, 4>), dim3(grid), dim3(kThreads), 0, stream, params);
      break;
    case MVSD_F16:
      hipLaunchKernelGGL((verify_kernel<MVSD_F16, 16, 4>), dim3(grid), dim3(kThreads), 0, stream, params);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mvsd
