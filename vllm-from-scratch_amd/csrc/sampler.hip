// Row kernels of the regular sampler as the rejection sampler uses it for bonus tokens
// (minivllm/sample/sampler.py:73-120, :243-349; ops/topk_topp_sampler.py:82-91):
//   argmax_rows      greedy_sample: argmax of each row (NaN first, lowest index on ties)
//   min_p_rows       apply_min_p: p = softmax(x); entries with p < max(p) * min_p -> -inf
//   log_softmax_rows compute_logprobs: (x - max) - log(sum exp(x - max))
// one 256-thread workgroup per row; and the exponential race of random_sample (argmax of
// softmax(x / T) / E per row) in one pass over 8192-column chunks of every row:
//   race_kernel  each chunk's best key of v log2(e) - log2(E), v = fl(x / T) or x (the
//                argmax of softmax(v) / E, whose max and sum are common to the row), or of x
//                for greedy rows
//   race_pick    one wavefront per row takes the best chunk key
// Rows are fp32 (or, for the race, bf16 / fp16 upcast in the kernel) with unit column stride.
#include <type_traits>

#include "mvsd_device.h"
#include "sampler.h"

namespace mvsd {

constexpr int kSmpThreads = 256;
constexpr int kSmpWaves = kSmpThreads / kWave;

// Block (max, sum exp(x - max)) of a row; every thread receives both.
__device__ inline void row_stats(const float* x, int V, float* s_m, float* s_s, float& M,
                                 float& S) {
  float m = -INFINITY, s = 0.f;
  for (int i = threadIdx.x; i < V; i += kSmpThreads) {
    const float v = x[i];
    if (v > m) {
      s = s * expf(m - v);
      m = v;
    }
    if (v != -INFINITY) s += expf(v - m);  // masked entries add nothing (and no NaN)
  }
  const float wm = wave_max(m);
  const float ws = wave_sum(m == -INFINITY ? 0.f : s * expf(m - wm));
  if (lane_id() == 0) {
    s_m[wave_id()] = wm;
    s_s[wave_id()] = ws;
  }
  __syncthreads();
  M = -INFINITY;
  for (int w = 0; w < kSmpWaves; ++w) M = fmaxf(M, s_m[w]);
  S = 0.f;
  for (int w = 0; w < kSmpWaves; ++w)
    if (s_m[w] != -INFINITY) S += s_s[w] * expf(s_m[w] - M);
}

// Block argmax of (value, index) keys to every thread.
__device__ inline uint64_t block_max_key(uint64_t k, uint64_t* s_k) {
  const uint64_t w = wave_max_u64(k);
  if (lane_id() == 0) s_k[wave_id()] = w;
  __syncthreads();
  uint64_t best = 0;
  for (int i = 0; i < kSmpWaves; ++i) best = s_k[i] > best ? s_k[i] : best;
  return best;
}

__global__ __launch_bounds__(kSmpThreads) void argmax_rows_kernel(int32_t* out, const float* x,
                                                                  int64_t stride, int V) {
  __shared__ uint64_t s_k[kSmpWaves];
  const float* row = x + (int64_t)blockIdx.x * stride;
  uint64_t best = 0;
  for (int i = threadIdx.x; i < V; i += kSmpThreads) {
    const uint64_t k = argmax_key(row[i], i);
    best = k > best ? k : best;
  }
  best = block_max_key(best, s_k);
  if (threadIdx.x == 0) out[blockIdx.x] = min(max(key_index(best), 0), V - 1);
}

__global__ __launch_bounds__(kSmpThreads) void min_p_rows_kernel(float* x, int64_t stride, int V,
                                                                 const float* min_p) {
#pragma clang fp contract(off)
  __shared__ float s_m[kSmpWaves], s_s[kSmpWaves];
  const float mp = min_p[blockIdx.x];
  if (!(mp > 0.f)) return;  // no min_p on this row: the mask is empty (probabilities >= 0)
  float* row = x + (int64_t)blockIdx.x * stride;
  float M, S;
  row_stats(row, V, s_m, s_s, M, S);
  // the largest probability is exp(0) / S; the threshold is that times min_p
  const float adjusted = (1.f / S) * mp;
  for (int i = threadIdx.x; i < V; i += kSmpThreads) {
    const float prob = expf(row[i] - M) / S;
    if (prob < adjusted) row[i] = -INFINITY;
  }
}

// ------------------------------------------------------------------ the race ---------
// random_sample's token is argmax_i softmax(v)_i / E_i (v = fl(x / T), or x): with M and S the
// row's max and sum of exp(v - M), softmax(v)_i / E_i = exp(v_i - M) / (S E_i), whose argmax is
// that of v_i log2(e) - log2(E_i), M and S being common to the row.  So one pass over the row
// needs no statistics: each workgroup keeps its chunk's best key of v log2(e) - log2(E) (one
// FMA after the hardware log2), and race_pick takes the row's best.  The evaluated keys differ
// from the reference's two fp32 roundings of exp(v - M) / S / E by a few ulps of their
// magnitude (|v| log2(e) + |log2 E|), so only near-ties closer than that can pick another
// index.  Rows the reference maps to all-NaN probabilities (a NaN or +inf value: x - max is
// NaN; or every value -inf) give index 0, the first NaN.  Greedy rows (temperature below
// greedy_eps) take the argmax of the raw row and read no noise.
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kRaceMode = 0, kRaceDivide = 1, kRaceGreedy = 2;
constexpr uint64_t kRaceNaNRow = ~0ull;  // chunk key of a row whose probabilities are NaN: index 0

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ inline float4 f32x4_of(u32x4 q) {
  return make_float4(__uint_as_float(q[0]), __uint_as_float(q[1]), __uint_as_float(q[2]),
                     __uint_as_float(q[3]));
}

template <int DT>
using RaceQuad = std::conditional_t<Elem<DT>::kVec == 4, u32x4, u32x2>;

// 4 consecutive columns of a DT row starting at column i (16-byte aligned for fp32, 8-byte
// for 16-bit types), as fp32.
template <int DT>
__device__ inline void race_load4(const typename Elem<DT>::storage* row, int i, float (&v)[4]) {
  using S = typename Elem<DT>::storage;
  const RaceQuad<DT> q = __builtin_nontemporal_load(reinterpret_cast<const RaceQuad<DT>*>(row + i));
  const S* s = reinterpret_cast<const S*>(&q);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = Elem<DT>::cvt(s[j]);
}

template <int DT, int MODE, bool VEC>
__device__ inline uint64_t race_chunk(const typename Elem<DT>::storage* row, const float* e,
                                      int begin, int end, const Divider& dv) {
  uint64_t best = 0;
  bool nan_row = false;
  auto score = [&](float xv, float ev, int i) {
    if constexpr (MODE == kRaceGreedy) {
      best = umax64(best, argmax_key(xv, i));
    } else {
      const float v = MODE == kRaceDivide ? divide(dv, xv) : xv;
      nan_row |= (v != v) | (v == INFINITY);
      const float key = fmaf(v, kLog2e, -__builtin_amdgcn_logf(ev));
      best = umax64(best, argmax_key(key, i));
    }
  };
  int i = begin;
  if (VEC) {
    // 4 columns per lane and step: one 16-byte (fp32) or 8-byte (16-bit) load of the row and
    // one 16-byte load of the noise
    constexpr int kStep = 4 * kSmpThreads;
    const int vend = begin + ((end - begin) & ~(kStep - 1));
#pragma unroll 4
    for (; i < vend; i += kStep) {
      const int j = i + 4 * threadIdx.x;
      float xv[4];
      race_load4<DT>(row, j, xv);
      float4 ev = make_float4(1.f, 1.f, 1.f, 1.f);  // greedy rows read no noise
      if constexpr (MODE != kRaceGreedy)
        ev = f32x4_of(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(e + j)));
      score(xv[0], ev.x, j);
      score(xv[1], ev.y, j + 1);
      score(xv[2], ev.z, j + 2);
      score(xv[3], ev.w, j + 3);
    }
  }
  for (i += threadIdx.x; i < end; i += kSmpThreads)
    score(Elem<DT>::cvt(row[i]), MODE == kRaceGreedy ? 1.f : e[i], i);
  if constexpr (MODE == kRaceGreedy) return best;
  // probabilities of the whole row are NaN: this chunk's key outranks every other
  return __builtin_amdgcn_ballot_w64(nan_row) != 0 ? kRaceNaNRow : best;
}

// One workgroup per (row r, chunk c of kRaceChunk columns): keys[r * nch + c] = the chunk's
// best key.  Row r is x + row_index[r] * stride, the index clamped to [0, num_x_rows) (or
// x + r * stride).  Without noise every row is greedy.
template <int DT, bool VEC>
__global__ __launch_bounds__(kSmpThreads) void race_kernel(
    uint64_t* keys, const void* x, int64_t stride, const int32_t* row_index, int64_t num_x_rows,
    const float* noise, int64_t noise_stride, const float* temperature, float greedy_eps, int V,
    int nch) {
  using S = typename Elem<DT>::storage;
  __shared__ uint64_t s_k[kSmpWaves];
  const int r = blockIdx.x / nch, c = blockIdx.x % nch;
  const int64_t xr = row_index ? min(max((int64_t)row_index[r], (int64_t)0), num_x_rows - 1)
                               : (int64_t)r;
  const S* row = static_cast<const S*>(x) + xr * stride;
  const float* e = noise ? noise + (int64_t)r * noise_stride : nullptr;
  const int begin = c * kRaceChunk, end = min(V, begin + kRaceChunk);
  const float T = temperature ? temperature[r] : 1.f;
  const Divider dv = make_divider(T);
  uint64_t best;
  if (!noise || (temperature && T < greedy_eps))
    best = race_chunk<DT, kRaceGreedy, VEC>(row, e, begin, end, dv);
  else if (!temperature) best = race_chunk<DT, kRaceMode, VEC>(row, e, begin, end, dv);
  else best = race_chunk<DT, kRaceDivide, VEC>(row, e, begin, end, dv);
  const uint64_t w = wave_max_u64(best);
  if (lane_id() == 0) s_k[wave_id()] = w;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = 0;
    for (int k = 0; k < kSmpWaves; ++k) b = umax64(b, s_k[k]);
    keys[blockIdx.x] = b;
  }
}

// One wavefront per row: the best of the row's chunk keys.
__global__ __launch_bounds__(kSmpThreads) void race_pick_kernel(int32_t* ids,
                                                                const uint64_t* keys,
                                                                int64_t rows, int nch, int V) {
  const int64_t r = (int64_t)blockIdx.x * kSmpWaves + wave_id();
  if (r >= rows) return;
  uint64_t best = 0;
  for (int j = lane_id(); j < nch; j += kWave) {
    const uint64_t k = keys[r * nch + j];
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  if (lane_id() == 0) ids[r] = min(max(key_index(best), 0), V - 1);
}

__global__ __launch_bounds__(kSmpThreads) void log_softmax_rows_kernel(float* out,
                                                                       int64_t out_stride,
                                                                       const float* x,
                                                                       int64_t stride, int V) {
#pragma clang fp contract(off)
  __shared__ float s_m[kSmpWaves], s_s[kSmpWaves];
  const float* row = x + (int64_t)blockIdx.x * stride;
  float* dst = out + (int64_t)blockIdx.x * out_stride;
  float M, S;
  row_stats(row, V, s_m, s_s, M, S);
  const float L = logf(S);
  for (int i = threadIdx.x; i < V; i += kSmpThreads) dst[i] = (row[i] - M) - L;
}

hipError_t launch_sampler_rows(int op, int32_t* ids, float* out, int64_t out_stride,
                               float* x, int64_t stride, const float* aux, int64_t aux_stride,
                               int64_t rows, int64_t V, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const dim3 grid((unsigned)rows), block(kSmpThreads);
  switch (op) {
    case kSamplerArgmax:
      hipLaunchKernelGGL(argmax_rows_kernel, grid, block, 0, stream, ids, x, stride, (int)V);
      break;
    case kSamplerMinP:
      hipLaunchKernelGGL(min_p_rows_kernel, grid, block, 0, stream, x, stride, (int)V, aux);
      break;
    case kSamplerLogSoftmax:
      hipLaunchKernelGGL(log_softmax_rows_kernel, grid, block, 0, stream, out, out_stride, x,
                         stride, (int)V);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int64_t sampler_race_workspace_bytes(int64_t rows, int64_t V) {
  const int64_t nch = (V + kRaceChunk - 1) / kRaceChunk;
  return rows * nch * (int64_t)sizeof(uint64_t);
}

template <int DT>
static void launch_race_dt(int32_t* ids, const void* x, int64_t stride, const int32_t* row_index,
                           int64_t num_x_rows, const float* noise, int64_t noise_stride,
                           const float* temperature, float greedy_eps, int64_t rows, int V,
                           int nch, uint64_t* keys, bool vec, hipStream_t stream) {
  const dim3 grid((unsigned)(rows * nch)), block(kSmpThreads);
  if (vec)
    hipLaunchKernelGGL((race_kernel<DT, true>), grid, block, 0, stream, keys, x, stride,
                       row_index, num_x_rows, noise, noise_stride, temperature, greedy_eps, V,
                       nch);
  else
    hipLaunchKernelGGL((race_kernel<DT, false>), grid, block, 0, stream, keys, x, stride,
                       row_index, num_x_rows, noise, noise_stride, temperature, greedy_eps, V,
                       nch);
  hipLaunchKernelGGL(race_pick_kernel, dim3((unsigned)((rows + kSmpWaves - 1) / kSmpWaves)),
                     block, 0, stream, ids, keys, rows, nch, V);
}

hipError_t launch_sampler_race(int32_t* ids, const void* x, int x_dtype, int64_t stride,
                               const int32_t* row_index, int64_t num_x_rows, const float* noise,
                               int64_t noise_stride, const float* temperature, float greedy_eps,
                               int64_t rows, int64_t V, void* workspace, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int nch = (int)((V + kRaceChunk - 1) / kRaceChunk);
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  const int esize = x_dtype == MVSD_F32 ? 4 : 2;
  // every 4-column quad of every row is aligned (16 bytes for fp32 rows, 8 for 16-bit rows)
  // and so is every noise quad; greedy-only calls may pass no noise
  const bool vec = (reinterpret_cast<uintptr_t>(x) & (4 * esize - 1)) == 0 && stride % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(noise) & 15) == 0 && noise_stride % 4 == 0;
  switch (x_dtype) {
    case MVSD_F32:
      launch_race_dt<MVSD_F32>(ids, x, stride, row_index, num_x_rows, noise, noise_stride,
                               temperature, greedy_eps, rows, (int)V, nch, keys, vec, stream);
      break;
    case MVSD_BF16:
      launch_race_dt<MVSD_BF16>(ids, x, stride, row_index, num_x_rows, noise, noise_stride,
                                temperature, greedy_eps, rows, (int)V, nch, keys, vec, stream);
      break;
    case MVSD_F16:
      launch_race_dt<MVSD_F16>(ids, x, stride, row_index, num_x_rows, noise, noise_stride,
                               temperature, greedy_eps, rows, (int)V, nch, keys, vec, stream);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mvsd
