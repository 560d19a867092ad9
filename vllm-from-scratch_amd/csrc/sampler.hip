// Row kernels of the regular sampler as the rejection sampler uses it for bonus tokens
// (minivllm/sample/sampler.py:73-120, :243-349; ops/topk_topp_sampler.py:82-91):
//   argmax_rows      greedy_sample: argmax of each row (NaN first, lowest index on ties)
//   min_p_rows       apply_min_p: p = softmax(x); entries with p < max(p) * min_p -> -inf
//   log_softmax_rows compute_logprobs: (x - max) - log(sum exp(x - max))
// one 256-thread workgroup per row; and the exponential race of random_sample (argmax of
// softmax(x / T) / E per row) over 8192-column chunks of every row:
//   race_stats   (max, sum exp(v - max)) of each chunk, v = fl(x / T) or x
//   race_keys    each chunk combines its row's chunk statistics in chunk order (the same
//                M and S in every workgroup of the row) and keeps its best
//                (exp(v - M) / S) / E key, the reference's two fp32 roundings
//   race_pick    one wavefront per row takes the best chunk key
// Every row is fp32 with unit column stride.
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

// Chunk (max, sum exp(v - max)) of v = x[i] / T (DIV) or x[i] over [begin, end); thread 0
// receives the block's pair.  Four columns per thread and iteration from 16-byte loads when
// VEC (row and chunk start 16-byte aligned), then the chunk's scalar tail.
template <bool DIV, bool VEC>
__device__ inline float2 race_chunk_stats(const float* row, int begin, int end, float T,
                                          float* s_m, float* s_s) {
  float m = -INFINITY, s = 0.f;
  auto add = [&](float x) {
    const float v = DIV ? x / T : x;
    if (v > m) {
      s = s * expf(m - v);
      m = v;
    }
    if (v != -INFINITY) s += expf(v - m);
  };
  int i = begin;
  if (VEC) {
    const int vend = begin + ((end - begin) & ~(4 * kSmpThreads - 1));
    for (; i < vend; i += 4 * kSmpThreads) {
      const float4 x = *reinterpret_cast<const float4*>(row + i + 4 * threadIdx.x);
      add(x.x);
      add(x.y);
      add(x.z);
      add(x.w);
    }
  }
  for (i += threadIdx.x; i < end; i += kSmpThreads) add(row[i]);
  const float wm = wave_max(m);
  const float ws = wave_sum(m == -INFINITY ? 0.f : s * expf(m - wm));
  if (lane_id() == 0) {
    s_m[wave_id()] = wm;
    s_s[wave_id()] = ws;
  }
  __syncthreads();
  float M = -INFINITY, S = 0.f;
  for (int w = 0; w < kSmpWaves; ++w) M = fmaxf(M, s_m[w]);
  for (int w = 0; w < kSmpWaves; ++w)
    if (s_m[w] != -INFINITY) S += s_s[w] * expf(s_m[w] - M);
  return make_float2(M, S);
}

template <bool DIV, bool VEC>
__global__ __launch_bounds__(kSmpThreads) void race_stats_kernel(float2* part, const float* x,
                                                                 int64_t stride,
                                                                 const float* temperature,
                                                                 int V, int nch) {
  __shared__ float s_m[kSmpWaves], s_s[kSmpWaves];
  const int r = blockIdx.x / nch, c = blockIdx.x % nch;
  const int begin = c * kRaceChunk, end = min(V, begin + kRaceChunk);
  const float T = DIV ? temperature[r] : 1.f;
  const float2 ms = race_chunk_stats<DIV, VEC>(x + (int64_t)r * stride, begin, end, T, s_m, s_s);
  if (threadIdx.x == 0) part[blockIdx.x] = ms;
}

template <bool DIV, bool VEC>
__global__ __launch_bounds__(kSmpThreads) void race_keys_kernel(
    uint64_t* keys, const float2* part, const float* x, int64_t stride, const float* noise,
    int64_t noise_stride, const float* temperature, int V, int nch) {
#pragma clang fp contract(off)
  __shared__ float2 s_part[kRaceMaxChunks];
  __shared__ uint64_t s_k[kSmpWaves];
  const int r = blockIdx.x / nch, c = blockIdx.x % nch;
  for (int j = threadIdx.x; j < nch; j += kSmpThreads) s_part[j] = part[(int64_t)r * nch + j];
  __syncthreads();
  // the row's statistics, combined in chunk order
  float M = -INFINITY, S = 0.f;
  for (int j = 0; j < nch; ++j) M = fmaxf(M, s_part[j].x);
  for (int j = 0; j < nch; ++j)
    if (s_part[j].x != -INFINITY) S += s_part[j].y * expf(s_part[j].x - M);
  const float T = DIV ? temperature[r] : 1.f;
  const float* row = x + (int64_t)r * stride;
  const float* e = noise + (int64_t)r * noise_stride;
  const int begin = c * kRaceChunk, end = min(V, begin + kRaceChunk);
  uint64_t best = 0;
  auto score = [&](float xv, float ev, int i) {
    const float v = DIV ? xv / T : xv;
    const float prob = expf(v - M) / S;
    const uint64_t k = argmax_key(prob / ev, i);
    best = k > best ? k : best;
  };
  int i = begin;
  if (VEC) {
    const int vend = begin + ((end - begin) & ~(4 * kSmpThreads - 1));
    for (; i < vend; i += 4 * kSmpThreads) {
      const int j = i + 4 * threadIdx.x;
      const float4 xv = *reinterpret_cast<const float4*>(row + j);
      const float4 ev = *reinterpret_cast<const float4*>(e + j);
      score(xv.x, ev.x, j);
      score(xv.y, ev.y, j + 1);
      score(xv.z, ev.z, j + 2);
      score(xv.w, ev.w, j + 3);
    }
  }
  for (i += threadIdx.x; i < end; i += kSmpThreads) score(row[i], e[i], i);
  best = block_max_key(best, s_k);
  if (threadIdx.x == 0) keys[blockIdx.x] = best;
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
  const int64_t part = (rows * nch * (int64_t)sizeof(float2) + 255) & ~int64_t(255);
  return part + rows * nch * (int64_t)sizeof(uint64_t);
}

template <bool DIV, bool VEC>
static void launch_race(int32_t* ids, const float* x, int64_t stride, const float* noise,
                        int64_t noise_stride, const float* temperature, int64_t rows, int V,
                        int nch, float2* part, uint64_t* keys, hipStream_t stream) {
  const dim3 grid((unsigned)(rows * nch)), block(kSmpThreads);
  hipLaunchKernelGGL((race_stats_kernel<DIV, VEC>), grid, block, 0, stream, part, x, stride,
                     temperature, V, nch);
  hipLaunchKernelGGL((race_keys_kernel<DIV, VEC>), grid, block, 0, stream, keys, part, x,
                     stride, noise, noise_stride, temperature, V, nch);
  hipLaunchKernelGGL(race_pick_kernel, dim3((unsigned)((rows + kSmpWaves - 1) / kSmpWaves)),
                     block, 0, stream, ids, keys, rows, nch, V);
}

hipError_t launch_sampler_race(int32_t* ids, const float* x, int64_t stride, const float* noise,
                               int64_t noise_stride, const float* temperature, int64_t rows,
                               int64_t V, void* workspace, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int nch = (int)((V + kRaceChunk - 1) / kRaceChunk);
  float2* part = static_cast<float2*>(workspace);
  const int64_t part_bytes = (rows * nch * (int64_t)sizeof(float2) + 255) & ~int64_t(255);
  uint64_t* keys = reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(workspace) + part_bytes);
  const bool vec = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(noise)) & 15) == 0
                   && stride % 4 == 0 && noise_stride % 4 == 0;
  if (temperature) {
    if (vec)
      launch_race<true, true>(ids, x, stride, noise, noise_stride, temperature, rows, (int)V,
                              nch, part, keys, stream);
    else
      launch_race<true, false>(ids, x, stride, noise, noise_stride, temperature, rows, (int)V,
                               nch, part, keys, stream);
  } else {
    if (vec)
      launch_race<false, true>(ids, x, stride, noise, noise_stride, nullptr, rows, (int)V, nch,
                               part, keys, stream);
    else
      launch_race<false, false>(ids, x, stride, noise, noise_stride, nullptr, rows, (int)V, nch,
                                part, keys, stream);
  }
  return hipGetLastError();
}

}  // namespace mvsd
