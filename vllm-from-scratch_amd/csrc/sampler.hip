// Row kernels of the regular sampler as the rejection sampler uses it for bonus tokens
// (minivllm/sample/sampler.py:73-120, :243-349; ops/topk_topp_sampler.py:82-91):
//   argmax_rows      greedy_sample: argmax of each row (NaN first, lowest index on ties)
//   min_p_rows       apply_min_p: p = softmax(x); entries with p < max(p) * min_p -> -inf
//   race_rows        random_sample: argmax of softmax(x) / E per row (exponential race)
//   log_softmax_rows compute_logprobs: (x - max) - log(sum exp(x - max))
// One 256-thread workgroup per row; every row is fp32 with unit column stride.
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

__global__ __launch_bounds__(kSmpThreads) void race_rows_kernel(int32_t* out, const float* x,
                                                                int64_t stride, const float* noise,
                                                                int64_t noise_stride, int V) {
  __shared__ float s_m[kSmpWaves], s_s[kSmpWaves];
  __shared__ uint64_t s_k[kSmpWaves];
  const float* row = x + (int64_t)blockIdx.x * stride;
  const float* e = noise + (int64_t)blockIdx.x * noise_stride;
  float M, S;
  row_stats(row, V, s_m, s_s, M, S);
  uint64_t best = 0;
  for (int i = threadIdx.x; i < V; i += kSmpThreads) {
    const float prob = expf(row[i] - M) / S;
    const uint64_t k = argmax_key(prob / e[i], i);
    best = k > best ? k : best;
  }
  best = block_max_key(best, s_k);
  if (threadIdx.x == 0) out[blockIdx.x] = min(max(key_index(best), 0), V - 1);
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
    case kSamplerRace:
      hipLaunchKernelGGL(race_rows_kernel, grid, block, 0, stream, ids, x, stride, aux,
                         aux_stride, (int)V);
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

}  // namespace mvsd
