// Row-wise helpers behind the reference's module-level functions:
//   expand_batch_to_tokens   (minivllm/sample/rejection_sampler.py:574-597, :826-847)
//   softmax over verify rows (minivllm/sample/rejection_sampler.py:502)
//   sample_recovered_tokens  (minivllm/sample/rejection_sampler.py:627-670, :850-928)
// The fused path (verify.hip) does not use these; they keep the reference's standalone
// functions and test seams available with the same semantics.
#include <float.h>

#include "mvsd_device.h"
#include "rows.h"

namespace mvsd {

// ------------------------------------------------------------------ expand -----------
// One 64-lane block per request: out[j] = replace(x[i]) for j in [cu[i-1], cu[i]).
template <typename T>
__global__ __launch_bounds__(64) void expand_kernel(T* out, const T* x, const int32_t* cu,
                                                    int64_t num_tokens, T from, T to) {
  const int r = blockIdx.x;
  const int begin = r == 0 ? 0 : cu[r - 1];
  const int end = cu[r];
  T v = x[r];
  if (v == from) v = to;
  for (int j = begin + (int)threadIdx.x; j < end; j += 64) {
    if (j >= 0 && j < num_tokens) out[j] = v;
  }
}

hipError_t launch_expand(void* out, const void* x, int dtype, const int32_t* cu, int64_t B,
                         int64_t num_tokens, double from, double to, hipStream_t stream) {
  const dim3 grid((unsigned)B), block(64);
  switch (dtype) {
    case MVSD_F32:
      hipLaunchKernelGGL(expand_kernel<float>, grid, block, 0, stream, (float*)out,
                         (const float*)x, cu, num_tokens, (float)from, (float)to);
      break;
    case MVSD_F64:
      hipLaunchKernelGGL(expand_kernel<double>, grid, block, 0, stream, (double*)out,
                         (const double*)x, cu, num_tokens, from, to);
      break;
    case MVSD_I32:
      hipLaunchKernelGGL(expand_kernel<int32_t>, grid, block, 0, stream, (int32_t*)out,
                         (const int32_t*)x, cu, num_tokens, (int32_t)from, (int32_t)to);
      break;
    case MVSD_I64:
      hipLaunchKernelGGL(expand_kernel<int64_t>, grid, block, 0, stream, (int64_t*)out,
                         (const int64_t*)x, cu, num_tokens, (int64_t)from, (int64_t)to);
      break;
    case MVSD_U8:
      hipLaunchKernelGGL(expand_kernel<uint8_t>, grid, block, 0, stream, (uint8_t*)out,
                         (const uint8_t*)x, cu, num_tokens, (uint8_t)from, (uint8_t)to);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ softmax ----------
// One block per row: online (max, sumexp) over the row, then write exp(x - M) / S.
template <int DT>
__global__ __launch_bounds__(kThreads) void softmax_rows_kernel(float* probs, int64_t probs_stride,
                                                                const void* logits,
                                                                int64_t logits_stride,
                                                                const float* temperature,
                                                                int64_t V) {
  using S = typename Elem<DT>::storage;
  __shared__ float s_red[kWaves];
  const int64_t row = blockIdx.x;
  const S* src = static_cast<const S*>(logits) + row * logits_stride;
  float t = temperature ? temperature[row] : 1.f;
  if (t == 0.f) t = 1.f;
  float m = -INFINITY, s = 0.f;
  for (int64_t v = threadIdx.x; v < V; v += kThreads) {
    float x = Elem<DT>::cvt(src[v]);
    if (t != 1.f) x = x / t;
    if (x > m) {
      s = (m == -INFINITY) ? 0.f : s * expf(m - x);
      m = x;
    }
    if (x != -INFINITY) s += expf(x - m);
  }
  float mm[1] = {m};
  block_max<1>(mm, s_red);
  float ss[1] = {(m == -INFINITY) ? 0.f : s * expf(m - mm[0])};
  block_sum<1>(ss, s_red);
  const float M = mm[0], Ssum = ss[0];
  float* dst = probs + row * probs_stride;
  for (int64_t v = threadIdx.x; v < V; v += kThreads) {
    float x = Elem<DT>::cvt(src[v]);
    if (t != 1.f) x = x / t;
    dst[v] = expf(x - M) / Ssum;
  }
}

hipError_t launch_softmax_rows(float* probs, int64_t probs_stride, const void* logits, int dtype,
                               int64_t logits_stride, const float* temperature,
                               int64_t num_rows, int64_t V, hipStream_t stream) {
  const dim3 grid((unsigned)num_rows), block(kThreads);
  switch (dtype) {
    case MVSD_F32:
      hipLaunchKernelGGL(softmax_rows_kernel<MVSD_F32>, grid, block, 0, stream, probs,
                         probs_stride, logits, logits_stride, temperature, V);
      break;
    case MVSD_BF16:
      hipLaunchKernelGGL(softmax_rows_kernel<MVSD_BF16>, grid, block, 0, stream, probs,
                         probs_stride, logits, logits_stride, temperature, V);
      break;
    case MVSD_F16:
      hipLaunchKernelGGL(softmax_rows_kernel<MVSD_F16>, grid, block, 0, stream, probs,
                         probs_stride, logits, logits_stride, temperature, V);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ recovered --------
// Grid (B, max_spec_len) as in the reference kernel: block (r, pos) scores verify row
// cu[r-1] + pos over the whole vocabulary and writes the first-index argmax, clamped to V-1.
__global__ __launch_bounds__(kThreads) void recovered_kernel(
    int32_t* out, const int32_t* cu, const int32_t* draft_ids, const float* draft_probs,
    int64_t draft_stride, const float* target_probs, int64_t target_stride,
    const float* noise, int64_t noise_stride, int64_t V, int64_t P) {
  __shared__ float s_v[kWaves];
  __shared__ int s_i[kWaves];
  const int r = blockIdx.x;
  const int pos = blockIdx.y;
  // request range clamped to [0, P] so inconsistent cu values cannot index out of bounds
  int64_t begin = r == 0 ? 0 : cu[r - 1];
  int64_t end = cu[r];
  begin = begin < 0 ? 0 : (begin > P ? P : begin);
  end = end < begin ? begin : (end > P ? P : end);
  if (pos >= end - begin) return;
  const int64_t row = begin + pos;
  const int d = draft_ids[row];
  const float* tp = target_probs + row * target_stride;
  const float* dp = draft_probs ? draft_probs + row * draft_stride : nullptr;
  const float* np = noise + (int64_t)r * noise_stride;
  float bv = -INFINITY;
  int bi = INT_MAX;
  for (int64_t v = threadIdx.x; v < V; v += kThreads) {
    const float prob = tp[v];
    const float w = dp ? fmaxf(prob - dp[v], 0.f) : (v == d ? 0.f : prob);
    const float score = w * (1.0f / np[v]);
    argmax_update(bv, bi, score, (int)v, true);
  }
  float vv[1] = {bv};
  int ii[1] = {bi};
  block_argmax<1>(vv, ii, s_v, s_i);
  if (threadIdx.x == 0) out[row] = min(ii[0], (int)V - 1);
}

hipError_t launch_recovered(int32_t* out, const int32_t* cu, const int32_t* draft_ids,
                            const float* draft_probs, int64_t draft_stride,
                            const float* target_probs, int64_t target_stride,
                            const float* noise, int64_t noise_stride, int64_t B,
                            int64_t max_spec_len, int64_t V, int64_t P, hipStream_t stream) {
  hipLaunchKernelGGL(recovered_kernel, dim3((unsigned)B, (unsigned)max_spec_len), dim3(kThreads),
                     0, stream, out, cu, draft_ids, draft_probs, draft_stride, target_probs,
                     target_stride, noise, noise_stride, V, P);
  return hipGetLastError();
}

}  // namespace mvsd
