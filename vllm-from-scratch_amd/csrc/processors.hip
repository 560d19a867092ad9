// Logits processors of the verify rows: penalties and min_tokens over each row's hypothetical
// history (minivllm/sample/rejection_sampler.py:338-406, minivllm/sample/ops/penalties.py:51-72,
// minivllm/sample/sampler.py:192-228), in place on the fp32 processed rows.
//
// Verify row j of request r (rows of a request are consecutive, request-major) sees the history
// "committed output + draft prefix spec[:j]" (rejection_sampler.py:387-406).  Per token t of
// the row:
//   in_prompt(t), count(t) = committed count + occurrences of t in spec[:j];
//   if in_prompt or count > 0:  x *= x > 0 ? 1 / repetition : repetition;
//   x -= frequency * count;  x -= presence * (count > 0)
// in that order and in fp32, as penalties.py:64-71 computes it over the whole row (for tokens
// outside the history the three steps are exact no-ops).  Then rows whose history is still
// shorter than min_tokens get their stop tokens set to -inf (sampler.py:204-228).
//
// The host lists, per request, every distinct token of prompt, committed output and drafts
// (ent_tok), with its committed count and prompt flag (ent_info = count | in_prompt << 31);
// the kernel adds the draft-prefix counts row by row.  One workgroup per verify row.
#include "processors.h"

namespace mvsd {

constexpr int kProcThreads = 256;

__global__ __launch_bounds__(kProcThreads) void logits_processors_kernel(ProcessorParams p) {
  // every product and difference rounds separately, as the reference's tensor ops compute
  // them: a contracted fma of v - freq * count rounds once and can differ in the last bit
#pragma clang fp contract(off)
  const int row = blockIdx.x;
  // request of the row: the first r with cu[r] > row (cu has no leading 0)
  int lo = 0, hi = p.B - 1;
  while (lo < hi) {
    const int mid = (lo + hi) / 2;
    if (p.cu[mid] > row) hi = mid;
    else lo = mid + 1;
  }
  const int r = lo;
  const int begin = r == 0 ? 0 : p.cu[r - 1];
  const int j = row - begin;  // position of the row in its request's draft block
  float* x = p.logits + (int64_t)row * p.stride;

  if (p.ent_off) {
    const float rep = p.repetition ? p.repetition[r] : 1.f;
    const float freq = p.frequency ? p.frequency[r] : 0.f;
    const float pres = p.presence ? p.presence[r] : 0.f;
    const float inv_rep = 1.f / rep;
    const int e0 = p.ent_off[r], e1 = p.ent_off[r + 1];
    for (int e = e0 + (int)threadIdx.x; e < e1; e += kProcThreads) {
      const int t = p.ent_tok[e];
      if (t < 0 || t >= p.V) continue;
      const uint32_t info = (uint32_t)p.ent_info[e];
      int cnt = (int)(info & 0x7fffffffu);
      for (int m = 0; m < j; ++m) cnt += p.spec[begin + m] == t ? 1 : 0;
      const bool in_prompt = info >> 31;
      float v = x[t];
      if (in_prompt || cnt > 0) v *= v > 0.f ? inv_rep : rep;
      v -= freq * (float)cnt;
      v -= pres * (cnt > 0 ? 1.f : 0.f);
      x[t] = v;
    }
  }
  if (p.n_mask && j < p.n_mask[r]) {
    __syncthreads();  // the penalties of this row are written first
    const int s0 = p.stop_off[r], s1 = p.stop_off[r + 1];
    for (int s = s0 + (int)threadIdx.x; s < s1; s += kProcThreads) {
      const int t = p.stop_tok[s];
      if (t >= 0 && t < p.V) x[t] = -INFINITY;
    }
  }
}

hipError_t launch_logits_processors(const ProcessorParams& p, hipStream_t stream) {
  if (p.P <= 0) return hipSuccess;
  hipLaunchKernelGGL(logits_processors_kernel, dim3((unsigned)p.P), dim3(kProcThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mvsd
