// Host/device interface of the speculative-logprobs kernel (logprobs.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

struct LogprobParams {
  const float* target;         // verify rows, fp32, row stride tstride
  int64_t tstride;
  const int32_t* target_rows;  // [P] row of verify row v in `target`, or null (row v)
  const float* bonus;          // [B] bonus rows, fp32, row stride bstride
  int64_t bstride;
  const int32_t* cu_sampled;   // [B] cumulative K_r + 1, no leading 0
  const int32_t* tokens;       // [B, W] sampled ids, -1 padded
  int64_t tok_stride;
  int B, P, V, W, k;
  int logits_mode;             // 1: report the values themselves, 0: their log-softmax
  int flat;                    // 1: position n reads row bonus + n * bstride, token tokens[n]
  int rank_raw;                // 1: top-k order and rank compare raw values, not log-softmax
  int32_t* ids;                // [B * W, k + 1]
  float* lps;                  // [B * W, k + 1]
  int32_t* ranks;              // [B * W]
};

// Largest k the kernel supports.
hipError_t launch_spec_logprobs(const LogprobParams& p, hipStream_t stream);

}  // namespace mvsd
