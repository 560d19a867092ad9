// Host launchers of the row-wise helper kernels (rows.hip) and the ngram kernel (ngram.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

hipError_t launch_expand(void* out, const void* x, int dtype, const int32_t* cu, int64_t B,
                         int64_t num_tokens, double from, double to, hipStream_t stream);

hipError_t launch_softmax_rows(float* probs, int64_t probs_stride, const void* logits, int dtype,
                               int64_t logits_stride, const float* temperature,
                               int64_t num_rows, int64_t V, hipStream_t stream);

hipError_t launch_recovered(int32_t* out, const int32_t* cu, const int32_t* draft_ids,
                            const float* draft_probs, int64_t draft_stride,
                            const float* target_probs, int64_t target_stride,
                            const float* noise, int64_t noise_stride, int64_t B,
                            int64_t max_spec_len, int64_t V, int64_t P, hipStream_t stream);

constexpr int kNgramMaxN = 32;  // longest n-gram the ngram kernel supports

struct NgramParams {
  int32_t* drafts;            // [R, k]
  int32_t* num_valid;         // [R]
  int32_t* tokens;            // [R, row_stride]
  int64_t row_stride;
  int64_t max_seq_len;
  const int32_t* num_tokens;  // [R]
  const int32_t* new_tokens;  // [R, new_stride] or null
  int64_t new_stride;
  int64_t max_new;
  const int32_t* new_counts;  // [R] or null
  const uint8_t* active;      // [R] or null
  int gate_on_new_counts;
  int min_n;
  int max_n;
  int k;
  int cap_by_model_len;
  int64_t max_model_len;
};

hipError_t launch_ngram(const NgramParams& p, int64_t num_reqs, hipStream_t stream);

hipError_t launch_ngram_valid_sampled(int32_t* next_token_ids, int32_t* counts,
                                      int32_t* valid_ids, int64_t valid_stride,
                                      const int32_t* sampled, int64_t sampled_stride,
                                      int64_t width, const uint8_t* discard,
                                      const int32_t* token_ids, int64_t row_stride,
                                      const int32_t* num_tokens, int32_t vocab_size,
                                      int64_t num_reqs, hipStream_t stream);

}  // namespace mvsd
