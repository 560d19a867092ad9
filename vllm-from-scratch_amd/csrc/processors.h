// Host/device interface of the verify-row logits processors (processors.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

struct ProcessorParams {
  float* logits;  // [P, stride] fp32 verify rows, request-major, modified in place
  int64_t stride;
  int P;
  int V;
  int B;
  const int32_t* cu;    // [B] cumulative draft counts, no leading 0
  const int32_t* spec;  // [P] draft token of each row (request r's drafts, in order)
  // penalties (ent_off null: none)
  const int32_t* ent_off;   // [B + 1] offsets into ent_tok / ent_info
  const int32_t* ent_tok;   // distinct tokens of each request's prompt, output and drafts
  const int32_t* ent_info;  // committed output count | in_prompt << 31
  const float* presence;    // [B] or null (0)
  const float* frequency;   // [B] or null (0)
  const float* repetition;  // [B] or null (1)
  // min_tokens (n_mask null: none)
  const int32_t* n_mask;    // [B] leading rows of each request whose stop tokens are masked
  const int32_t* stop_off;  // [B + 1]
  const int32_t* stop_tok;
};

hipError_t launch_logits_processors(const ProcessorParams& p, hipStream_t stream);

}  // namespace mvsd
