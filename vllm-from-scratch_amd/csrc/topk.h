// Host launcher of the top-k / top-p masking kernel (topk.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

// In place on fp32 rows: logits + r * stride, r < num_rows.  top_k [num_rows] int64 or null;
// top_p [num_rows] fp32 or null.
hipError_t launch_topk_topp(float* logits, int64_t stride, const int64_t* top_k,
                            const float* top_p, int64_t num_rows, int64_t vocab_size,
                            hipStream_t stream);

}  // namespace mvsd
