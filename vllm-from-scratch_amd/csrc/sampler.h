// Host/device interface of the sampler row kernels (sampler.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

constexpr int kSamplerArgmax = 0;      // ids[r] = argmax of row r
constexpr int kSamplerMinP = 1;        // min_p mask of row r in place (aux = min_p [rows])
constexpr int kSamplerRace = 2;        // ids[r] = argmax softmax(row r) / noise row r (aux)
constexpr int kSamplerLogSoftmax = 3;  // out row r = log-softmax of row r

hipError_t launch_sampler_rows(int op, int32_t* ids, float* out, int64_t out_stride,
                               float* x, int64_t stride, const float* aux, int64_t aux_stride,
                               int64_t rows, int64_t V, hipStream_t stream);

}  // namespace mvsd
