// Host/device interface of the sampler row kernels (sampler.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

constexpr int kSamplerArgmax = 0;      // ids[r] = argmax of row r
constexpr int kSamplerMinP = 1;        // min_p mask of row r in place (aux = min_p [rows])
constexpr int kSamplerLogSoftmax = 3;  // out row r = log-softmax of row r
// (op 2, the exponential race, is launch_sampler_race, which takes a workspace)

constexpr int kRaceChunk = 8192;       // columns per race workgroup
constexpr int kRaceMaxChunks = 1024;   // V <= kRaceChunk * kRaceMaxChunks

hipError_t launch_sampler_rows(int op, int32_t* ids, float* out, int64_t out_stride,
                               float* x, int64_t stride, const float* aux, int64_t aux_stride,
                               int64_t rows, int64_t V, hipStream_t stream);

// Workspace bytes of launch_sampler_race for `rows` rows of V columns.
int64_t sampler_race_workspace_bytes(int64_t rows, int64_t V);

// ids[r] = argmax over i of softmax(v)_i / noise[r][i] with v = fl(x_r[i] / temperature[r])
// (or x_r[i] when temperature is null), evaluated as argmax of v log2(e) - log2(noise[r][i]);
// rows whose temperature is below greedy_eps, and every row when noise is null, take the
// argmax of the raw row.  x_r = x + row_index[r] * stride (clamped to [0, num_x_rows)) or
// x + r * stride; x is x_dtype (MVSD_F32 / MVSD_BF16 / MVSD_F16).
hipError_t launch_sampler_race(int32_t* ids, const void* x, int x_dtype, int64_t stride,
                               const int32_t* row_index, int64_t num_x_rows, const float* noise,
                               int64_t noise_stride, const float* temperature, float greedy_eps,
                               int64_t rows, int64_t V, void* workspace, hipStream_t stream);

}  // namespace mvsd
