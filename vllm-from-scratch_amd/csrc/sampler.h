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

// ids[r] = argmax over i of (exp(v_i - M) / S) / noise[r][i], v = fl(x[r][i] / temperature[r])
// (or x when temperature is null), M, S the max and sum exp(v - M) of row r.
hipError_t launch_sampler_race(int32_t* ids, const float* x, int64_t stride, const float* noise,
                               int64_t noise_stride, const float* temperature, int64_t rows,
                               int64_t V, void* workspace, hipStream_t stream);

}  // namespace mvsd
