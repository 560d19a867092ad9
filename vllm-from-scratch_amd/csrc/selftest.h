// Host launchers of the on-device arithmetic self-checks (selftest.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace mvsd {

// Adds to *failures the number of fp32 b in [2^-126, 2^126) with recip_rn(b) != 1.0f / b.
hipError_t launch_selftest_reciprocal(unsigned long long* failures, hipStream_t stream);
// Adds to *failures the number of (t, x), t in divisors[0, n) (host array), x every float,
// with divide(make_divider(t), x) != x / t.
hipError_t launch_selftest_division(const float* divisors, int n, unsigned long long* failures,
                                    hipStream_t stream);

}  // namespace mvsd
