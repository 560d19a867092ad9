// On-device checks of the arithmetic assumptions the kernels rely on (mvsd_selftest).
#include "mvsd_device.h"
#include "selftest.h"

namespace mvsd {
namespace {

// recip_rn(b) == 1.0f / b for every b = 2^(e - 127) * 1.m, e in [e0, e1], every mantissa.
__global__ __launch_bounds__(256) void reciprocal_kernel(int e0, int e1,
                                                         unsigned long long* failures) {
  const uint32_t m = blockIdx.x * 256 + threadIdx.x;
  if (m >= (1u << 23)) return;
  int bad = 0;
  for (int e = e0; e <= e1; ++e) {
    const float b = __uint_as_float(((uint32_t)e << 23) | m);
    bad += recip_rn(b) != 1.0f / b;
  }
  if (bad) atomicAdd(failures, (unsigned long long)bad);
}

// divide(make_divider(t), x) == x / t (bit for bit; any NaN equals any NaN) for every float x.
__global__ __launch_bounds__(256) void division_kernel(float t, unsigned long long* failures) {
  const Divider d = make_divider(t);
  const uint32_t base = (blockIdx.x * 256u + threadIdx.x) * 256u;
  int bad = 0;
  for (uint32_t j = 0; j < 256u; ++j) {
    const float x = __uint_as_float(base + j);
    const float a = divide(d, x), b = x / t;
    bad += (__float_as_uint(a) != __float_as_uint(b)) & !((a != a) & (b != b));
  }
  if (bad) atomicAdd(failures, (unsigned long long)bad);
}

}  // namespace

hipError_t launch_selftest_division(const float* divisors, int n, unsigned long long* failures,
                                    hipStream_t stream) {
  for (int i = 0; i < n; ++i) {
    hipLaunchKernelGGL(division_kernel, dim3(65536), dim3(256), 0, stream, divisors[i], failures);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

hipError_t launch_selftest_reciprocal(unsigned long long* failures, hipStream_t stream) {
  hipLaunchKernelGGL(reciprocal_kernel, dim3((1u << 23) / 256), dim3(256), 0, stream, 1, 252,
                     failures);
  return hipGetLastError();
}

}  // namespace mvsd
