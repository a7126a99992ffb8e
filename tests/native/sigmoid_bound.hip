// Test support: the largest |fast_sigmoid(x) - exact_sigmoid(x)| over every fp32
// bit pattern x (non-finite x skipped), with the device code the routing kernels
// use. The routing fast path certifies its cuts with a bound of 2^-20 on this
// difference. 65,536 workgroups x 256 threads, 256 consecutive patterns each;
// one maximum per workgroup, reduced on the host.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "../../flashinfer_mlsys_amd/csrc/moe_route_token.h"

namespace {

constexpr int kBlocks = 65536, kThreads = 256, kPerThread = 256;
static_assert((uint64_t)kBlocks * kThreads * kPerThread == (1ull << 32), "every fp32 pattern once");

__global__ __launch_bounds__(kThreads) void sigmoid_bound_kernel(double* __restrict__ block_max) {
  const uint64_t first = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) * kPerThread;
  double m = 0.0;
  for (int j = 0; j < kPerThread; ++j) {
    const float x = __uint_as_float((uint32_t)(first + j));
    if (!(fabsf(x) <= 3.402823466e+38f)) continue;
    m = fmax(m, fabs((double)moe::fast_sigmoid(x) - (double)moe::exact_sigmoid(x)));
  }
  __shared__ double red[kThreads];
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = kThreads / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] = fmax(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) block_max[blockIdx.x] = red[0];
}

}  // namespace

// Writes the maximum to *out; returns 0, or the HIP error code.
extern "C" int moe_test_fast_sigmoid_max_error(double* out) {
  double* d = nullptr;
  hipError_t e = hipMalloc(&d, kBlocks * sizeof(double));
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(sigmoid_bound_kernel, dim3(kBlocks), dim3(kThreads), 0, 0, d);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipDeviceSynchronize();
  std::vector<double> h(kBlocks);
  if (e == hipSuccess) e = hipMemcpy(h.data(), d, kBlocks * sizeof(double), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return (int)e;
  double m = 0.0;
  for (double v : h) m = v > m ? v : m;
  *out = m;
  return 0;
}
