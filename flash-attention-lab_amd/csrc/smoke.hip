// Toolchain check kernel: out = alpha * x + y (the reference's smoke_axpy op,
// csrc/common/smoke.cu:12-45). It proves the gfx950 code object loads and runs on a new box.
#include "gfx950.hpp"
#include "launch.hpp"

namespace fl {
namespace {

__global__ void __launch_bounds__(256) axpy_kernel(const float* __restrict__ x,
                                                   const float* __restrict__ y, float alpha,
                                                   float* __restrict__ out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = alpha * x[i] + y[i];
}

}  // namespace

hipError_t launch_axpy(const float* x, const float* y, float alpha, float* out, int64_t n,
                       hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(axpy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, x, y,
                     alpha, out, n);
  return hipGetLastError();
}

}  // namespace fl
