// k_elem.hip -- small elementwise kernels used around the hot path.
#include "qh_internal.h"

namespace qh {

thread_local LaunchTiming g_launch_timing;

namespace {

__global__ void k_axpy_inplace(float *__restrict__ y, const float *__restrict__ x,
                               int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = y[i] + x[i];
}

__global__ void k_zero(float *__restrict__ y, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = 0.0f;
}

__global__ void k_bf16_to_f32(const uint16_t *__restrict__ x, float *__restrict__ y,
                              int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = __uint_as_float((uint32_t)x[i] << 16);
}

}  // namespace

hipError_t launch_axpy_inplace(float *y, const float *x, int64_t n,
                               hipStream_t s) {
  if (n == 0) return hipSuccess;
  k_axpy_inplace<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(y, x, n);
  return hipGetLastError();
}

// A fill kernel rather than hipMemsetAsync, so that a caller may capture the
// call in a HIP graph.
hipError_t launch_zero(float *y, int64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  k_zero<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(y, n);
  return hipGetLastError();
}

hipError_t launch_bf16_to_f32(const uint16_t *x, float *y, int64_t n,
                              hipStream_t s) {
  if (n == 0) return hipSuccess;
  k_bf16_to_f32<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(x, y, n);
  return hipGetLastError();
}

}  // namespace qh
