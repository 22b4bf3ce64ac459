// Diagnostic entry points with no reference counterpart: elementwise access to the
// arithmetic building blocks the kernels share, so the parity tests can check them on
// the device bit for bit (deterministic sin/cos/tanh; division through a float64
// reciprocal with its subnormal redo).

#include "hipenvs_device.h"

namespace hipenvs {
namespace diag {

__global__ __launch_bounds__(kBlock) void detmath_kernel(const float* __restrict__ x, float* __restrict__ s,
                                                         float* __restrict__ c, float* __restrict__ th, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  float sv, cv;
  det_sincos(x[i], &sv, &cv);
  s[i] = sv;
  c[i] = cv;
  th[i] = det_tanh(x[i]);
}

// q = a / d as the legged kernels divide: DivRecip, redone by IEEE division on a lane
// whose quotient came out subnormal (marked = 1 there).
__global__ __launch_bounds__(kBlock) void div_recip_kernel(const float* __restrict__ a, const float* __restrict__ d,
                                                           float* __restrict__ q, uint8_t* __restrict__ marked,
                                                           int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  DivRecip div;
  float v = div(a[i], d[i], recip(d[i]));
  const bool redo = div.saw_subnormal();
  if (redo) {
    DivIEEE ieee;
    v = ieee(a[i], d[i], 0.0);
  }
  q[i] = v;
  marked[i] = redo ? 1 : 0;
}

}  // namespace diag
}  // namespace hipenvs

using namespace hipenvs;

extern "C" int hipenvs_detmath(const float* x, float* sin_out, float* cos_out, float* tanh_out, int64_t n,
                               hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!x || !sin_out || !cos_out || !tanh_out))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(diag::detmath_kernel, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), x, sin_out,
                     cos_out, tanh_out, n);
  return launch_status();
}

extern "C" int hipenvs_div_recip(const float* a, const float* d, float* q, uint8_t* marked, int64_t n,
                                 hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!a || !d || !q || !marked))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(diag::div_recip_kernel, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), a, d, q, marked,
                     n);
  return launch_status();
}
