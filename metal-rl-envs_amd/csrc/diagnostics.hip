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

// Every float32 bit pattern first + i, i < count: sqrt_rn against IEEE sqrtf and recip
// against 1.0 / (double)x, bit for bit (a NaN matches any NaN). Mismatches are counted into
// counts[0] (square root) and counts[1] (reciprocal).
__global__ __launch_bounds__(kBlock) void sqrt_recip_check_kernel(uint64_t first, uint64_t count,
                                                                  unsigned long long* __restrict__ counts) {
  const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= count) return;
  const float x = __uint_as_float((uint32_t)(first + i));
  const float s = sqrt_rn(x), s_ieee = sqrtf(x);
  const double r = recip(x), r_ieee = 1.0 / (double)x;
  const bool s_ok = __float_as_uint(s) == __float_as_uint(s_ieee) || (s != s && s_ieee != s_ieee);
  const bool r_ok = __double_as_longlong(r) == __double_as_longlong(r_ieee) || (r != r && r_ieee != r_ieee);
  if (!s_ok) atomicAdd(&counts[0], 1ull);
  if (!r_ok) atomicAdd(&counts[1], 1ull);
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

extern "C" int hipenvs_sqrt_recip_check(uint64_t first, uint64_t count, unsigned long long* counts,
                                        hipenvs_stream_t stream) {
  if (!counts || first > 0xFFFFFFFFull || count > (1ull << 32) - first) return HIPENVS_E_ARG;
  if (count == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(diag::sqrt_recip_check_kernel, dim3((unsigned)((count + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                     as_stream(stream), first, count, counts);
  return launch_status();
}
