// Library-wide C-ABI pieces: version string and the per-thread last HIP error.
#include "hipenvs_device.h"

namespace hipenvs {
namespace {
thread_local int g_last_hip_error = 0;
std::atomic<int> g_cus[kMaxDevices];  // 0 until the device's CU count has been queried
}  // namespace
void set_last_hip_error(int err) { g_last_hip_error = err; }

int current_device(int* dev) {
  const hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) {
    set_last_hip_error((int)e);
    return HIPENVS_E_HIP;
  }
  return (*dev >= 0 && *dev < kMaxDevices) ? HIPENVS_OK : HIPENVS_E_ARG;
}

int device_cus(int* cus) {
  int dev = 0;
  const int status = current_device(&dev);
  if (status != HIPENVS_OK) return status;
  int n = g_cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    const hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || n <= 0) {
      set_last_hip_error((int)(e != hipSuccess ? e : hipErrorInvalidDevice));
      return HIPENVS_E_HIP;
    }
    g_cus[dev].store(n, std::memory_order_relaxed);  // every thread that races here stores the same value
  }
  *cus = n;
  return HIPENVS_OK;
}
}  // namespace hipenvs

extern "C" const char* hipenvs_version(void) { return "hipenvs 0.1 gfx950 fp-contract=off"; }

extern "C" int hipenvs_last_hip_error(void) { return hipenvs::g_last_hip_error; }
