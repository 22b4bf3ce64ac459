// Library-wide C-ABI pieces: version string and the per-thread last HIP error.
#include "hipenvs_device.h"

namespace hipenvs {
namespace {
thread_local int g_last_hip_error = 0;
}
void set_last_hip_error(int err) { g_last_hip_error = err; }
}  // namespace hipenvs

extern "C" const char* hipenvs_version(void) { return "hipenvs 0.1 gfx950 fp-contract=off"; }

extern "C" int hipenvs_last_hip_error(void) { return hipenvs::g_last_hip_error; }
