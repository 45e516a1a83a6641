// Error state and library introspection for the C-ABI.
#include <cstdarg>
#include <cstring>

#include "common.h"
#include "../../include/loraforge_amd.h"

namespace lf {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
}

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

int hip_status(hipError_t err, const char* what) {
  return fail(kHip, "%s failed: %s", what, hipGetErrorString(err));
}

}  // namespace lf

extern "C" const char* lf_last_error(void) { return lf::g_error; }

extern "C" int lf_abi_version(void) { return LF_ABI_VERSION; }

extern "C" int lf_device_arch(int device, char* name, int capacity) {
  hipDeviceProp_t prop;
  LF_HIP(hipGetDeviceProperties(&prop, device));
  LF_REQUIRE(name != nullptr && capacity > 0, "name buffer required");
  std::strncpy(name, prop.gcnArchName, capacity - 1);
  name[capacity - 1] = '\0';
  return lf::kOk;
}
