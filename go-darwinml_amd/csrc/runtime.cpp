// Error plumbing and device information for the C ABI.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"

namespace ghip {

int set_error(GHipError* err, int code, const char* fmt, ...) {
  if (err) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (err->message) free(const_cast<char*>(err->message));
    err->code = code;
    err->message = strdup(buf);
  }
  return code;
}

int check_hip(hipError_t e, GHipError* err, const char* what) {
  return set_error(err, GHIP_ERR_HIP, "%s: HIP error %d (%s)", what, static_cast<int>(e),
                   hipGetErrorString(e));
}

}  // namespace ghip

extern "C" void ghip_error_clear(GHipError* err) {
  if (!err) return;
  if (err->message) free(const_cast<char*>(err->message));
  err->message = nullptr;
  err->code = 0;
}

extern "C" const char* ghip_version(void) { return "gomlx-hip 0.1.0 (gfx950)"; }

extern "C" int ghip_device_name(int device, char* buf, size_t buflen, GHipError* err) {
  if (!buf || buflen == 0) return ghip::set_error(err, GHIP_ERR_INVALID_ARG, "device_name: empty buffer");
  hipDeviceProp_t prop;
  GHIP_CHECK(hipGetDeviceProperties(&prop, device), err);
  snprintf(buf, buflen, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
  return GHIP_OK;
}
