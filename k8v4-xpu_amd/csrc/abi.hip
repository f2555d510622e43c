// Error reporting and version entry points of the C ABI.
#include "k8v4_common.h"

namespace k8v4 {

static thread_local std::string g_last_error;

void set_error(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int launch_status(const char *what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(err));
    return K8V4_ERR_HIP;
  }
  return K8V4_OK;
}

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

}  // namespace k8v4

extern "C" int k8v4_abi_version(void) { return K8V4_ABI_VERSION; }

extern "C" const char *k8v4_last_error(void) { return k8v4::g_last_error.c_str(); }
