// Library set-up entry points and the thread-local error slot.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "common.h"

namespace th {

static thread_local std::string g_last_error;
static std::mutex g_init_mutex;
static bool g_ready[64];
static int g_cus[64];

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

bool device_ready() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  return g_ready[dev];
}

int device_cus() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  return g_cus[dev];
}

}  // namespace th

extern "C" int th_abi_version(void) { return TH_ABI_VERSION; }

extern "C" const char* th_last_error(void) { return th::g_last_error.c_str(); }

extern "C" int th_init(int device) {
  if (device < 0 || device >= 64) {
    th::set_error("th_init: device %d out of range", device);
    return TH_ERR_INVALID;
  }
  std::lock_guard<std::mutex> lock(th::g_init_mutex);
  TH_CHECK_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  TH_CHECK_HIP(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    th::set_error("th_init: device %d is %s; this library is built for gfx950 only", device,
                  prop.gcnArchName);
    return TH_ERR_UNSUPPORTED;
  }
  int st = th::ssd_init_device();
  if (st != TH_OK) return st;
  st = th::fp8_scratch_init_device(device);
  if (st != TH_OK) return st;
  th::g_cus[device] = prop.multiProcessorCount;
  th::g_ready[device] = true;
  th::g_last_error.clear();
  return TH_OK;
}
