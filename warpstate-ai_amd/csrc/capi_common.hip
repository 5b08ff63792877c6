// Error reporting, device properties and per-device kernel attributes of the C ABI.
#include <mutex>
#include <string>
#include <vector>

#include "../../include/warpstate_hip.h"
#include "launch.h"

namespace ws {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

static constexpr int kMaxDevices = 64;
static std::mutex g_mu;
static int g_cus[kMaxDevices];

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_cus[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    g_cus[dev] = cus;
  }
  return g_cus[dev];
}

// hipFuncSetAttribute applies to the current device. The limit set for each (kernel,
// device) is remembered and only ever raised: a kernel whose LDS size depends on its
// arguments (the RMSNorm backward's per-wave partial rows of d floats) may come first
// with a small size.
int ensure_lds(const void* kernel, int bytes) {
  struct Limit {
    const void* kernel;
    int dev;
    int bytes;
  };
  static std::mutex mu;
  static std::vector<Limit>* seen = new std::vector<Limit>();
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(kHipError, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(mu);
  Limit* entry = nullptr;
  for (auto& e : *seen)
    if (e.kernel == kernel && e.dev == dev) entry = &e;
  if (entry && entry->bytes >= bytes) return kOk;
  hipError_t err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (err != hipSuccess)
    return set_error(kHipError, "hipFuncSetAttribute(%d bytes LDS): %s", bytes, hipGetErrorString(err));
  if (entry)
    entry->bytes = bytes;
  else
    seen->push_back({kernel, dev, bytes});
  return kOk;
}

}  // namespace ws

extern "C" const char* ws_last_error(void) { return ws::g_last_error.c_str(); }

extern "C" const char* ws_version(void) { return "warpstate-hip 0.1 gfx950"; }
