// Device runtime: one process-wide GPU (device 0), initialized once under a
// mutex, and its identity string. Mirrors src/cuda/device.cpp:40-92 of the
// reference (init_default_device / available / runtime_identity).
#include "runtime.h"

#include <mutex>
#include <sstream>

namespace wv {
namespace {
std::mutex g_mu;
bool g_ready = false;
hipDeviceProp_t g_prop;
}  // namespace

Status init_device() {
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_ready) return hip_status(hipSetDevice(0), "hipSetDevice");
  int n = 0;
  const hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return Status::err(kUnsupported, "no HIP device visible");
  }
  WV_HIP(hipSetDevice(0));
  WV_HIP(hipGetDeviceProperties(&g_prop, 0));
  g_ready = true;
  return Status::ok();
}

bool device_available() {
  int n = 0;
  const hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) (void)hipGetLastError();
  return e == hipSuccess && n > 0;
}

std::string identity() {
  if (!init_device()) return "hip:unavailable";
  std::lock_guard<std::mutex> lock(g_mu);
  std::ostringstream os;
  os << "hip:" << g_prop.name << ":idx=0:arch=" << g_prop.gcnArchName
     << ":cu=" << g_prop.multiProcessorCount << ":mem=" << (g_prop.totalGlobalMem >> 20) << "MiB";
  return os.str();
}

int cu_count() {
  if (!init_device()) return 0;
  return g_prop.multiProcessorCount;
}

Status Stream::create() {
  if (s) return Status::ok();
  WV_TRY(init_device());
  WV_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  return Status::ok();
}

Stream::~Stream() {
  if (s) (void)hipStreamDestroy(s);
}

}  // namespace wv
