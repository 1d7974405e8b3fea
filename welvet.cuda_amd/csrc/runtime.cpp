// Device runtime: one process-wide GPU (device 0), initialized once under a
// mutex, and its identity string. Mirrors src/cuda/device.cpp:40-92 of the
// reference (init_default_device / available / runtime_identity).
#include "runtime.h"

#include <cstring>
#include <mutex>
#include <sstream>

namespace wv {
namespace {
std::mutex g_mu;
bool g_ready = false;
hipDeviceProp_t g_prop;

// Device name for the identity: the runtime's marketing name, else the
// name hipDeviceGetName reports, else one built from what the properties
// always carry (architecture, compute units, peak engine clock).
std::string device_name() {
  std::string name(g_prop.name, strnlen(g_prop.name, sizeof(g_prop.name)));
  if (name.empty()) {
    char buf[256] = {0};
    if (hipDeviceGetName(buf, sizeof(buf) - 1, 0) == hipSuccess) name = buf;
    else (void)hipGetLastError();
  }
  if (name.empty()) {
    std::string arch(g_prop.gcnArchName);
    arch = arch.substr(0, arch.find(':'));
    std::ostringstream os;
    os << "AMD " << arch << " " << g_prop.multiProcessorCount << "CU "
       << g_prop.clockRate / 1000 << "MHz";
    name = os.str();
  }
  return name;
}

// Pinned staging: two buffers, so the host copy of one chunk overlaps the
// DMA of the other.
constexpr size_t kStageBytes = 8u << 20;
std::mutex g_stage_mu;
void* g_stage[2] = {nullptr, nullptr};
hipEvent_t g_stage_ev[2] = {nullptr, nullptr};

Status stage_ready() {
  for (int i = 0; i < 2; ++i) {
    if (!g_stage[i]) WV_HIP(hipHostMalloc(&g_stage[i], kStageBytes, hipHostMallocDefault));
    if (!g_stage_ev[i])
      WV_HIP(hipEventCreateWithFlags(&g_stage_ev[i], hipEventDisableTiming));
  }
  return Status::ok();
}
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
  os << "hip:" << device_name() << ":idx=0:arch=" << g_prop.gcnArchName
     << ":cu=" << g_prop.multiProcessorCount << ":mem=" << (g_prop.totalGlobalMem >> 20) << "MiB";
  return os.str();
}

int cu_count() {
  if (!init_device()) return 0;
  return g_prop.multiProcessorCount;
}

Status copy_h2d(void* dst, const void* src, size_t n, hipStream_t st) {
  if (n == 0) return Status::ok();
  if (!dst || !src) return Status::err(kInvalid, "copy_h2d: null buffer");
  std::lock_guard<std::mutex> lock(g_stage_mu);
  WV_TRY(stage_ready());
  bool used[2] = {false, false};
  // The next caller refills the buffers, so every DMA queued here must have
  // read its buffer before this returns, on the error paths too. A failed
  // copy or record leaves an earlier event that may still be pending; the
  // whole stream is drained then, since that event no longer marks the last
  // use of its buffer.
  auto fail = [&](Status s) {
    if (hipStreamSynchronize(st) != hipSuccess) (void)hipGetLastError();
    return s;
  };
  int i = 0;
  for (size_t off = 0; off < n; off += kStageBytes, i ^= 1) {
    const size_t len = n - off < kStageBytes ? n - off : kStageBytes;
    // the DMA that last read this buffer must be done before it is refilled
    if (used[i]) {
      Status s = hip_status(hipEventSynchronize(g_stage_ev[i]), "copy_h2d: stage wait");
      if (!s) return fail(s);
    }
    std::memcpy(g_stage[i], static_cast<const char*>(src) + off, len);
    used[i] = true;
    Status s = hip_status(hipMemcpyAsync(static_cast<char*>(dst) + off, g_stage[i], len,
                                         hipMemcpyHostToDevice, st),
                          "copy_h2d: hipMemcpyAsync");
    if (s) s = hip_status(hipEventRecord(g_stage_ev[i], st), "copy_h2d: hipEventRecord");
    if (!s) return fail(s);
  }
  for (int k = 0; k < 2; ++k)
    if (used[k]) {
      Status s = hip_status(hipEventSynchronize(g_stage_ev[k]), "copy_h2d: stage wait");
      if (!s) return fail(s);
    }
  return Status::ok();
}

Status copy_d2h(void* dst, const void* src, size_t n, hipStream_t st) {
  if (n == 0) return Status::ok();
  if (!dst || !src) return Status::err(kInvalid, "copy_d2h: null buffer");
  std::lock_guard<std::mutex> lock(g_stage_mu);
  WV_TRY(stage_ready());
  bool pend[2] = {false, false};
  size_t pend_off[2] = {0, 0}, pend_len[2] = {0, 0};
  // as in copy_h2d: no DMA into a staging buffer may still be running when
  // this returns, on the error paths too
  auto fail = [&](Status s) {
    if (hipStreamSynchronize(st) != hipSuccess) (void)hipGetLastError();
    return s;
  };
  auto drain = [&](int k) -> Status {
    WV_HIP(hipEventSynchronize(g_stage_ev[k]));
    std::memcpy(static_cast<char*>(dst) + pend_off[k], g_stage[k], pend_len[k]);
    pend[k] = false;
    return Status::ok();
  };
  int i = 0;
  for (size_t off = 0; off < n; off += kStageBytes, i ^= 1) {
    const size_t len = n - off < kStageBytes ? n - off : kStageBytes;
    if (pend[i]) {
      Status s = drain(i);
      if (!s) return fail(s);
    }
    Status s = hip_status(hipMemcpyAsync(g_stage[i], static_cast<const char*>(src) + off, len,
                                         hipMemcpyDeviceToHost, st),
                          "copy_d2h: hipMemcpyAsync");
    if (s) s = hip_status(hipEventRecord(g_stage_ev[i], st), "copy_d2h: hipEventRecord");
    if (!s) return fail(s);
    pend[i] = true, pend_off[i] = off, pend_len[i] = len;
  }
  for (int k = 0; k < 2; ++k)
    if (pend[i ^ k]) {
      Status s = drain(i ^ k);
      if (!s) return fail(s);
    }
  return Status::ok();
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
