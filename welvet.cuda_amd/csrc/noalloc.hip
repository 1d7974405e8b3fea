// Dense execute that allocates nothing (welvet_dense_execute_noalloc).
//
// For callers that cannot call the allocator: code under HIP graph capture,
// tight serving loops, harnesses that forbid allocation. The rows x in
// activation split and the K-split partial sums that the matrix-core paths
// (more than 4 rows) keep in scratch memory come from `scratch`, a
// file-scope device array of kScratchBytes, instead of the session's
// workspace. Each device holds its own copy of the array until the process
// ends; host code reaches it only through the address hipGetSymbolAddress
// returns on that device (kept per device; the array's name on the host is
// a host-side stand-in, not a device address).
//
// Every call on one device shares that device's array and finds the previous
// call's contents in it. Nothing in it needs to start at zero: the split
// kernels write every byte of the terms they cover, and every K split writes
// the partial sums of all output rows and columns that the reduce reads.
// Calls that overlap on one device (different streams, or host threads
// without ordering) race on the array.
#include <mutex>
#include <new>
#include <string>

#include "common.h"
#include "layers.h"
#include "sessions.h"

namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;  // 64 MiB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device with that device current.
wv::Status scratch_on_current_device(void** out) {
  int dev = -1;
  WV_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return wv::Status::err(wv::kInternal, "noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      return wv::hip_status(e == hipSuccess ? hipErrorInvalidSymbol : e,
                            "hipGetSymbolAddress(scratch)");
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return wv::Status::ok();
}

// Lends the scratch array to a Workspace's split buffer for one call. The
// buffer is handed back (pointer cleared) when the guard leaves scope, on
// every path including unwinding, so ~DevBuf never frees the array.
struct ScratchLoan {
  wv::DevBuf* buf;
  ScratchLoan(wv::DevBuf* b, void* p, size_t bytes) : buf(b) {
    buf->p = p;
    buf->bytes = bytes;
  }
  ~ScratchLoan() {
    buf->p = nullptr;
    buf->bytes = 0;
  }
  ScratchLoan(const ScratchLoan&) = delete;
  ScratchLoan& operator=(const ScratchLoan&) = delete;
};

welvet_status status_out(const wv::Status& st) {
  welvet_status out{};
  out.code = st.code;
  const size_t n = st.message.size() < sizeof(out.message) - 1 ? st.message.size()
                                                                  : sizeof(out.message) - 1;
  st.message.copy(out.message, n);
  out.message[n] = '\0';
  return out;
}

}  // namespace

extern "C" welvet_status welvet_dense_execute_noalloc(welvet_dense_session* s, int32_t rows,
                                                      const float* x, float* pre, float* post,
                                                      void* stream) {
  if (!s || !x || !pre || !post)
    return status_out(wv::Status::err(wv::kInvalid, "noalloc: null execute args"));
  if (rows <= 0) return status_out(wv::Status::err(wv::kInvalid, "noalloc: rows must be > 0"));
  if (pre == post && s->layer.need_epi())
    return status_out(wv::Status::err(wv::kInvalid, "noalloc: pre and post must differ"));
  try {
    const size_t need = wv::dense_workspace_bytes(s->layer, rows);
    if (need > kScratchBytes)
      return status_out(wv::Status::err(
          wv::kInvalid, "noalloc: " + std::to_string(rows) + " rows of " +
                            std::to_string(s->layer.in) + " inputs need " + std::to_string(need) +
                            " bytes of scratch; the fixed scratch holds " +
                            std::to_string(kScratchBytes)));
    void* p = nullptr;
    if (need > 0) {
      wv::Status st = scratch_on_current_device(&p);
      if (!st) return status_out(st);
    }
    wv::Workspace ws;  // its split buffer is the scratch array, on loan
    ScratchLoan loan(&ws.b, p, p ? kScratchBytes : 0);
    hipStream_t st = stream ? static_cast<hipStream_t>(stream) : s->stream.s;
    return status_out(wv::dense_forward(s->layer, rows, x, pre, post, &ws, st));
  } catch (const std::bad_alloc&) {
    return status_out(wv::Status::err(wv::kInternal, "out of host memory"));
  } catch (...) {
    return status_out(wv::Status::err(wv::kInternal, "unknown native failure"));
  }
}
