// Device runtime (device 0, identity) and an owning stream handle.
#pragma once

#include <string>

#include "common.h"

namespace wv {

Status init_device();
bool device_available();
std::string identity();
int cu_count();

// Copies between pageable host memory and device memory through pinned
// staging buffers the library allocates once (hipHostMalloc). The runtime
// is never handed a pageable buffer, so it never pins the caller's pages in
// place for a large transfer (host memory registration is refused on some
// systems, and the failed pin surfaces in a later call).
// copy_h2d returns once `src` has been read; the device writes are ordered
// on `st`. copy_d2h returns once `dst` holds the data (work queued on `st`
// before it is complete). Calls from different threads serialize.
Status copy_h2d(void* dst, const void* src, size_t n, hipStream_t st);
Status copy_d2h(void* dst, const void* src, size_t n, hipStream_t st);

// Owning HIP stream at the default priority.
struct Stream {
  hipStream_t s = nullptr;
  Stream() = default;
  Stream(const Stream&) = delete;
  Stream& operator=(const Stream&) = delete;
  ~Stream();
  Status create();
};

}  // namespace wv
