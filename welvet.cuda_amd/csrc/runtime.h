// Device runtime (device 0, identity) and an owning stream handle.
#pragma once

#include <string>

#include "common.h"

namespace wv {

Status init_device();
bool device_available();
std::string identity();
int cu_count();

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
