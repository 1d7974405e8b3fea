// Device state the library keeps for a layer between calls: the quantized
// weights resident in HBM, the layer's HIP stream, its workspace and the
// device copies of its inputs and outputs. Opaque to callers; a layer owns
// one through DeviceHandle and releases it when destroyed. This takes the
// place of the reference's cuda::ResidentDense member
// (reference include/welvet/cuda/matvec.hpp:14-25).
#pragma once

#include "welvet/export.hpp"

namespace welvet {

struct DeviceState;
WELVET_API void release_device_state(DeviceState* s);

// Move-only owner of one DeviceState.
class DeviceHandle {
 public:
  DeviceHandle() = default;
  DeviceHandle(const DeviceHandle&) = delete;
  DeviceHandle& operator=(const DeviceHandle&) = delete;
  DeviceHandle(DeviceHandle&& o) noexcept : p_(o.p_) { o.p_ = nullptr; }
  DeviceHandle& operator=(DeviceHandle&& o) noexcept {
    if (this != &o) {
      reset();
      p_ = o.p_;
      o.p_ = nullptr;
    }
    return *this;
  }
  ~DeviceHandle() { reset(); }

  DeviceState* get() const { return p_; }
  void reset(DeviceState* p = nullptr) {
    if (p_) release_device_state(p_);
    p_ = p;
  }

 private:
  DeviceState* p_ = nullptr;
};

}  // namespace welvet
