// Result of every C++ API call: a code and a message, the C ABI's
// welvet_status in C++ form. Same codes and meaning as the reference's
// welvet::Status (reference include/welvet/status.hpp:8-30).
#pragma once

#include <string>
#include <string_view>

namespace welvet {

enum class StatusCode {
  Ok = 0,
  InvalidArgument = 1,  // a shape, pointer or argument the call cannot accept
  Unsupported = 2,      // outside what this library serves (no device, another dtype)
  Gap = 3,              // an entry point of the reference that is not on this path
  Internal = 4,         // a runtime or device failure
};

struct Status {
  StatusCode code = StatusCode::Ok;
  std::string message;

  static Status Ok() { return Status{}; }
  static Status Err(StatusCode c, std::string_view msg) { return Status{c, std::string(msg)}; }
  // A gap carries the "gap? " prefix callers search for.
  static Status Gap(std::string_view what) {
    return Status{StatusCode::Gap, "gap? " + std::string(what)};
  }

  bool ok() const { return code == StatusCode::Ok; }
  explicit operator bool() const { return ok(); }
};

}  // namespace welvet
