// Shared host-side plumbing: status values, HIP error mapping, device buffers
// and the derived device layout of a quantized weight matrix.
#pragma once

#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <utility>
#include <vector>

namespace wv {

// Status codes of the reference (include/welvet/status.hpp:8-14).
enum Code : int32_t { kOk = 0, kInvalid = 1, kUnsupported = 2, kGap = 3, kInternal = 4 };

struct Status {
  int32_t code = kOk;
  std::string message;
  static Status ok() { return Status{}; }
  static Status err(int32_t c, std::string m) { return Status{c, std::move(m)}; }
  explicit operator bool() const { return code == kOk; }
};

inline Status hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return Status::ok();
  return Status::err(kInternal, std::string(what) + ": " + hipGetErrorString(e));
}

#define WV_TRY(expr)                  \
  do {                                \
    ::wv::Status wv_st_ = (expr);     \
    if (!wv_st_) return wv_st_;       \
  } while (0)

#define WV_HIP(call) WV_TRY(::wv::hip_status((call), #call))

// Activation ids (include/welvet/activate.hpp:8-17).
enum Act : int32_t {
  kLinear = -1, kReLU = 0, kSilu = 1, kGELU = 2, kTanh = 3, kSigmoid = 4, kLeaky = 5, kReLU2 = 6
};
inline bool act_valid(int a) { return a >= -1 && a <= 6; }

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Owning device allocation.
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr, o.bytes = 0; }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      reset();
      p = o.p, bytes = o.bytes;
      o.p = nullptr, o.bytes = 0;
    }
    return *this;
  }
  ~DevBuf() { reset(); }
  void reset() {
    if (p) (void)hipFree(p);
    p = nullptr, bytes = 0;
  }
  Status alloc(size_t n) {
    reset();
    if (n == 0) n = 16;
    WV_HIP(hipMalloc(&p, n));
    bytes = n;
    return Status::ok();
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// Derived device layout of one quantized [rows x cols] weight matrix
// (rows = outputs, cols = inputs). Rows are padded to a multiple of 128 and
// columns to a multiple of 256 elements; padding codes are zero, padding
// scales are 1 (E8M0 byte 127). Codes are stored in canonical form (see
// codec.h), row-major with `pitch` bytes per row; FP4 packs two codes per byte,
// the even column in the low nibble.
struct DeviceWeights {
  int dtype = 0, scheme = 0, rows = 0, cols = 0;
  int rpad = 0, kpad = 0, pitch = 0, nblk = 0;
  DevBuf codes;      // [rpad][pitch]
  DevBuf row_scale;  // float[rpad]
  DevBuf blk;        // uint8[rpad][nblk], BLOCK32 only
  // the same exponents in matrix-core lane order, BLOCK32 only: per 16-row
  // block and group of 4 K chunks of 128, one dword per lane l (row l % 16,
  // block l / 16 of each chunk), byte j = chunk j of the group:
  // uint8[rpad / 16][ceil(kpad / 512)][64][4]
  DevBuf blk_frag;
  // optional copy of the codes in matrix-core operand order for the 5..32-row
  // GEMM (built by sessions whose batch runs it): per 16-row block, K chunk
  // of 128 and operand half (FP8: 2, FP4: 1), lane l's 16 bytes (row l % 16,
  // chunk bytes 64 h + 16 (l / 16) ..) at 16 l, so a wave's operand load is
  // 1 KiB contiguous: uint8[rpad / 16][kpad / 128][halves][64][16]
  DevBuf codes_frag;
  // rows holding non-finite codes (E5M2 only), device and host copies
  DevBuf nf_rows;
  std::vector<int> nf_host;
  int nf_count() const { return (int)nf_host.size(); }
  const uint8_t* d_codes() const { return codes.as<const uint8_t>(); }
  const float* d_scale() const { return row_scale.as<const float>(); }
  const uint8_t* d_blk() const { return scheme == 3 ? blk.as<const uint8_t>() : nullptr; }
  const uint8_t* d_blkf() const { return scheme == 3 ? blk_frag.as<const uint8_t>() : nullptr; }
  const uint8_t* d_codesf() const { return codes_frag.as<const uint8_t>(); }
};

constexpr int kRowPad = 128;
constexpr int kColPad = 256;

}  // namespace wv
