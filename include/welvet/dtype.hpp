// Storage types (reference include/welvet/dtype.hpp:9-46): the ids the C ABI's
// `dtype` argument and the WMN1 store payloads carry. This library serves the
// quantized path: FP8E4M3 (4), FP8E5M2 (5) and FP4 (16); every other id is
// reported as Unsupported by the calls that take a dtype.
#pragma once

#include <cstdint>
#include <string_view>

#include "welvet/export.hpp"

namespace welvet {

enum class DType : int32_t {
  Float64 = 0,
  Float32 = 1,
  Float16 = 2,
  BFloat16 = 3,
  FP8E4M3 = 4,
  FP8E5M2 = 5,
  Int64 = 6,
  Int32 = 7,
  Int16 = 8,
  Int8 = 9,
  Uint64 = 10,
  Uint32 = 11,
  Uint16 = 12,
  Uint8 = 13,
  Int4 = 14,
  Uint4 = 15,
  FP4 = 16,
  Int2 = 17,
  Uint2 = 18,
  Ternary = 19,
  Binary = 20,
  Int = 21,
  Uint = 22,
  Uintptr = 23,
  Complex64 = 24,
  Complex128 = 25,
  NF4 = 26,
  FP6 = 27,
  Int6 = 28,
  Uint6 = 29,
  Int5 = 30,
  Uint5 = 31,
  Int3 = 32,
  Uint3 = 33,
};

constexpr int kNumDTypes = 34;

// Lower-case name of a dtype ("fp8e4m3", "fp4", ...); "unknown" outside 0-33.
WELVET_API std::string_view dtype_name(DType dt);
// True for the dtypes whose Dense forward this library runs (4, 5 and 16).
WELVET_API bool dtype_implemented_forward(DType dt);

}  // namespace welvet
