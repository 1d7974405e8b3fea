// Host tensor of the C++ API (reference include/welvet/tensor.hpp:9-15):
// a shape and row-major fp32 data.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "welvet/export.hpp"

namespace welvet {

struct WELVET_API TensorF32 {
  std::vector<int64_t> shape;
  std::vector<float> data;

  // A [a, b] tensor of zeros.
  static TensorF32 zeros(int64_t a, int64_t b);
  std::size_t numel() const { return data.size(); }
};

}  // namespace welvet
