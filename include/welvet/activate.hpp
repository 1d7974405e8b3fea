// Activation ids of the Dense epilogue (reference include/welvet/activate.hpp:
// 8-21). The kernels evaluate them in f64 on the device; the two host
// functions give the same formulas for callers that need a scalar.
#pragma once

#include <cstdint>

#include "welvet/export.hpp"

namespace welvet {

enum class Activation : int32_t {
  Linear = -1,
  ReLU = 0,
  Silu = 1,
  GELU = 2,
  Tanh = 3,
  Sigmoid = 4,
  LeakyReLU = 5,
  ReLU2 = 6,
};

WELVET_API double activate_f64(double x, Activation act);
WELVET_API double activate_deriv_f64(double x, Activation act);

}  // namespace welvet
