// Dense epilogue activations in f64, as the reference's device epilogue
// computes them (src/cuda/kernels.cu:22-46 activate_dev; host twin
// src/layers/activate.cpp:7-29): ids from src/layers/activate.hpp:8-17.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace wv {

__device__ __forceinline__ double act_f64(int act, double x) {
  switch (act) {
  case kReLU: return x < 0.0 ? 0.0 : x;
  case kSilu: return x / (1.0 + exp(-x));
  case kGELU: {
    const double k = 0.7978845608028654;
    return 0.5 * x * (1.0 + tanh(k * (x + 0.044715 * x * x * x)));
  }
  case kTanh: return tanh(x);
  case kSigmoid: return 1.0 / (1.0 + exp(-x));
  case kLeaky: return x < 0.0 ? 0.01 * x : x;
  case kReLU2: return x < 0.0 ? 0.0 : x * x;
  default: return x;
  }
}

}  // namespace wv
