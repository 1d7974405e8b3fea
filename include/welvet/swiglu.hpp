// SwiGLU feed-forward (reference include/welvet/swiglu.hpp:10-53): pre = h =
// SiLU(Gate x) * Up x with the reference's f32 / f64 rounding, post = Down h.
// Gate and Up run as one fused product on the GPU.
#pragma once

#include "welvet/dense.hpp"
#include "welvet/device_state.hpp"
#include "welvet/dtype.hpp"
#include "welvet/export.hpp"
#include "welvet/status.hpp"
#include "welvet/tensor.hpp"

namespace welvet::swiglu {

struct Config {
  int input_dim = 0;
  int intermediate_dim = 0;
};

WELVET_API Status validate(const Config& cfg);

// intermediate = 8/3 d_model rounded up to a multiple of 8 (2 d_model when
// that is smaller than d_model).
WELVET_API Config default_ffn(int d_model);

struct WELVET_API Layer {
  Config cfg{};
  dense::Layer Gate, Up, Down;
  // the layer's stream, workspace and activation buffers on the device
  mutable DeviceHandle gpu;
};

WELVET_API Status new_configured(const Config& cfg, DType dt, const float* gate_init,
                                 const float* up_init, const float* down_init, Layer* out);

// input [batch, in] or [batch, seq, in]; pre = h, post = Down h.
WELVET_API Status forward(Layer& layer, const TensorF32& input, TensorF32* pre, TensorF32* post);

// NormalBP: grad_w = [dGate | dUp | dDown]; pre must be the forward's h.
WELVET_API Status backward_f32(Layer& layer, const TensorF32& grad_out, const TensorF32& input,
                               const TensorF32& pre, TensorF32* grad_in, TensorF32* grad_w);

// SGD with the concatenated dW (Gate, Up, Down).
WELVET_API Status apply_grad_sgd(Layer* layer, const TensorF32& dW, double lr);

WELVET_API int grad_w_size(const Layer& layer);
WELVET_API Status export_weights_f32(const Layer& layer, float* dst);

}  // namespace welvet::swiglu
