// Dense layer over quantized weights (reference include/welvet/dense.hpp:
// 13-59): y = W x with W [output_height][input_height] in `weights`, then
// bias and activation as the reference's f64 epilogue. The first forward at a
// batch size (and the first after invalidate_gpu) puts the weights on the
// GPU; later calls reuse them. Every call runs the HIP kernels of this
// library; without a device they return Unsupported.
#pragma once

#include "welvet/activate.hpp"
#include "welvet/device_state.hpp"
#include "welvet/dtype.hpp"
#include "welvet/export.hpp"
#include "welvet/status.hpp"
#include "welvet/tensor.hpp"
#include "welvet/weights.hpp"

namespace welvet::dense {

struct WELVET_API Layer {
  int input_height = 0;
  int output_height = 0;
  Activation activation = Activation::Linear;
  WeightStore weights;

  // the device copy of `weights` and the layer's buffers; valid while
  // gpu_valid, sized for gpu_batch rows
  mutable DeviceHandle gpu;
  mutable bool gpu_valid = false;
  mutable int gpu_batch = -1;

  Layer() = default;
  Layer(const Layer&) = delete;
  Layer& operator=(const Layer&) = delete;
  Layer(Layer&& o) noexcept
      : input_height(o.input_height),
        output_height(o.output_height),
        activation(o.activation),
        weights(std::move(o.weights)),
        gpu(std::move(o.gpu)),
        gpu_valid(o.gpu_valid),
        gpu_batch(o.gpu_batch) {
    o.gpu_valid = false;
    o.gpu_batch = -1;
  }
  Layer& operator=(Layer&& o) noexcept {
    if (this != &o) {
      input_height = o.input_height;
      output_height = o.output_height;
      activation = o.activation;
      weights = std::move(o.weights);
      gpu = std::move(o.gpu);
      gpu_valid = o.gpu_valid;
      gpu_batch = o.gpu_batch;
      o.gpu_valid = false;
      o.gpu_batch = -1;
    }
    return *this;
  }
  ~Layer() = default;

  // Call after changing `weights`: the next call re-uploads them.
  void invalidate_gpu() const { gpu_valid = false; }
};

// W [out_h][in_h] (null: zeros) quantized to dt with the reference codec.
WELVET_API Status new_layer(int in_h, int out_h, Activation act, DType dt,
                            const float* init_or_null, Layer* layer);
// extension: the same with a scale scheme
WELVET_API Status new_layer_scaled(int in_h, int out_h, Activation act, DType dt,
                                   ScaleScheme scheme, const float* init_or_null, Layer* layer);

// True for the dtypes this library's Dense forward runs (4, 5, 16).
WELVET_API bool dtype_supported_cuda_forward(DType dt);

// input [batch, in] -> pre, post [batch, out].
WELVET_API Status forward_f32(const Layer& layer, const TensorF32& input, TensorF32* pre,
                              TensorF32* post);

// NormalBP backward over the quantized weights: grad_in [batch, in] and
// grad_w [out, in] from grad_out [batch, out], the forward's input and pre.
WELVET_API Status backward_f32(const Layer& layer, const TensorF32& grad_out,
                               const TensorF32& input, const TensorF32& pre, TensorF32* grad_in,
                               TensorF32* grad_w);

// gx = W^T gy with no activation derivative; gy is resized to batch * out
// by averaging ranges when its length differs.
WELVET_API Status linear_grad_in(const Layer& layer, const TensorF32& gy, const TensorF32& input,
                                 TensorF32* gx);

// dW alone (gy resized as above; pre of the wrong size is taken as zeros).
WELVET_API Status grad_w_only(const Layer& layer, const TensorF32& gy, const TensorF32& input,
                              const TensorF32& pre, TensorF32* dw);

// W <- W - lr * dW on the quantized store (re-quantized); the device copy is
// refreshed with it.
WELVET_API Status apply_grad_sgd(Layer* layer, const TensorF32& dW, double lr);

// Puts `weights` on the GPU for `batch` rows.
WELVET_API Status sync_gpu_from_weights(const Layer& layer, int batch);

}  // namespace welvet::dense
