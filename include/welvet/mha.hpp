// Multi-head attention layer (reference include/welvet/mha.hpp:10-108): Q, K,
// V projections on [batch * seq, d_model], the attention core with the
// reference's global positions and KV ring, the O projection. pre = the
// attention output [batch, seq, q_dim], post = O(pre) [batch, seq, d_model].
#pragma once

#include <cstdint>

#include "welvet/dense.hpp"
#include "welvet/device_state.hpp"
#include "welvet/dtype.hpp"
#include "welvet/export.hpp"
#include "welvet/status.hpp"
#include "welvet/tensor.hpp"

namespace welvet::mha {

// Kind values are those of the WMN1 wire and the C ABI.
enum class MaskKind : int32_t {
  Unspecified = 0,
  Causal = 1,
  Bidirectional = 2,
  SlidingWindow = 3,
  PrefixLM = 4,
  Custom = 5,
};

enum class PosKind : int32_t {
  RoPE = 0,
  None = 1,
  ALiBi = 2,
  RoPEALiBi = 3,
};

enum class AttnMode : int32_t {
  Self = 0,
  Cross = 1,
};

enum class SoftmaxKind : int32_t {
  Standard = 0,
  Sigmoid = 1,
};

struct WELVET_API Config {
  int d_model = 0;
  int num_heads = 0;
  int num_kv_heads = 0;  // 0: num_heads
  int head_dim = 0;      // 0: d_model / num_heads
  int max_seq_len = 0;   // 0: 512

  MaskKind mask = MaskKind::Causal;
  PosKind pos = PosKind::RoPE;
  AttnMode mode = AttnMode::Self;
  SoftmaxKind softmax = SoftmaxKind::Standard;

  bool causal = true;
  int window = 0;
  bool window_causal = true;
  int prefix_len = 0;
  double rope_theta = 10000.0;
  double scale_override = 0.0;

  int q_dim() const { return num_heads * head_dim; }
  int kv_dim() const { return num_kv_heads * head_dim; }
  int heads_per_kv() const { return num_heads / num_kv_heads; }
  // scale_override when positive, else 1 / sqrt(head_dim)
  double scale() const;
  bool uses_rope() const { return pos == PosKind::RoPE || pos == PosKind::RoPEALiBi; }
  bool uses_alibi() const { return pos == PosKind::ALiBi || pos == PosKind::RoPEALiBi; }
};

// Fills the defaults above and checks the head counts.
WELVET_API Status validate(Config* cfg);

WELVET_API Config decoder_causal(int d_model, int num_heads, int num_kv_heads);

struct WELVET_API Layer {
  Config cfg{};
  dense::Layer Q, K, V, O;
  // the layer's stream, workspace and activation buffers on the device
  mutable DeviceHandle gpu;
};

WELVET_API Status new_configured(const Config& cfg, DType dt, const float* q_init,
                                 const float* k_init, const float* v_init, const float* o_init,
                                 Layer* out);

// Self-attention forward; input [batch, seq, d_model] or [seq, d_model].
WELVET_API Status forward(Layer& layer, const TensorF32& input, TensorF32* pre, TensorF32* post);

// Length of the concatenated Q | K | V | O weight gradient.
WELVET_API int grad_w_size(const Layer& layer);

// The attention backward is not part of this library: Gap.
WELVET_API Status backward_f32(const Layer& layer, const TensorF32& grad_out,
                               const TensorF32& input, const TensorF32& pre, TensorF32* grad_in,
                               TensorF32* grad_w);

// SGD with the concatenated dW (Q, K, V, O).
WELVET_API Status apply_grad_sgd(Layer* layer, const TensorF32& dW, double lr);

// Q | K | V | O dequantized into dst (length grad_w_size).
WELVET_API Status export_weights_f32(const Layer& layer, float* dst);

}  // namespace welvet::mha
