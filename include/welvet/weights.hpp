// Quantized weight storage (reference include/welvet/weights.hpp:12-51).
// A WeightStore holds one [rows][cols] matrix (rows = outputs) as the
// reference's FormatNone payload: `native` is the codes of W row-major, one
// byte per FP8 code or two FP4 codes per byte (even element in the low
// nibble). This library serves FP8E4M3, FP8E5M2 and FP4; quantizing and
// decoding run on the GPU (the calls return Unsupported without a device).
//
// Extension (no counterpart in the reference): a scale scheme. Reference
// stores (scheme Reference) hold the codes of W itself and `scale` 1; scaled
// stores hold the codes of W / s with s per tensor (`scale`, also in every
// row_scale entry), per output row (row_scale) or 2^e per 32 consecutive
// columns (blk_exp, E8M0 bytes e + 127). The dequantized weight is
// decode(code) * s.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "welvet/dtype.hpp"
#include "welvet/export.hpp"
#include "welvet/status.hpp"

namespace welvet {

enum class QuantFormat : int32_t {
  None = 0,
  // the packed block formats are reached through welvet_dense_mount_format
};

enum class ScaleScheme : int32_t {
  Reference = 0,  // unscaled codes of W (the reference's stores)
  PerTensor = 1,  // s = amax / max representable
  PerRow = 2,     // s per output row
  Block32 = 3,    // E8M0 2^e per 32 columns of a row
};

struct WELVET_API WeightStore {
  DType dtype = DType::Float32;
  QuantFormat format = QuantFormat::None;
  int rows = 0;
  int cols = 0;
  std::vector<float> f32;       // Float32 payload: not served by this library (empty)
  std::vector<uint8_t> native;  // the FormatNone codes
  float scale = 1.0f;
  std::vector<double> bias;

  // extension: see the file comment
  ScaleScheme scheme = ScaleScheme::Reference;
  std::vector<float> row_scale;  // [rows]; all 1 for Reference and Block32
  std::vector<uint8_t> blk_exp;  // [rows][ceil(cols / 32)], Block32 only

  // W [rows][cols] (null: zeros) quantized to dt with the reference codec.
  static Status make(int rows, int cols, DType dt, const float* init_or_null, WeightStore* out);
  static Status make_f32(int rows, int cols, const float* init_or_null, WeightStore* out) {
    return make(rows, cols, DType::Float32, init_or_null, out);
  }
  // extension: the same with a scale scheme
  static Status make_scaled(int rows, int cols, DType dt, ScaleScheme scheme,
                            const float* init_or_null, WeightStore* out);

  // Replaces the payload with the codes of scratch[0, n), n = rows * cols
  // (scheme Reference).
  Status encode_format_none(DType dt, const float* scratch, int n);
  // Row `row` dequantized, widened to f64.
  Status decode_row_f64(int row, double* dst) const;
  // The whole matrix dequantized to f32 [rows][cols].
  Status export_f32(float* dst) const;
  // Re-quantizes from rows * cols f32 values, keeping dtype and scheme.
  Status set_from_f32(const std::vector<float>& values);

  // Host products are not served: Unsupported, as in the reference.
  Status matvec_f32(const float* x, float* y) const;
  Status matvect_f32(const float* gy, float* gx) const;

  // w <- quantize(f32(f64(w) - lr * dW)) per element (dequantized w; the
  // reference's SGD element rule), re-quantized with the store's scheme.
  Status apply_sgd(const double* dW, double lr);
  // bias <- bias - lr * dB (no-op without a bias).
  Status apply_bias_sgd(const double* dB, int n, double lr);
};

}  // namespace welvet
