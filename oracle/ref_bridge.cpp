// C bridge over the reference's own host codec and FormatNone store, compiled
// from the reference sources where they lie (see oracle/Makefile). Test
// infrastructure only: used to generate and check golden vectors.
#include "welvet/activate.hpp"
#include "welvet/float_codecs.hpp"
#include "welvet/weights.hpp"

#include <cstring>

extern "C" {

uint8_t ref_enc(int dtype, float f) {
  switch (dtype) {
  case 4: return welvet::float32_to_fp8e4m3(f);
  case 5: return welvet::float32_to_fp8e5m2(f);
  case 16: return welvet::float32_to_fp4(f);
  }
  return 0;
}

float ref_dec(int dtype, uint8_t b) {
  switch (dtype) {
  case 4: return welvet::fp8e4m3_to_float32(b);
  case 5: return welvet::fp8e5m2_to_float32(b);
  case 16: return welvet::fp4_to_float32(b);
  }
  return 0.0f;
}

// Encodes the f32 patterns of 2^20-pattern chunks; same digest definition as
// the oracle's or_sweep_digest.
void ref_sweep_digest(int dtype, uint32_t first_chunk, uint32_t n_chunks, int64_t* out) {
  for (uint32_t c = 0; c < n_chunks; ++c) {
    const uint32_t chunk = first_chunk + c;
    int64_t s1 = 0, s2 = 0;
    for (uint32_t i = 0; i < (1u << 20); ++i) {
      const uint32_t u = (chunk << 20) | i;
      float f;
      std::memcpy(&f, &u, 4);
      const int64_t code = ref_enc(dtype, f);
      s1 += code;
      s2 += code * static_cast<int64_t>(i);
    }
    out[2 * static_cast<size_t>(c)] = s1;
    out[2 * static_cast<size_t>(c) + 1] = s2;
  }
}

// WeightStore::make (store.cpp:7-22) for a rows x cols fp32 matrix; writes the
// native payload (native_cap bytes available), its length, and the store scale.
// Returns the status code.
int ref_store_make(int dtype, int rows, int cols, const float* W, uint8_t* native,
                   size_t native_cap, size_t* native_len, float* scale) {
  welvet::WeightStore s;
  auto st = welvet::WeightStore::make(rows, cols, static_cast<welvet::DType>(dtype), W, &s);
  if (!st) return static_cast<int>(st.code);
  *native_len = s.native.size();
  *scale = s.scale;
  if (s.native.size() > native_cap) return 1;
  std::memcpy(native, s.native.data(), s.native.size());
  return 0;
}

// WeightStore::export_f32 (store.cpp:42-71) of a store built from native bytes.
int ref_store_export(int dtype, int rows, int cols, const uint8_t* native, size_t native_len,
                     float* out) {
  welvet::WeightStore s;
  auto st = welvet::WeightStore::make(rows, cols, static_cast<welvet::DType>(dtype), nullptr, &s);
  if (!st) return static_cast<int>(st.code);
  if (native_len != s.native.size()) return 1;
  std::memcpy(s.native.data(), native, native_len);
  st = s.export_f32(out);
  return static_cast<int>(st.code);
}

// WeightStore::decode_row_f64 (native_codec.cpp:1043-1078).
int ref_store_decode_row(int dtype, int rows, int cols, const uint8_t* native, size_t native_len,
                         int row, double* out) {
  welvet::WeightStore s;
  auto st = welvet::WeightStore::make(rows, cols, static_cast<welvet::DType>(dtype), nullptr, &s);
  if (!st) return static_cast<int>(st.code);
  if (native_len != s.native.size()) return 1;
  std::memcpy(s.native.data(), native, native_len);
  st = s.decode_row_f64(row, out);
  return static_cast<int>(st.code);
}

// activate_f64 / activate_deriv_f64 (src/core/activate.cpp:7-63).
double ref_activate(int act, double x) {
  return welvet::activate_f64(x, static_cast<welvet::Activation>(act));
}
double ref_act_deriv(int act, double x) {
  return welvet::activate_deriv_f64(x, static_cast<welvet::Activation>(act));
}

// WeightStore::apply_sgd (native_codec.cpp:1080-1133) on a store holding the
// native bytes; the updated bytes are written back in place.
int ref_store_apply_sgd(int dtype, int rows, int cols, uint8_t* native, size_t native_len,
                        const double* dW, double lr) {
  welvet::WeightStore s;
  auto st = welvet::WeightStore::make(rows, cols, static_cast<welvet::DType>(dtype), nullptr, &s);
  if (!st) return static_cast<int>(st.code);
  if (native_len != s.native.size()) return 1;
  std::memcpy(s.native.data(), native, native_len);
  st = s.apply_sgd(dW, lr);
  if (!st) return static_cast<int>(st.code);
  std::memcpy(native, s.native.data(), native_len);
  return 0;
}

}  // extern "C"
