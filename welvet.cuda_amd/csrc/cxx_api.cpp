// C++ layer/weights API of the quantized Dense path (include/welvet/*.hpp):
// the reference's welvet::WeightStore, dense::, dense session, swiglu:: and
// mha:: entry points (reference include/welvet/weights.hpp:18-51,
// dense.hpp:13-59, dense_session.hpp:12-19, swiglu.hpp:10-53, mha.hpp:10-108)
// over the same device layers as the C ABI. Quantizing, decoding and every
// product run on the GPU; without a device the calls return Unsupported.
//
// Device state: a dense::Layer keeps its weights on the device in a
// DeviceState (the wv::DenseLayer the kernels read) from its first forward
// until invalidate_gpu(). SwiGLU and MHA layers lend their parts' device
// weights to one fused layer object for the duration of a call (moved in,
// moved back on every exit), so a part synced once serves both the part's own
// Dense calls and the fused layer.
#include <cmath>
#include <cstring>
#include <exception>
#include <new>
#include <string>
#include <utility>
#include <vector>

#include "welvet/dense.hpp"
#include "welvet/dense_session.hpp"
#include "welvet/mha.hpp"
#include "welvet/swiglu.hpp"
#include "welvet_c.h"

#include "layers.h"
#include "runtime.h"
#include "sessions.h"

namespace welvet {

struct DeviceState {
  wv::Stream stream;
  wv::DenseLayer dense;  // dense layers: the device copy of the weights
  wv::Workspace ws;
  int64_t rows = 0;      // rows the activation buffers below are sized for
  wv::DevBuf x, pre, post, aux;
};

void release_device_state(DeviceState* s) { delete s; }

namespace {

Status from_wv(const wv::Status& s) {
  if (s) return Status::Ok();
  return Status::Err(static_cast<StatusCode>(s.code), s.message);
}

Status with_prefix(const Status& s, const char* prefix) {
  if (s) return s;
  return Status::Err(s.code, std::string(prefix) + s.message);
}

template <class F>
Status guarded(F&& fn) {
  try {
    return fn();
  } catch (const std::bad_alloc&) {
    return Status::Err(StatusCode::Internal, "out of host memory");
  } catch (const std::exception& e) {
    return Status::Err(StatusCode::Internal, e.what());
  } catch (...) {
    return Status::Err(StatusCode::Internal, "unknown native failure");
  }
}

#define CX_TRY(expr)                        \
  do {                                      \
    const ::welvet::Status cx_st_ = (expr); \
    if (!cx_st_) return cx_st_;             \
  } while (0)
#define CX_WV(expr) CX_TRY(from_wv(expr))

bool served(DType dt) {
  return dt == DType::FP8E4M3 || dt == DType::FP8E5M2 || dt == DType::FP4;
}

Status unserved(const char* who, DType dt) {
  return Status::Err(StatusCode::Unsupported,
                     std::string(who) + ": dtype " + std::string(dtype_name(dt)) +
                         " is outside the FP8/FP4 path of this library (fp8e4m3, fp8e5m2, fp4)");
}

int64_t elems(const WeightStore& s) { return static_cast<int64_t>(s.rows) * s.cols; }

wv::StoreView view_of(const WeightStore& s) {
  wv::StoreView v;
  v.dtype = static_cast<int>(s.dtype);
  v.scheme = static_cast<int>(s.scheme);
  v.rows = s.rows;
  v.cols = s.cols;
  v.native = s.native.data();
  v.native_len = s.native.size();
  v.row_scale = s.row_scale.data();
  v.row_scale_len = s.row_scale.size();
  v.blk_exp = s.blk_exp.data();
  v.blk_exp_len = s.blk_exp.size();
  return v;
}

wv::WeightStore to_wv(const WeightStore& s) {
  wv::WeightStore w;
  w.dtype = static_cast<int>(s.dtype);
  w.scheme = static_cast<int>(s.scheme);
  w.rows = s.rows;
  w.cols = s.cols;
  w.native = s.native;
  w.scale = s.scale;
  w.row_scale = s.row_scale;
  w.blk_exp = s.blk_exp;
  w.bias = s.bias;
  return w;
}

// The codes and scales of a library store into an API store (bias kept).
void take_codes(wv::WeightStore&& w, WeightStore* s) {
  s->dtype = static_cast<DType>(w.dtype);
  s->format = QuantFormat::None;
  s->rows = w.rows;
  s->cols = w.cols;
  s->f32.clear();
  s->native = std::move(w.native);
  s->scale = w.scale;
  s->scheme = static_cast<ScaleScheme>(w.scheme);
  s->row_scale = std::move(w.row_scale);
  s->blk_exp = std::move(w.blk_exp);
}

// Quantizes W [rows][cols] on the device into s (codes and scales).
Status quantize_into(int rows, int cols, DType dt, ScaleScheme scheme, const float* W,
                     WeightStore* s) {
  if (!served(dt)) return unserved("weights", dt);
  const int sc = static_cast<int>(scheme);
  if (sc < 0 || sc > 3) return Status::Err(StatusCode::InvalidArgument, "weights: scale scheme 0..3");
  CX_WV(wv::init_device());
  wv::WeightStore w;
  CX_WV(wv::store_quantize(rows, cols, static_cast<int>(dt), sc, W, &w, nullptr));
  take_codes(std::move(w), s);
  return Status::Ok();
}

// Grows a device buffer to at least n bytes.
wv::Status fit(wv::DevBuf* b, size_t n) {
  if (b->bytes >= n && b->p) return wv::Status::ok();
  return b->alloc(n);
}

DeviceState* state_of(const DeviceHandle& h) {
  if (!h.get()) const_cast<DeviceHandle&>(h).reset(new DeviceState());
  return h.get();
}

// The layer's weights on the device (built when not valid).
Status ensure_weights(const dense::Layer& layer) {
  if (!served(layer.weights.dtype)) return unserved("dense", layer.weights.dtype);
  if (layer.weights.format != QuantFormat::None) return Status::Gap("dense over packed formats");
  if (layer.weights.rows != layer.output_height || layer.weights.cols != layer.input_height)
    return Status::Err(StatusCode::InvalidArgument, "dense: weights are not [out][in]");
  DeviceState* d = state_of(layer.gpu);
  if (layer.gpu_valid) return Status::Ok();
  CX_WV(d->stream.create());
  wv::DenseLayer fresh;
  CX_WV(wv::dense_build_from_store(layer.input_height, layer.output_height,
                                   static_cast<int>(layer.activation), to_wv(layer.weights), &fresh,
                                   d->stream.s));
  d->dense = std::move(fresh);
  layer.gpu_valid = true;
  layer.gpu_batch = -1;
  return Status::Ok();
}

}  // namespace

// ------------------------------------------------------------------ types --
TensorF32 TensorF32::zeros(int64_t a, int64_t b) {
  TensorF32 t;
  t.shape = {a, b};
  t.data.assign(static_cast<size_t>(a * b), 0.0f);
  return t;
}

std::string_view dtype_name(DType dt) {
  static const char* const kNames[kNumDTypes] = {
      "float64", "float32", "float16", "bfloat16", "fp8e4m3", "fp8e5m2", "int64",
      "int32",   "int16",   "int8",    "uint64",   "uint32",  "uint16",  "uint8",
      "int4",    "uint4",   "fp4",     "int2",     "uint2",   "ternary", "binary",
      "int",     "uint",    "uintptr", "complex64", "complex128", "nf4", "fp6",
      "int6",    "uint6",   "int5",    "uint5",    "int3",    "uint3"};
  const int id = static_cast<int>(dt);
  return (id >= 0 && id < kNumDTypes) ? kNames[id] : "unknown";
}

bool dtype_implemented_forward(DType dt) { return served(dt); }

// Host twins of the device epilogue (act.h) and of the backward's act'.
double activate_f64(double x, Activation act) {
  switch (act) {
  case Activation::ReLU: return x < 0.0 ? 0.0 : x;
  case Activation::Silu: return x / (1.0 + std::exp(-x));
  case Activation::GELU: {
    const double k = 0.7978845608028654;  // sqrt(2 / pi)
    return 0.5 * x * (1.0 + std::tanh(k * (x + 0.044715 * x * x * x)));
  }
  case Activation::Tanh: return std::tanh(x);
  case Activation::Sigmoid: return 1.0 / (1.0 + std::exp(-x));
  case Activation::LeakyReLU: return x < 0.0 ? 0.01 * x : x;
  case Activation::ReLU2: return x < 0.0 ? 0.0 : x * x;
  default: return x;
  }
}

double activate_deriv_f64(double x, Activation act) {
  switch (act) {
  case Activation::ReLU: return x > 0.0 ? 1.0 : 0.0;
  case Activation::ReLU2: return x > 0.0 ? 2.0 * x : 0.0;
  case Activation::LeakyReLU: return x > 0.0 ? 1.0 : 0.01;
  case Activation::Silu: {
    const double sg = 1.0 / (1.0 + std::exp(-x));
    return sg * (1.0 + x * (1.0 - sg));
  }
  case Activation::GELU: {
    const double k = 0.7978845608028654;
    const double th = std::tanh(k * (x + 0.044715 * x * x * x));
    const double du = k * (1.0 + 3.0 * 0.044715 * x * x);
    return 0.5 * (1.0 + th) + 0.5 * x * (1.0 - th * th) * du;
  }
  case Activation::Tanh: {
    const double t = std::tanh(x);
    return 1.0 - t * t;
  }
  case Activation::Sigmoid: {
    const double sg = 1.0 / (1.0 + std::exp(-x));
    return sg * (1.0 - sg);
  }
  default: return 1.0;
  }
}

// ------------------------------------------------------------ WeightStore --
Status WeightStore::make(int rows, int cols, DType dt, const float* init_or_null,
                         WeightStore* out) {
  return make_scaled(rows, cols, dt, ScaleScheme::Reference, init_or_null, out);
}

Status WeightStore::make_scaled(int rows, int cols, DType dt, ScaleScheme scheme,
                                const float* init_or_null, WeightStore* out) {
  if (!out || rows <= 0 || cols <= 0)
    return Status::Err(StatusCode::InvalidArgument, "weights: need rows > 0 and cols > 0");
  return guarded([&]() -> Status {
    WeightStore s;
    s.rows = rows;
    s.cols = cols;
    CX_TRY(quantize_into(rows, cols, dt, scheme, init_or_null, &s));
    *out = std::move(s);
    return Status::Ok();
  });
}

Status WeightStore::encode_format_none(DType dt, const float* scratch, int n) {
  if (!scratch || rows <= 0 || cols <= 0 || static_cast<int64_t>(n) != elems(*this))
    return Status::Err(StatusCode::InvalidArgument, "weights: encode needs rows * cols values");
  return guarded([&]() -> Status {
    WeightStore s;
    CX_TRY(quantize_into(rows, cols, dt, ScaleScheme::Reference, scratch, &s));
    s.bias = std::move(bias);
    *this = std::move(s);
    return Status::Ok();
  });
}

Status WeightStore::decode_row_f64(int row, double* dst) const {
  if (!dst || row < 0 || row >= rows)
    return Status::Err(StatusCode::InvalidArgument, "weights: decode row out of range");
  if (format != QuantFormat::None) return Status::Gap("decode_row_f64 of packed formats");
  if (!served(dtype)) return unserved("weights", dtype);
  return guarded([&]() -> Status {
    CX_WV(wv::init_device());
    std::vector<float> v(static_cast<size_t>(cols));
    CX_WV(wv::store_decode_rows(view_of(*this), row, 1, v.data(), nullptr));
    for (int c = 0; c < cols; ++c) dst[c] = static_cast<double>(v[static_cast<size_t>(c)]);
    return Status::Ok();
  });
}

Status WeightStore::export_f32(float* dst) const {
  if (!dst) return Status::Err(StatusCode::InvalidArgument, "weights: null export buffer");
  if (format != QuantFormat::None) return Status::Gap("export_f32 of packed formats");
  if (!served(dtype)) return unserved("weights", dtype);
  return guarded([&]() -> Status {
    CX_WV(wv::init_device());
    CX_WV(wv::store_decode_rows(view_of(*this), 0, rows, dst, nullptr));
    return Status::Ok();
  });
}

Status WeightStore::set_from_f32(const std::vector<float>& values) {
  if (rows <= 0 || cols <= 0 || static_cast<int64_t>(values.size()) != elems(*this) ||
      format != QuantFormat::None)
    return Status::Err(StatusCode::InvalidArgument,
                       "weights: replacement needs rows * cols values of a FormatNone store");
  return guarded([&]() -> Status {
    WeightStore s;
    CX_TRY(quantize_into(rows, cols, dtype, scheme, values.data(), &s));
    s.bias = std::move(bias);
    *this = std::move(s);
    return Status::Ok();
  });
}

Status WeightStore::matvec_f32(const float*, float*) const {
  return Status::Err(StatusCode::Unsupported,
                     "weights.matvec_f32: products run on the GPU (dense::forward_f32)");
}

Status WeightStore::matvect_f32(const float*, float*) const {
  return Status::Err(StatusCode::Unsupported,
                     "weights.matvect_f32: products run on the GPU (dense::backward_f32)");
}

Status WeightStore::apply_sgd(const double* dW, double lr) {
  if (!dW) return Status::Err(StatusCode::InvalidArgument, "weights: null dW");
  if (format != QuantFormat::None) return Status::Gap("apply_sgd of packed formats");
  if (!served(dtype)) return unserved("weights", dtype);
  return guarded([&]() -> Status {
    CX_WV(wv::init_device());
    wv::DenseLayer L;
    CX_WV(wv::dense_build_from_store(cols, rows, wv::kLinear, to_wv(*this), &L, nullptr));
    const size_t n = static_cast<size_t>(elems(*this));
    wv::DevBuf g;
    CX_WV(g.alloc(n * sizeof(double)));
    CX_WV(wv::copy_h2d(g.p, dW, n * sizeof(double), nullptr));
    CX_WV(wv::dense_apply_sgd(&L, g.as<const double>(), lr, nullptr));
    CX_WV(wv::hip_status(hipStreamSynchronize(nullptr), "sgd"));
    take_codes(std::move(L.store), this);
    return Status::Ok();
  });
}

Status WeightStore::apply_bias_sgd(const double* dB, int n, double lr) {
  if (bias.empty()) return Status::Ok();
  if (!dB) return Status::Err(StatusCode::InvalidArgument, "weights: null dB");
  if (n < static_cast<int>(bias.size()))
    return Status::Err(StatusCode::InvalidArgument, "weights: dB shorter than the bias");
  for (size_t i = 0; i < bias.size(); ++i) bias[i] -= lr * dB[i];
  return Status::Ok();
}

// ------------------------------------------------------------------ dense --
namespace dense {
namespace {

// Weights valid, workspace and buffers sized for `batch` rows.
Status ensure_batch(const Layer& layer, int batch) {
  CX_TRY(ensure_weights(layer));
  if (layer.gpu_batch == batch) return Status::Ok();
  DeviceState* d = layer.gpu.get();
  CX_WV(wv::dense_prepare_rows(&d->dense, batch, d->stream.s));
  CX_WV(wv::ensure_split(&d->ws, wv::dense_workspace_bytes(d->dense, batch)));
  const size_t xb = static_cast<size_t>(batch) * layer.input_height * sizeof(float);
  const size_t yb = static_cast<size_t>(batch) * layer.output_height * sizeof(float);
  CX_WV(fit(&d->x, xb));
  CX_WV(fit(&d->pre, yb));
  CX_WV(fit(&d->post, yb));
  d->rows = batch;
  layer.gpu_batch = batch;
  return Status::Ok();
}

Status check_input(const Layer& layer, const TensorF32& input, int* batch, const char* who) {
  if (input.shape.size() != 2)
    return Status::Err(StatusCode::InvalidArgument, std::string(who) + ": input must be [batch, in]");
  const int64_t b = input.shape[0];
  if (b <= 0 || b > (1 << 30) || input.shape[1] != layer.input_height ||
      static_cast<int64_t>(input.data.size()) != b * layer.input_height)
    return Status::Err(StatusCode::InvalidArgument,
                       std::string(who) + ": input does not match [batch, in]");
  *batch = static_cast<int>(b);
  return Status::Ok();
}

// Backward on host tensors: d_pre from gy and pre (act' unless linear), then
// dX and dW over the device weights.
Status run_backward(const Layer& layer, int batch, const float* gy, const float* x,
                    const float* pre, bool linear, TensorF32* grad_in, TensorF32* grad_w) {
  CX_TRY(ensure_batch(layer, batch));
  DeviceState* d = layer.gpu.get();
  hipStream_t st = d->stream.s;
  const size_t in = static_cast<size_t>(layer.input_height);
  const size_t out = static_cast<size_t>(layer.output_height);
  const size_t yb = batch * out * sizeof(float), xb = batch * in * sizeof(float);
  wv::DevBuf g, dpre, dx, dw;
  CX_WV(g.alloc(yb));
  CX_WV(dpre.alloc(yb));
  CX_WV(dx.alloc(xb));
  CX_WV(dw.alloc(out * in * sizeof(float)));
  CX_WV(wv::copy_h2d(g.p, gy, yb, st));
  CX_WV(wv::copy_h2d(d->x.p, x, xb, st));
  CX_WV(wv::copy_h2d(d->pre.p, pre, yb, st));
  CX_WV(wv::dense_backward(d->dense, batch, d->x.as<float>(), d->pre.as<float>(), nullptr,
                           g.as<float>(), false, dpre.as<float>(), dx.as<float>(), dw.as<float>(),
                           nullptr, &d->ws, st, linear));
  TensorF32 gi = TensorF32::zeros(batch, static_cast<int64_t>(in));
  TensorF32 gw = TensorF32::zeros(static_cast<int64_t>(out), static_cast<int64_t>(in));
  CX_WV(wv::copy_d2h(gi.data.data(), dx.p, xb, st));
  CX_WV(wv::copy_d2h(gw.data.data(), dw.p, out * in * sizeof(float), st));
  CX_WV(wv::hip_status(hipStreamSynchronize(st), "dense backward"));
  if (grad_in) *grad_in = std::move(gi);
  if (grad_w) *grad_w = std::move(gw);
  return Status::Ok();
}

}  // namespace

bool dtype_supported_cuda_forward(DType dt) { return served(dt); }

Status new_layer_scaled(int in_h, int out_h, Activation act, DType dt, ScaleScheme scheme,
                        const float* init_or_null, Layer* layer) {
  if (!layer) return Status::Err(StatusCode::InvalidArgument, "dense: null layer");
  if (in_h <= 0 || out_h <= 0)
    return Status::Err(StatusCode::InvalidArgument, "dense: need in > 0 and out > 0");
  if (!served(dt)) return unserved("dense", dt);
  return guarded([&]() -> Status {
    Layer L;
    L.input_height = in_h;
    L.output_height = out_h;
    L.activation = act;
    CX_TRY(WeightStore::make_scaled(out_h, in_h, dt, scheme, init_or_null, &L.weights));
    *layer = std::move(L);
    return Status::Ok();
  });
}

Status new_layer(int in_h, int out_h, Activation act, DType dt, const float* init_or_null,
                 Layer* layer) {
  return new_layer_scaled(in_h, out_h, act, dt, ScaleScheme::Reference, init_or_null, layer);
}

Status sync_gpu_from_weights(const Layer& layer, int batch) {
  if (batch <= 0) return Status::Err(StatusCode::InvalidArgument, "dense: batch must be > 0");
  return guarded([&]() -> Status {
    layer.gpu_valid = false;  // an explicit sync always re-uploads the weights
    return ensure_batch(layer, batch);
  });
}

Status forward_f32(const Layer& layer, const TensorF32& input, TensorF32* pre, TensorF32* post) {
  if (!pre || !post) return Status::Err(StatusCode::InvalidArgument, "dense: null pre / post");
  if (!served(layer.weights.dtype)) return unserved("dense", layer.weights.dtype);
  int batch = 0;
  CX_TRY(check_input(layer, input, &batch, "dense"));
  return guarded([&]() -> Status {
    CX_TRY(ensure_batch(layer, batch));
    DeviceState* d = layer.gpu.get();
    hipStream_t st = d->stream.s;
    const size_t xb = static_cast<size_t>(batch) * layer.input_height * sizeof(float);
    const size_t yb = static_cast<size_t>(batch) * layer.output_height * sizeof(float);
    CX_WV(wv::copy_h2d(d->x.p, input.data.data(), xb, st));
    CX_WV(wv::dense_forward(d->dense, batch, d->x.as<float>(), d->pre.as<float>(),
                            d->post.as<float>(), &d->ws, st));
    TensorF32 p = TensorF32::zeros(batch, layer.output_height);
    TensorF32 q = TensorF32::zeros(batch, layer.output_height);
    CX_WV(wv::copy_d2h(p.data.data(), d->pre.p, yb, st));
    CX_WV(wv::copy_d2h(q.data.data(), d->post.p, yb, st));
    CX_WV(wv::hip_status(hipStreamSynchronize(st), "dense forward"));
    *pre = std::move(p);
    *post = std::move(q);
    return Status::Ok();
  });
}

Status backward_f32(const Layer& layer, const TensorF32& grad_out, const TensorF32& input,
                    const TensorF32& pre, TensorF32* grad_in, TensorF32* grad_w) {
  if (!grad_in || !grad_w)
    return Status::Err(StatusCode::InvalidArgument, "dense: null gradient outputs");
  int batch = 0;
  CX_TRY(check_input(layer, input, &batch, "dense backward"));
  const int64_t ny = static_cast<int64_t>(batch) * layer.output_height;
  if (grad_out.shape.size() != 2 || pre.shape.size() != 2 || grad_out.shape[0] != batch ||
      grad_out.shape[1] != layer.output_height || pre.shape[0] != batch ||
      pre.shape[1] != layer.output_height || static_cast<int64_t>(grad_out.data.size()) != ny ||
      static_cast<int64_t>(pre.data.size()) != ny)
    return Status::Err(StatusCode::InvalidArgument,
                       "dense backward: grad_out and pre must be [batch, out]");
  return guarded([&]() -> Status {
    return run_backward(layer, batch, grad_out.data.data(), input.data.data(), pre.data.data(),
                        false, grad_in, grad_w);
  });
}

Status linear_grad_in(const Layer& layer, const TensorF32& gy, const TensorF32& input,
                      TensorF32* gx) {
  if (!gx || input.shape.size() != 2 || input.data.empty() || gy.data.empty())
    return Status::Err(StatusCode::InvalidArgument, "dense: linear_grad_in needs gy and input");
  int batch = 0;
  CX_TRY(check_input(layer, input, &batch, "dense linear_grad_in"));
  return guarded([&]() -> Status {
    const size_t ny = static_cast<size_t>(batch) * layer.output_height;
    const std::vector<float> g = wv::remap_len(gy.data.data(), gy.data.size(), ny);
    const std::vector<float> zero(ny, 0.0f);
    return run_backward(layer, batch, g.data(), input.data.data(), zero.data(), true, gx,
                        nullptr);
  });
}

Status grad_w_only(const Layer& layer, const TensorF32& gy, const TensorF32& input,
                   const TensorF32& pre, TensorF32* dw) {
  if (!dw || input.shape.size() != 2 || gy.data.empty())
    return Status::Err(StatusCode::InvalidArgument, "dense: grad_w_only needs gy and input");
  int batch = 0;
  CX_TRY(check_input(layer, input, &batch, "dense grad_w_only"));
  return guarded([&]() -> Status {
    const size_t ny = static_cast<size_t>(batch) * layer.output_height;
    const std::vector<float> g = wv::remap_len(gy.data.data(), gy.data.size(), ny);
    std::vector<float> p(ny, 0.0f);
    if (pre.shape.size() == 2 && pre.data.size() >= ny)
      std::memcpy(p.data(), pre.data.data(), ny * sizeof(float));
    return run_backward(layer, batch, g.data(), input.data.data(), p.data(), false, nullptr, dw);
  });
}

Status apply_grad_sgd(Layer* layer, const TensorF32& dW, double lr) {
  if (!layer) return Status::Err(StatusCode::InvalidArgument, "dense: null layer");
  const int64_t n = elems(layer->weights);
  if (static_cast<int64_t>(dW.data.size()) < n)
    return Status::Err(StatusCode::InvalidArgument, "dense: dW shorter than the weights");
  return guarded([&]() -> Status {
    CX_TRY(ensure_weights(*layer));
    DeviceState* d = layer->gpu.get();
    hipStream_t st = d->stream.s;
    wv::DevBuf g;
    CX_WV(g.alloc(static_cast<size_t>(n) * sizeof(float)));
    CX_WV(wv::copy_h2d(g.p, dW.data.data(), static_cast<size_t>(n) * sizeof(float), st));
    CX_WV(wv::dense_apply_sgd(&d->dense, g.as<const float>(), lr, st));
    CX_WV(wv::hip_status(hipStreamSynchronize(st), "dense sgd"));
    // the device copy is the updated store; the host store follows it
    wv::WeightStore w = d->dense.store;
    take_codes(std::move(w), &layer->weights);
    return Status::Ok();
  });
}

// --------------------------------------------------------------- sessions --
struct Session {
  welvet_dense_session* c = nullptr;
};

namespace {
Status from_c(const welvet_status& s) {
  if (s.code == 0) return Status::Ok();
  return Status::Err(static_cast<StatusCode>(s.code), s.message);
}
}  // namespace

Status session_mount(int32_t batch, int32_t in, int32_t out, Activation act, DType dt,
                     const float* W_init, const double* bias, size_t bias_len, Session** sess) {
  if (!sess || !W_init) return Status::Err(StatusCode::InvalidArgument, "dense: null mount args");
  *sess = nullptr;
  if (!served(dt)) return unserved("dense", dt);
  return guarded([&]() -> Status {
    welvet_dense_session* c = nullptr;
    CX_TRY(from_c(welvet_dense_mount(batch, in, out, static_cast<int32_t>(act),
                                     static_cast<int32_t>(dt), W_init, bias, bias_len, &c)));
    *sess = new Session{c};
    return Status::Ok();
  });
}

Status session_execute(Session* s, const float* x, float* pre, float* post) {
  if (!s || !s->c || !x || !pre || !post)
    return Status::Err(StatusCode::InvalidArgument, "dense: null execute args");
  return from_c(welvet_dense_execute(s->c, x, pre, post));
}

void session_release(Session* s) {
  if (!s) return;
  welvet_dense_release(s->c);
  delete s;
}

}  // namespace dense

// ------------------------------------------------------------ fused parts --
namespace {

// Lends the device weights of `n` parts to a fused layer object for one call:
// moved in at construction, moved back on every exit.
template <int N>
struct PartsLoan {
  wv::DenseLayer* fused[N];
  wv::DenseLayer* own[N];
  PartsLoan(wv::DenseLayer* const (&f)[N], wv::DenseLayer* const (&o)[N]) {
    for (int i = 0; i < N; ++i) {
      fused[i] = f[i], own[i] = o[i];
      *fused[i] = std::move(*own[i]);
    }
  }
  ~PartsLoan() {
    for (int i = 0; i < N; ++i) *own[i] = std::move(*fused[i]);
  }
  PartsLoan(const PartsLoan&) = delete;
  PartsLoan& operator=(const PartsLoan&) = delete;
};

// [batch, in] or [batch, seq, in] (seq_first false) / [batch, seq, d] or
// [seq, d] (seq_first true) into batch, seq.
Status layout_of(const TensorF32& input, int width, bool mha, int* batch, int* seq,
                 const char* who) {
  const auto& s = input.shape;
  int64_t b = 0, q = 0;
  if (input.data.empty())
    return Status::Err(StatusCode::InvalidArgument, std::string(who) + ": empty input");
  if (s.size() == 3 && s[2] == width) {
    b = s[0], q = s[1];
  } else if (s.size() == 2 && s[1] == width) {
    if (mha) b = 1, q = s[0];
    else b = s[0], q = 1;
  } else {
    return Status::Err(StatusCode::InvalidArgument,
                       std::string(who) + (mha ? ": input must be [batch, seq, d_model] or "
                                                 "[seq, d_model]"
                                               : ": input must be [batch, in] or [batch, seq, in]"));
  }
  if (b <= 0 || q <= 0 || b * q > (1 << 30) ||
      static_cast<int64_t>(input.data.size()) < b * q * width)
    return Status::Err(StatusCode::InvalidArgument, std::string(who) + ": bad batch / seq / data");
  *batch = static_cast<int>(b), *seq = static_cast<int>(q);
  return Status::Ok();
}

}  // namespace

// ----------------------------------------------------------------- swiglu --
namespace swiglu {

Status validate(const Config& cfg) {
  if (cfg.input_dim <= 0 || cfg.intermediate_dim <= 0)
    return Status::Err(StatusCode::InvalidArgument,
                       "swiglu: need input_dim > 0 and intermediate_dim > 0");
  return Status::Ok();
}

Config default_ffn(int d_model) {
  // 8/3 of d_model, rounded up to a multiple of 8 (the Llama feed-forward)
  int inter = (d_model * 8 / 3 + 7) / 8 * 8;
  if (inter < d_model) inter = 2 * d_model;
  return Config{d_model, inter};
}

Status new_configured(const Config& cfg, DType dt, const float* gate_init, const float* up_init,
                      const float* down_init, Layer* out) {
  if (!out) return Status::Err(StatusCode::InvalidArgument, "swiglu: null out");
  CX_TRY(validate(cfg));
  Layer L;
  L.cfg = cfg;
  const int in = cfg.input_dim, inter = cfg.intermediate_dim;
  CX_TRY(with_prefix(dense::new_layer(in, inter, Activation::Linear, dt, gate_init, &L.Gate),
                     "swiglu Gate: "));
  CX_TRY(with_prefix(dense::new_layer(in, inter, Activation::Linear, dt, up_init, &L.Up),
                     "swiglu Up: "));
  CX_TRY(with_prefix(dense::new_layer(inter, in, Activation::Linear, dt, down_init, &L.Down),
                     "swiglu Down: "));
  *out = std::move(L);
  return Status::Ok();
}

namespace {

// Gate, Up and Down of the configured shapes with their weights on the device.
Status parts_on_device(const Layer& L) {
  const int in = L.cfg.input_dim, inter = L.cfg.intermediate_dim;
  if (L.Gate.input_height != in || L.Gate.output_height != inter || L.Up.input_height != in ||
      L.Up.output_height != inter || L.Down.input_height != inter || L.Down.output_height != in)
    return Status::Err(StatusCode::InvalidArgument, "swiglu: Gate / Up / Down differ from cfg");
  if (L.Gate.weights.dtype != L.Up.weights.dtype || L.Gate.weights.scheme != L.Up.weights.scheme)
    return Status::Err(StatusCode::InvalidArgument, "swiglu: Gate and Up differ in dtype or scheme");
  CX_TRY(with_prefix(ensure_weights(L.Gate), "swiglu Gate: "));
  CX_TRY(with_prefix(ensure_weights(L.Up), "swiglu Up: "));
  CX_TRY(with_prefix(ensure_weights(L.Down), "swiglu Down: "));
  return Status::Ok();
}

// Runs fn(fused layer, state) with the parts' device weights lent to a
// wv::SwiGLULayer.
template <class F>
Status with_fused(Layer& L, int rows, F&& fn) {
  CX_TRY(parts_on_device(L));
  DeviceState* d = state_of(L.gpu);
  CX_WV(d->stream.create());
  wv::SwiGLULayer f;
  f.in = L.cfg.input_dim;
  f.inter = L.cfg.intermediate_dim;
  PartsLoan<3> loan({&f.gate, &f.up, &f.down},
                    {&L.Gate.gpu.get()->dense, &L.Up.gpu.get()->dense, &L.Down.gpu.get()->dense});
  CX_WV(wv::swiglu_finish(&f, d->stream.s));
  CX_WV(wv::swiglu_prepare_rows(&f, rows, d->stream.s));
  return fn(f, d);
}

}  // namespace

Status forward(Layer& layer, const TensorF32& input, TensorF32* pre, TensorF32* post) {
  if (!pre || !post) return Status::Err(StatusCode::InvalidArgument, "swiglu: null pre / post");
  CX_TRY(validate(layer.cfg));
  int batch = 0, seq = 0;
  CX_TRY(layout_of(input, layer.cfg.input_dim, false, &batch, &seq, "swiglu"));
  const int rows = batch * seq, in = layer.cfg.input_dim, inter = layer.cfg.intermediate_dim;
  return guarded([&]() -> Status {
    return with_fused(layer, rows, [&](const wv::SwiGLULayer& f, DeviceState* d) -> Status {
      hipStream_t st = d->stream.s;
      const size_t xb = static_cast<size_t>(rows) * in * sizeof(float);
      const size_t hb = static_cast<size_t>(rows) * inter * sizeof(float);
      CX_WV(fit(&d->x, xb));
      CX_WV(fit(&d->pre, hb));
      CX_WV(fit(&d->post, xb));
      CX_WV(wv::ensure_split(&d->ws, wv::swiglu_workspace_bytes(f, rows)));
      CX_WV(wv::copy_h2d(d->x.p, input.data.data(), xb, st));
      CX_WV(wv::swiglu_forward(f, rows, d->x.as<float>(), d->pre.as<float>(), d->post.as<float>(),
                               &d->ws, st));
      TensorF32 h, y;
      h.data.resize(static_cast<size_t>(rows) * inter);
      y.data.resize(static_cast<size_t>(rows) * in);
      CX_WV(wv::copy_d2h(h.data.data(), d->pre.p, hb, st));
      CX_WV(wv::copy_d2h(y.data.data(), d->post.p, xb, st));
      CX_WV(wv::hip_status(hipStreamSynchronize(st), "swiglu forward"));
      if (seq == 1) {
        h.shape = {batch, inter};
        y.shape = {batch, in};
      } else {
        h.shape = {batch, seq, inter};
        y.shape = {batch, seq, in};
      }
      *pre = std::move(h);
      *post = std::move(y);
      return Status::Ok();
    });
  });
}

Status backward_f32(Layer& layer, const TensorF32& grad_out, const TensorF32& input,
                    const TensorF32& pre, TensorF32* grad_in, TensorF32* grad_w) {
  if (!grad_in || !grad_w)
    return Status::Err(StatusCode::InvalidArgument, "swiglu: null gradient outputs");
  CX_TRY(validate(layer.cfg));
  int batch = 0, seq = 0;
  CX_TRY(layout_of(input, layer.cfg.input_dim, false, &batch, &seq, "swiglu"));
  const int rows = batch * seq, in = layer.cfg.input_dim, inter = layer.cfg.intermediate_dim;
  if (pre.data.size() < static_cast<size_t>(rows) * inter)
    return Status::Err(StatusCode::InvalidArgument, "swiglu: pre must be the forward's h");
  if (grad_out.data.size() < static_cast<size_t>(rows) * in)
    return Status::Err(StatusCode::InvalidArgument, "swiglu: grad_out shorter than the output");
  return guarded([&]() -> Status {
    return with_fused(layer, rows, [&](const wv::SwiGLULayer& f, DeviceState* d) -> Status {
      hipStream_t st = d->stream.s;
      const size_t xb = static_cast<size_t>(rows) * in * sizeof(float);
      const size_t hb = static_cast<size_t>(rows) * inter * sizeof(float);
      const size_t nw = static_cast<size_t>(grad_w_size(layer));
      wv::DevBuf g, y, dx, dw;
      CX_WV(fit(&d->x, xb));
      CX_WV(fit(&d->pre, hb));
      CX_WV(g.alloc(xb));
      CX_WV(y.alloc(xb));
      CX_WV(dx.alloc(xb));
      CX_WV(dw.alloc(nw * sizeof(float)));
      CX_WV(wv::copy_h2d(d->x.p, input.data.data(), xb, st));
      CX_WV(wv::copy_h2d(d->pre.p, pre.data.data(), hb, st));
      CX_WV(wv::copy_h2d(g.p, grad_out.data.data(), xb, st));
      // the Down product over the given h (its backward's pre; Linear)
      CX_WV(wv::dense_forward(f.down, rows, d->pre.as<float>(), y.as<float>(), nullptr, &d->ws,
                              st));
      CX_WV(wv::swiglu_backward(f, rows, d->x.as<float>(), d->pre.as<float>(), y.as<float>(),
                                g.as<float>(), false, dx.as<float>(), dw.as<float>(), nullptr,
                                &d->ws, st));
      TensorF32 gi;
      gi.data.resize(static_cast<size_t>(rows) * in);
      if (seq == 1) gi.shape = {batch, in};
      else gi.shape = {batch, seq, in};
      TensorF32 gw = TensorF32::zeros(1, static_cast<int64_t>(nw));
      CX_WV(wv::copy_d2h(gi.data.data(), dx.p, xb, st));
      CX_WV(wv::copy_d2h(gw.data.data(), dw.p, nw * sizeof(float), st));
      CX_WV(wv::hip_status(hipStreamSynchronize(st), "swiglu backward"));
      *grad_in = std::move(gi);
      *grad_w = std::move(gw);
      return Status::Ok();
    });
  });
}

int grad_w_size(const Layer& layer) {
  return static_cast<int>(elems(layer.Gate.weights) + elems(layer.Up.weights) +
                          elems(layer.Down.weights));
}

Status apply_grad_sgd(Layer* layer, const TensorF32& dW, double lr) {
  if (!layer) return Status::Err(StatusCode::InvalidArgument, "swiglu: null layer");
  if (static_cast<int64_t>(dW.data.size()) < grad_w_size(*layer))
    return Status::Err(StatusCode::InvalidArgument, "swiglu: dW shorter than the weights");
  size_t off = 0;
  for (dense::Layer* p : {&layer->Gate, &layer->Up, &layer->Down}) {
    const size_t n = static_cast<size_t>(elems(p->weights));
    TensorF32 slice;
    slice.shape = {p->weights.rows, p->weights.cols};
    slice.data.assign(dW.data.begin() + off, dW.data.begin() + off + n);
    CX_TRY(dense::apply_grad_sgd(p, slice, lr));
    off += n;
  }
  return Status::Ok();
}

Status export_weights_f32(const Layer& layer, float* dst) {
  if (!dst) return Status::Err(StatusCode::InvalidArgument, "swiglu: null export buffer");
  size_t off = 0;
  for (const dense::Layer* p : {&layer.Gate, &layer.Up, &layer.Down}) {
    CX_TRY(p->weights.export_f32(dst + off));
    off += static_cast<size_t>(elems(p->weights));
  }
  return Status::Ok();
}

}  // namespace swiglu

// -------------------------------------------------------------------- mha --
namespace mha {

double Config::scale() const {
  if (scale_override > 0) return scale_override;
  return 1.0 / std::sqrt(static_cast<double>(head_dim));
}

Status validate(Config* cfg) {
  if (!cfg) return Status::Err(StatusCode::InvalidArgument, "mha: null config");
  if (cfg->d_model <= 0 || cfg->num_heads <= 0)
    return Status::Err(StatusCode::InvalidArgument, "mha: need d_model > 0 and num_heads > 0");
  if (cfg->head_dim <= 0) {
    if (cfg->d_model % cfg->num_heads != 0)
      return Status::Err(StatusCode::InvalidArgument,
                         "mha: head_dim unset and d_model not a multiple of num_heads");
    cfg->head_dim = cfg->d_model / cfg->num_heads;
  }
  if (cfg->num_kv_heads <= 0) cfg->num_kv_heads = cfg->num_heads;
  if (cfg->num_heads % cfg->num_kv_heads != 0)
    return Status::Err(StatusCode::InvalidArgument, "mha: num_heads not a multiple of num_kv_heads");
  if (cfg->max_seq_len <= 0) cfg->max_seq_len = 512;
  if (cfg->mask == MaskKind::Unspecified) cfg->mask = MaskKind::Causal;
  if (cfg->mask == MaskKind::Causal) cfg->causal = true;
  if (cfg->rope_theta <= 0) cfg->rope_theta = 10000.0;
  if (cfg->softmax != SoftmaxKind::Standard && cfg->softmax != SoftmaxKind::Sigmoid)
    return Status::Err(StatusCode::InvalidArgument, "mha: unknown softmax kind");
  return Status::Ok();
}

Config decoder_causal(int d_model, int num_heads, int num_kv_heads) {
  Config c;
  c.d_model = d_model;
  c.num_heads = num_heads;
  c.num_kv_heads = num_kv_heads;
  c.mask = MaskKind::Causal;
  c.pos = PosKind::RoPE;
  c.mode = AttnMode::Self;
  c.causal = true;
  return c;
}

Status new_configured(const Config& cfg_in, DType dt, const float* q_init, const float* k_init,
                      const float* v_init, const float* o_init, Layer* out) {
  if (!out) return Status::Err(StatusCode::InvalidArgument, "mha: null out");
  Config cfg = cfg_in;
  CX_TRY(validate(&cfg));
  Layer L;
  L.cfg = cfg;
  const int d = cfg.d_model, qd = cfg.q_dim(), kvd = cfg.kv_dim();
  CX_TRY(with_prefix(dense::new_layer(d, qd, Activation::Linear, dt, q_init, &L.Q), "mha Q: "));
  CX_TRY(with_prefix(dense::new_layer(d, kvd, Activation::Linear, dt, k_init, &L.K), "mha K: "));
  CX_TRY(with_prefix(dense::new_layer(d, kvd, Activation::Linear, dt, v_init, &L.V), "mha V: "));
  CX_TRY(with_prefix(dense::new_layer(qd, d, Activation::Linear, dt, o_init, &L.O), "mha O: "));
  *out = std::move(L);
  return Status::Ok();
}

Status forward(Layer& layer, const TensorF32& input, TensorF32* pre, TensorF32* post) {
  if (!pre || !post) return Status::Err(StatusCode::InvalidArgument, "mha: null pre / post");
  Config cfg = layer.cfg;
  CX_TRY(validate(&cfg));
  if (cfg.mode != AttnMode::Self) return Status::Gap("mha forward: cross attention");
  int batch = 0, seq = 0;
  CX_TRY(layout_of(input, cfg.d_model, true, &batch, &seq, "mha"));
  if (seq > cfg.max_seq_len) return Status::Err(StatusCode::InvalidArgument, "mha: seq > max_seq_len");
  const int d = cfg.d_model, qd = cfg.q_dim(), kvd = cfg.kv_dim();
  const dense::Layer* parts[4] = {&layer.Q, &layer.K, &layer.V, &layer.O};
  const int shape[4][2] = {{qd, d}, {kvd, d}, {kvd, d}, {d, qd}};
  for (int i = 0; i < 4; ++i)
    if (parts[i]->output_height != shape[i][0] || parts[i]->input_height != shape[i][1])
      return Status::Err(StatusCode::InvalidArgument, "mha: Q / K / V / O differ from cfg");
  return guarded([&]() -> Status {
    static const char* const kPrefix[4] = {"mha Q: ", "mha K: ", "mha V: ", "mha O: "};
    for (int i = 0; i < 4; ++i) CX_TRY(with_prefix(ensure_weights(*parts[i]), kPrefix[i]));
    DeviceState* ds = state_of(layer.gpu);
    CX_WV(ds->stream.create());
    hipStream_t st = ds->stream.s;
    wv::MHALayer f;
    f.cfg.d_model = d;
    f.cfg.num_heads = cfg.num_heads;
    f.cfg.num_kv_heads = cfg.num_kv_heads;
    f.cfg.head_dim = cfg.head_dim;
    f.cfg.max_seq_len = cfg.max_seq_len;
    f.cfg.mask = static_cast<int>(cfg.mask);
    f.cfg.pos = static_cast<int>(cfg.pos);
    f.cfg.softmax = static_cast<int>(cfg.softmax);
    f.cfg.window = cfg.window;
    f.cfg.prefix_len = cfg.prefix_len;
    // the reference passes window_causal || causal to its attention kernel
    f.cfg.window_causal = (cfg.window_causal || cfg.causal) ? 1 : 0;
    f.cfg.rope_theta = cfg.rope_theta;
    f.cfg.scale_override = cfg.scale_override;
    CX_WV(wv::mha_validate(&f.cfg));
    PartsLoan<4> loan({&f.q, &f.k, &f.v, &f.o},
                      {&layer.Q.gpu.get()->dense, &layer.K.gpu.get()->dense,
                       &layer.V.gpu.get()->dense, &layer.O.gpu.get()->dense});
    const int T = batch * seq;
    const size_t xb = static_cast<size_t>(T) * d * sizeof(float);
    const size_t ab = static_cast<size_t>(T) * qd * sizeof(float);
    CX_WV(fit(&ds->x, xb));
    CX_WV(fit(&ds->pre, ab));
    CX_WV(fit(&ds->post, xb));
    CX_WV(wv::mha_prepare(f, batch, seq, &ds->ws));
    CX_WV(wv::copy_h2d(ds->x.p, input.data.data(), xb, st));
    CX_WV(wv::mha_forward(f, batch, seq, ds->x.as<float>(), ds->pre.as<float>(),
                          ds->post.as<float>(), &ds->ws, st));
    TensorF32 a, y;
    a.shape = {batch, seq, qd};
    y.shape = {batch, seq, d};
    a.data.resize(static_cast<size_t>(T) * qd);
    y.data.resize(static_cast<size_t>(T) * d);
    CX_WV(wv::copy_d2h(a.data.data(), ds->pre.p, ab, st));
    CX_WV(wv::copy_d2h(y.data.data(), ds->post.p, xb, st));
    CX_WV(wv::hip_status(hipStreamSynchronize(st), "mha forward"));
    *pre = std::move(a);
    *post = std::move(y);
    return Status::Ok();
  });
}

int grad_w_size(const Layer& layer) {
  return static_cast<int>(elems(layer.Q.weights) + elems(layer.K.weights) +
                          elems(layer.V.weights) + elems(layer.O.weights));
}

Status backward_f32(const Layer&, const TensorF32&, const TensorF32&, const TensorF32&,
                    TensorF32*, TensorF32*) {
  return Status::Gap("mha backward_f32: the attention backward is not part of the quantized "
                     "Dense path");
}

Status apply_grad_sgd(Layer* layer, const TensorF32& dW, double lr) {
  if (!layer) return Status::Err(StatusCode::InvalidArgument, "mha: null layer");
  if (static_cast<int64_t>(dW.data.size()) < grad_w_size(*layer))
    return Status::Err(StatusCode::InvalidArgument, "mha: dW shorter than the weights");
  size_t off = 0;
  for (dense::Layer* p : {&layer->Q, &layer->K, &layer->V, &layer->O}) {
    const size_t n = static_cast<size_t>(elems(p->weights));
    TensorF32 slice;
    slice.shape = {p->weights.rows, p->weights.cols};
    slice.data.assign(dW.data.begin() + off, dW.data.begin() + off + n);
    CX_TRY(dense::apply_grad_sgd(p, slice, lr));
    off += n;
  }
  return Status::Ok();
}

Status export_weights_f32(const Layer& layer, float* dst) {
  if (!dst) return Status::Err(StatusCode::InvalidArgument, "mha: null export buffer");
  size_t off = 0;
  for (const dense::Layer* p : {&layer.Q, &layer.K, &layer.V, &layer.O}) {
    CX_TRY(p->weights.export_f32(dst + off));
    off += static_cast<size_t>(elems(p->weights));
  }
  return Status::Ok();
}

}  // namespace mha
}  // namespace welvet
