// A C++ caller of the layer/weights API that includes only the public
// headers under include/welvet/ and links libwelvet.so, as an in-tree C++
// user of the reference API would (reference include/welvet/weights.hpp,
// dense.hpp, dense_session.hpp, swiglu.hpp, mha.hpp). The test suite loads
// it with ctypes: each entry point runs one API sequence on host arrays and
// returns the status code, with the status message in `msg`.
#include <cstring>
#include <string>
#include <vector>

#include "welvet/dense.hpp"
#include "welvet/dense_session.hpp"
#include "welvet/mha.hpp"
#include "welvet/swiglu.hpp"
#include "welvet/weights.hpp"

using namespace welvet;

namespace {

int report(const Status& s, char* msg, int msg_len) {
  if (msg && msg_len > 0) {
    const size_t n = s.message.size() < (size_t)msg_len - 1 ? s.message.size() : (size_t)msg_len - 1;
    std::memcpy(msg, s.message.data(), n);
    msg[n] = '\0';
  }
  return static_cast<int>(s.code);
}

void copy_out(const TensorF32& t, float* dst) {
  if (dst) std::memcpy(dst, t.data.data(), t.data.size() * sizeof(float));
}

}  // namespace

extern "C" {

// new_layer (scheme 0) or new_layer_scaled, then forward_f32 `repeats`
// times on x [batch][in] (the first call mounts, later ones reuse the
// device weights); pre and post [batch][out] from the last call.
__attribute__((visibility("default"))) int probe_dense_forward(
    int in, int out, int act, int dtype, int scheme, int batch, int repeats, const float* W,
    const float* x, float* pre, float* post, char* msg, int msg_len) {
  dense::Layer L;
  Status s = scheme == 0 ? dense::new_layer(in, out, Activation(act), DType(dtype), W, &L)
                         : dense::new_layer_scaled(in, out, Activation(act), DType(dtype),
                                                   ScaleScheme(scheme), W, &L);
  if (!s) return report(s, msg, msg_len);
  TensorF32 input;
  input.shape = {batch, in};
  input.data.assign(x, x + (size_t)batch * in);
  TensorF32 p, q;
  for (int r = 0; r < repeats && s; ++r) s = dense::forward_f32(L, input, &p, &q);
  if (!s) return report(s, msg, msg_len);
  if (p.shape != std::vector<int64_t>{batch, out} || q.shape != p.shape)
    return report(Status::Err(StatusCode::Internal, "probe: output shape"), msg, msg_len);
  copy_out(p, pre);
  copy_out(q, post);
  return report(s, msg, msg_len);
}

// WeightStore::make_scaled, then the payload (native, row scales, E8M0
// bytes; caps in bytes / counts), every row through decode_row_f64 and the
// whole matrix through export_f32.
__attribute__((visibility("default"))) int probe_store(int rows, int cols, int dtype, int scheme,
                                                       const float* W, uint8_t* native,
                                                       size_t native_cap, size_t* native_len,
                                                       float* row_scale, uint8_t* blk_exp,
                                                       size_t blk_cap, double* rows_f64,
                                                       float* exported, char* msg, int msg_len) {
  WeightStore ws;
  Status s = WeightStore::make_scaled(rows, cols, DType(dtype), ScaleScheme(scheme), W, &ws);
  if (!s) return report(s, msg, msg_len);
  if (native_len) *native_len = ws.native.size();
  if (ws.native.size() > native_cap || ws.blk_exp.size() > blk_cap)
    return report(Status::Err(StatusCode::InvalidArgument, "probe: caps"), msg, msg_len);
  std::memcpy(native, ws.native.data(), ws.native.size());
  std::memcpy(row_scale, ws.row_scale.data(), ws.row_scale.size() * sizeof(float));
  std::memcpy(blk_exp, ws.blk_exp.data(), ws.blk_exp.size());
  for (int r = 0; r < rows && s; ++r) s = ws.decode_row_f64(r, rows_f64 + (size_t)r * cols);
  if (s) s = ws.export_f32(exported);
  return report(s, msg, msg_len);
}

// A dense session mounted at `batch` (reference FormatNone codes), executed
// once.
__attribute__((visibility("default"))) int probe_session(int batch, int in, int out, int act,
                                                         int dtype, const float* W,
                                                         const double* bias, size_t bias_len,
                                                         const float* x, float* pre, float* post,
                                                         char* msg, int msg_len) {
  dense::Session* sess = nullptr;
  Status s = dense::session_mount(batch, in, out, Activation(act), DType(dtype), W, bias, bias_len,
                                  &sess);
  if (!s) return report(s, msg, msg_len);
  s = dense::session_execute(sess, x, pre, post);
  dense::session_release(sess);
  return report(s, msg, msg_len);
}

// Dense backward_f32 (and, with lr != 0, apply_grad_sgd then export of the
// updated weights).
__attribute__((visibility("default"))) int probe_dense_backward(
    int in, int out, int act, int dtype, int scheme, int batch, const float* W, const float* x,
    const float* gy, float* grad_in, float* grad_w, double lr, float* w_after, char* msg,
    int msg_len) {
  dense::Layer L;
  Status s = dense::new_layer_scaled(in, out, Activation(act), DType(dtype), ScaleScheme(scheme),
                                     W, &L);
  if (!s) return report(s, msg, msg_len);
  TensorF32 input, g, p, q, gi, gw;
  input.shape = {batch, in};
  input.data.assign(x, x + (size_t)batch * in);
  g.shape = {batch, out};
  g.data.assign(gy, gy + (size_t)batch * out);
  s = dense::forward_f32(L, input, &p, &q);
  if (s) s = dense::backward_f32(L, g, input, p, &gi, &gw);
  if (!s) return report(s, msg, msg_len);
  copy_out(gi, grad_in);
  copy_out(gw, grad_w);
  if (lr != 0.0) {
    s = dense::apply_grad_sgd(&L, gw, lr);
    if (s) s = L.weights.export_f32(w_after);
  }
  return report(s, msg, msg_len);
}

// swiglu::new_configured + forward on x [rows][in] (2-D input).
__attribute__((visibility("default"))) int probe_swiglu(int in, int inter, int dtype, int rows,
                                                        const float* G, const float* U,
                                                        const float* D, const float* x, float* h,
                                                        float* y, char* msg, int msg_len) {
  swiglu::Layer L;
  Status s = swiglu::new_configured(swiglu::Config{in, inter}, DType(dtype), G, U, D, &L);
  if (!s) return report(s, msg, msg_len);
  TensorF32 input, p, q;
  input.shape = {rows, in};
  input.data.assign(x, x + (size_t)rows * in);
  s = swiglu::forward(L, input, &p, &q);
  if (!s) return report(s, msg, msg_len);
  copy_out(p, h);
  copy_out(q, y);
  return report(s, msg, msg_len);
}

// mha::new_configured + forward on x [batch][seq][d_model].
__attribute__((visibility("default"))) int probe_mha(int batch, int seq, int d_model, int heads,
                                                     int kv_heads, int msl, int mask, int pos,
                                                     int dtype, const float* Q, const float* K,
                                                     const float* V, const float* O,
                                                     const float* x, float* attn, float* y,
                                                     char* msg, int msg_len) {
  mha::Config cfg = mha::decoder_causal(d_model, heads, kv_heads);
  cfg.max_seq_len = msl;
  cfg.mask = mha::MaskKind(mask);
  cfg.pos = mha::PosKind(pos);
  cfg.causal = mask == 1;
  mha::Layer L;
  Status s = mha::new_configured(cfg, DType(dtype), Q, K, V, O, &L);
  if (!s) return report(s, msg, msg_len);
  TensorF32 input, a, q;
  input.shape = {batch, seq, d_model};
  input.data.assign(x, x + (size_t)batch * seq * d_model);
  s = mha::forward(L, input, &a, &q);
  if (!s) return report(s, msg, msg_len);
  copy_out(a, attn);
  copy_out(q, y);
  return report(s, msg, msg_len);
}

// dtype_name of an id into buf; dtype_implemented_forward as the result.
__attribute__((visibility("default"))) int probe_dtype(int id, char* buf, int len) {
  const std::string_view n = dtype_name(DType(id));
  const size_t k = n.size() < (size_t)len - 1 ? n.size() : (size_t)len - 1;
  std::memcpy(buf, n.data(), k);
  buf[k] = '\0';
  return dtype_implemented_forward(DType(id)) ? 1 : 0;
}

}  // extern "C"
