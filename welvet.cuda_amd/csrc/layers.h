// Layer objects of the quantized Dense path: the host weight store, Dense,
// SwiGLU and MHA layers over device-resident quantized weights.
#pragma once

#include <vector>

#include "common.h"
#include "kernels.h"
#include "runtime.h"

namespace wv {

// Host mirror of the reference WeightStore (include/welvet/weights.hpp:18-51)
// for FP8/FP4, plus the scale extension. `native` is the reference FormatNone
// payload; `scale` is the reference's single float (the tensor scale under
// scheme 1, else 1).
struct WeightStore {
  int dtype = 0, scheme = 0, rows = 0, cols = 0;
  std::vector<uint8_t> native;
  float scale = 1.0f;
  std::vector<float> row_scale;   // [rows]
  std::vector<uint8_t> blk_exp;   // [rows][ceil(cols/32)], scheme 3
  std::vector<double> bias;
};

Status check_dtype_scheme(int dtype, int scheme);

// The ABI's `backend` argument: bits 0-3 the scale scheme (0-3); bit 4 asks
// for two activation terms instead of three on the matrix-core paths of a
// Dense layer: two thirds of the matrix-core work and activation bytes, a
// per-product rel-L2 of ~6.3e-4 instead of ~2e-5 (measured), inside the
// 1e-3 layer bound. SwiGLU and MHA layers refuse it (their chained products
// and the softmax take the error past the bound). Other bits are invalid.
constexpr int kBackendTwoTerms = 0x10;
// bit 5: one activation term (the throughput mode: about 2.7e-2 relative L2,
// outside the 1e-3 layer bound); Dense layers above 32 rows only
constexpr int kBackendOneTerm = 0x20;
Status decode_backend(int backend, int* scheme, int* terms);

// Scratch owned by a session and reused across calls (grown at mount).
struct Workspace {
  DevBuf a;  // quantized activations / intermediates
  DevBuf b;
  DevBuf c;  // MHA: RoPE (cos, sin) table for rope_tokens tokens of rope_hd, rope_theta
  DevBuf d;
  // a serial chain of Dense layers: the next layer's split terms (and its
  // partial sums), written by this layer's K-split reduce; swapped with b
  DevBuf e;
  int rope_tokens = 0, rope_hd = 0;
  double rope_theta = 0.0;
};

// Resident weights of a packed block format (formats.hip): the arrays that
// FmtArgs points at, and the packed blocks as mounted (a host copy, for
// export).
struct FormatWeights {
  int format = 0, rows = 0, cols = 0, rpad = 0, nsub = 0;
  DevBuf q, h, s, e;
  std::vector<uint8_t> blocks;
};

struct DenseLayer {
  int in = 0, out = 0, act = kLinear;
  int terms = kTerms;  // activation terms of the matrix-core paths (2 or 3)
  int format = kFmtNone;  // a packed block format: the weights are in fw, not dev
  FormatWeights fw;
  WeightStore store;
  DeviceWeights dev;
  DevBuf bias_dev;
  int bias_len = 0;
  bool need_epi() const { return act != kLinear || bias_len > 0; }
};

// Quantizes the host fp32 matrix W_host [out][in] on the device into L.
Status dense_build(int in, int out, int act, int dtype, int scheme, const float* W_host,
                   const double* bias, size_t bias_len, DenseLayer* L, hipStream_t st);
// Builds L from a stored payload (reference FormatNone bytes + scales).
Status dense_build_from_store(int in, int out, int act, const WeightStore& store, DenseLayer* L,
                              hipStream_t st);

// A Dense layer over a packed block format (QuantFormat): from fp32 W_host
// (quantized on the device, every built format: format_quantize) or from the
// format's packed row-major blocks (blocks_len bytes); exactly one is given.
// in must be a multiple of the format's block (32, or 256 for the K formats).
Status dense_build_format(int in, int out, int act, int format, const float* W_host,
                          const uint8_t* blocks, size_t blocks_len, const double* bias,
                          size_t bias_len, DenseLayer* L, hipStream_t st);
// The layer's weights dequantized to f32 [out][in] in device memory w (the
// role of WeightStore::export_f32, src/weights/store.cpp:42-71).
Status dense_export_f32(const DenseLayer& L, float* w, hipStream_t st);

// Batch rows at or below this go to the GEMV kernels.
int gemv_batch_limit();

// Device forward: x [batch][in] -> pre/post [batch][out]; queued on st.
// post may be null when the caller only wants pre (Linear, no bias).
Status dense_forward(const DenseLayer& L, int batch, const float* x, float* pre, float* post,
                     Workspace* ws, hipStream_t st);
// Workspace bytes dense_forward needs for this batch.
size_t dense_workspace_bytes(const DenseLayer& L, int batch);

// Dense backward on device buffers (the NormalBP leaf,
// src/interop/c_abi.cpp:119-200): from the forward's x, pre and post and
// either the output gradient (use_target false) or an MSE target in g,
// d_pre [batch][out], dX [batch][in] and dW [out][in]; with a target,
// loss_part [dpre_blocks(batch * out)] gets the partial sums of the squared
// differences. ws->d holds the dX partial sums.
// linear_act takes act' as 1 (the reference's linear backward,
// resident_backward(..., linear = true)).
Status dense_backward(const DenseLayer& L, int batch, const float* x, const float* pre,
                      const float* post, const float* g, bool use_target, float* dpre, float* dx,
                      float* dw, double* loss_part, Workspace* ws, hipStream_t st,
                      bool linear_act = false);
// SGD on the quantized store (native_codec.cpp:1080-1133): W <- quantize(
// f32(f64(dequant(W)) - lr * f64(dW))) with the layer's scheme; the device
// copy and the host store are replaced.
Status dense_apply_sgd(DenseLayer* L, const float* dw, double lr, hipStream_t st);
// The same with an f64 gradient (WeightStore::apply_sgd takes f64 dW).
Status dense_apply_sgd(DenseLayer* L, const double* dw, double lr, hipStream_t st);

// A weight store quantized on the device from host fp32 W [rows][cols] (null:
// zeros) with `scheme` (WeightStore::make: native codes, scales; no bias).
Status store_quantize(int rows, int cols, int dtype, int scheme, const float* W_host,
                      WeightStore* out, hipStream_t st);
// A store's payload in host memory, not owned (the C++ API's WeightStore
// and this library's share the layout).
struct StoreView {
  int dtype = 0, scheme = 0, rows = 0, cols = 0;
  const uint8_t* native = nullptr;
  size_t native_len = 0;
  const float* row_scale = nullptr;  // [rows], schemes 1 and 2
  size_t row_scale_len = 0;
  const uint8_t* blk_exp = nullptr;  // [rows][ceil(cols / 32)], scheme 3
  size_t blk_exp_len = 0;
};
// Rows [row0, row0 + nrows) of a store, dequantized on the device (decode
// times the row scale or block scale) into host_out [nrows][cols]. Only
// those rows' bytes are uploaded.
Status store_decode_rows(const StoreView& s, int row0, int nrows, float* host_out,
                         hipStream_t st);
// ABI remap_gap_len (reference src/layers/dense/dense.cpp:121-139): src
// resized to `need` values, a different length averaging ranges of src in
// f64.
std::vector<float> remap_len(const float* src, size_t sn, size_t need);
// True when `batch` rows take the split + batched-MFMA path.
bool uses_split(int batch);
// Builds the operand-order code copy when `batch` rows run the 5..32-row
// GEMM (sessions call this at mount, their batch being fixed); a no-op
// otherwise or when the copy exists. Without it that GEMM reads the
// row-major codes, with the same results.
Status dense_prepare_rows(DenseLayer* L, int batch, hipStream_t st);
// The activation-split workspace (Workspace::b): the split terms, then the
// K-split partial sums of the products that use them.
inline uint8_t* split_buf(Workspace* ws) { return ws->b.as<uint8_t>(); }
// Batched path (batch > 4 rows) on x [batch][L.in]. Above 32 rows the GEMM
// reads the split terms of x from split_buf(ws), made here unless
// `split_ready` (launch_split of x with L.dev.kpad already ran); up to 32
// rows the GEMM kernel splits x itself. keep_out: the next launch reads the
// output (MxgArgs::keep_out).
// next_split: the reduce of this layer's K-split product also writes the
// split of post there, for `next` (dense_fuses_next must hold).
Status dense_forward_split(const DenseLayer& L, int batch, const float* x, bool split_ready,
                           Workspace* ws, float* pre, float* post, hipStream_t st,
                           const double* rope_tab = nullptr, int rope_hd = 0,
                           bool keep_out = false, uint8_t* next_split = nullptr);
// True when `batch` rows of L and then `next` (whose input is L's post) can
// run with L's K-split reduce writing next's split terms: both on the
// split matrix-core path above 32 rows, L's product split along K, N a
// multiple of 256 equal to next's kpad, the same activation terms, and no
// weight rows of L with non-finite codes (whose recomputation follows the
// product).
bool dense_fuses_next(const DenseLayer& L, const DenseLayer& next, int batch);
// Grows ws->b to at least n bytes (mount time; a forward that finds it too
// small allocates, which a captured graph cannot do).
Status ensure_split(Workspace* ws, size_t n);

// Dense layers of one shape run together (independent cells of a volume):
// one split launch and one GEMM launch for all members. Inputs and outputs
// are fixed device buffers given at build time, so a group can be replayed
// (and captured) without host work. Only batches above 32 rows use the
// grouped kernels (dense_group_fused); smaller ones run member by member.
struct DenseGroup {
  int n = 0, batch = 0, dtype = 0, terms = kTerms;
  bool blk = false, vec = false;
  int in = 0, kpad = 0;
  MxgArgs shape;
  DevBuf split;  // n slices of split_bytes(batch, kpad)
  DevBuf jobs;   // SplitJob[n]
  DevBuf tab;    // MxgArgs[n]
  std::vector<SplitJob> hjobs;  // host copies of jobs and tab
  std::vector<MxgArgs> htab;
  std::vector<const DenseLayer*> layers;  // the members
};
bool dense_group_fused(int batch);
Status dense_group_build(const DenseLayer* const* layers, int n, int batch,
                         const float* const* x, float* const* pre, float* const* post,
                         DenseGroup* g);
Status dense_group_forward(const DenseGroup& g, hipStream_t st);

// Groups run in order where group k + 1 reads what group k writes (member i's
// x is member i's post, or its pre when the two are one buffer): the layers
// of a volume's cells. Where group k's out is a multiple of 256 (then the
// consumer's kpad equals it), group k's GEMM epilogue writes group k + 1's
// split buffer as well and group k + 1 runs no split kernel. Without
// keep_inner, such a group k writes only that split, not its own pre / post
// (the cells of a volume return their last layer's output only).
struct DenseChain {
  std::vector<const DenseGroup*> groups;
  std::vector<DevBuf> tabs;  // per link k -> k + 1: group k's MxgArgs[n] with `next` set
  std::vector<char> fused;   // per link: the epilogue writes the next split
};
Status dense_chain_build(const DenseGroup* const* groups, int count, DenseChain* c,
                         bool keep_inner = true);
Status dense_chain_forward(const DenseChain& c, hipStream_t st);

struct SwiGLULayer {
  int in = 0, inter = 0;
  DenseLayer gate, up, down;
  // union of the gate and up rows with non-finite codes
  DevBuf nf_gu;
  std::vector<int> nf_gu_host;
};
// Completes a SwiGLU layer whose three matrices are built (the row list above).
Status swiglu_finish(SwiGLULayer* L, hipStream_t st);
Status swiglu_build(int in, int inter, int dtype, int scheme, const float* G, const float* U,
                    const float* D, SwiGLULayer* L, hipStream_t st);
// x [rows][in] -> h [rows][inter] (pre), y [rows][in] (post).
Status swiglu_forward(const SwiGLULayer& L, int rows, const float* x, float* h, float* y,
                      Workspace* ws, hipStream_t st);
size_t swiglu_workspace_bytes(const SwiGLULayer& L, int rows);
// dense_prepare_rows for the three matrices.
Status swiglu_prepare_rows(SwiGLULayer* L, int rows, hipStream_t st);
// SwiGLU backward on device buffers (swiglu.cpp:156-248): from x [rows][in],
// the forward's h and y, and the output gradient (or, with use_target, the
// MSE target) in g: dx [rows][in] and dw = [dGate | dUp | dDown] (each
// [out][in] of its matrix); with a target, loss_part as dense_backward.
// Gate and Up are recomputed; scratch buffers come from the call.
Status swiglu_backward(const SwiGLULayer& L, int rows, const float* x, const float* h,
                       const float* y, const float* g, bool use_target, float* dx, float* dw,
                       double* loss_part, Workspace* ws, hipStream_t st);
// SGD on the three stores with their slices of dw (swiglu.cpp:250-268).
Status swiglu_apply_sgd(SwiGLULayer* L, const float* dw, double lr, hipStream_t st);

struct MHAConfig {
  int d_model = 0, num_heads = 0, num_kv_heads = 0, head_dim = 0, max_seq_len = 0;
  int mask = 1, pos = 0, softmax = 0, window = 0, prefix_len = 0, window_causal = 1;
  double rope_theta = 10000.0, scale_override = 0.0;
  int q_dim() const { return num_heads * head_dim; }
  int kv_dim() const { return num_kv_heads * head_dim; }
};
// Fills defaults and validates as src/layers/mha/mha.cpp:55-81.
Status mha_validate(MHAConfig* c);
struct MHALayer {
  MHAConfig cfg;
  DenseLayer q, k, v, o;
};
Status mha_build(const MHAConfig& cfg, int dtype, int scheme, const float* Q, const float* K,
                 const float* V, const float* O, MHALayer* L, hipStream_t st);
// x [batch*seq][d] -> attn [batch*seq][q_dim] (pre), y [batch*seq][d] (post).
Status mha_forward(const MHALayer& L, int batch, int seq, const float* x, float* attn, float* y,
                   Workspace* ws, hipStream_t st);
size_t mha_workspace_bytes(const MHALayer& L, int batch, int seq);
// Sizes the workspace for (batch, seq) ahead of forward calls.
Status mha_prepare(const MHALayer& L, int batch, int seq, Workspace* ws);

}  // namespace wv
