// Persistent model sessions over the WMN1 descriptor (Stack and Grid roots).
#pragma once

#include <memory>
#include <vector>

#include "layers.h"

namespace wv {

// One child of a Stack / one Grid cell (reference stack::Kind values,
// include/welvet/stack.hpp:50-77): 0 None, 1 Dense, 4 SwiGLU, 7 MHA,
// 19 NestedStack.
struct ModelNode {
  int kind = 0;
  // Dense
  int in = 0, out = 0, act = kLinear, dtype = 0;
  std::vector<float> W;  // child fp32 weights (the store payload overrides)
  // SwiGLU
  int inter = 0;
  // MHA
  MHAConfig mha_cfg;
  std::vector<float> W2, W3, W4;  // Up/Down or K/V/O
  std::vector<ModelNode> nested;
  // stores in collect order (Dense: 1, SwiGLU: 3, MHA: 4)
  std::vector<WeightStore> stores;
  // built layers
  std::unique_ptr<DenseLayer> dense;
  std::unique_ptr<SwiGLULayer> swiglu;
  std::unique_ptr<MHALayer> mha;
};

struct GridCell {
  int enabled = 0, remote = 0, tz = 0, ty = 0, tx = 0, tl = 0;
};

// Device memory a forward pass uses, kept across passes: the op outputs are
// taken from `bufs` in op order (the same sizes pass after pass, so a steady
// state allocates nothing), `ws` holds the split and K-split buffers, `in`
// the uploaded input of a host-buffer call. Calls on one model must not
// overlap (the session serializes them).
struct ModelScratch {
  std::vector<DevBuf> bufs;
  size_t next = 0;
  Workspace ws;
  DevBuf in;
};

struct Model {
  int root = 0;  // 0 Stack, 2 Grid
  int dims[4] = {1, 1, 1, 1};
  std::vector<ModelNode> children;  // Stack children or Grid cells in hop order
  std::vector<GridCell> cells;
  int scheme = 0;
  int terms = kTerms;  // activation terms of the Dense and MHA layers' matrix-core paths
  ModelScratch scratch;
};

// Parses and validates a WMN1 descriptor (src/interop/model_session.cpp:
// 319-404) without touching the device.
// `backend` as the ABI's (decode_backend): the re-quantization scheme (0:
// the stored payloads as they are) and the activation terms.
Status model_parse(const uint8_t* data, size_t size, int backend, Model* m);
// Mounts the parsed weights on the device. scheme 0 uses the stored payloads
// as they are (reference behaviour); schemes 1-3 re-quantize each child's
// fp32 weights.
Status model_build(Model* m, hipStream_t st);

// Forward over device buffers. x: [rows][width]; y: output; returns the
// output shape in out_shape. (runtime/forward.cpp:98-156 for Grid,
// stack/stack.cpp:470-494 for Stack.)
Status model_forward(Model& m, const std::vector<int>& in_shape, const float* x,
                     std::vector<int>* out_shape, float* y, size_t y_cap, hipStream_t st);
// The same pass, leaving the output in the model's scratch: *out points to
// it until the next pass on this model. Returns after the stream is idle.
Status model_forward_view(Model& m, const std::vector<int>& in_shape, const float* x,
                          std::vector<int>* out_shape, const float** out, hipStream_t st);

// Segment training of a Stack model of Dense and SwiGLU ops (model_session.cpp:435-507,
// stack.cpp:496-580). model_backward recomputes the forward of x (device)
// and backpropagates gy (device, the output's shape): *gx (input gradient,
// in_shape) and *dw (dW of the ops concatenated in op order, *dw_n floats)
// point into the model's scratch until its next pass. model_apply_sgd
// applies SGD to every op with its slice of dw (device), re-quantizing with
// the model's scheme. MHA children give code 3, other roots code 1.
Status model_backward(Model& m, const std::vector<int>& in_shape, const float* x,
                      const std::vector<int>& gy_shape, const float* gy, const float** gx,
                      const float** dw, size_t* dw_n, hipStream_t st);
Status model_apply_sgd(Model& m, const float* dw, size_t n, double lr, hipStream_t st);
// Segment forward of a Stack (model_session.cpp:420-434, stack.cpp:470-494):
// the last op's pre-activation and the output, both of *shape, in the
// model's scratch. The last op must be Dense here.
Status model_forward_pair(Model& m, const std::vector<int>& in_shape, const float* x,
                          std::vector<int>* shape, const float** pre, const float** post,
                          hipStream_t st);
// Dense proxy of a one-Dense Stack (model_session.cpp:475-493): kind 0 the
// linear input gradient (dense.cpp:141-166, act' = 1), kind 1 dW from the
// given pre-activation, or zeros when pre is null (dense.cpp:168-191). gy
// already has batch * out elements (the caller remaps it).
Status model_dense_proxy(Model& m, int kind, const std::vector<int>& in_shape, const float* x,
                         const float* gy, const float* pre, const float** result, hipStream_t st);

// NWS1 snapshot of all stores (model_session.cpp:523-550).
Status model_export(const Model& m, std::vector<uint8_t>* out);

}  // namespace wv
