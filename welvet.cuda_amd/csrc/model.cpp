// WMN1 model sessions: descriptor parsing, device mount and forward.
//
// Descriptor layout (reference src/interop/model_session.cpp:319-404,
// include/welvet/interop/child_wire.hpp:21-55/:95-118/:153-192/:409-421,
// include/welvet/interop/model_wire.hpp:195-262): little-endian
//   u32 'WMN1', i32 root, i32 count, i32 dims[4], count children,
//   root controls, per-child control trees, i32 store count, stores,
//   and for Grid roots per cell: i32 enabled, remote, tz, ty, tx, tl.
// Store payload (model_session.cpp:135-153): i32 dtype, rows, cols, f32 scale,
//   vec<f32> f32, vec<u8> native, vec<f64> bias (vec = i32 count + items);
//   scaled stores extend it (read_store).
// Only the quantized Dense path is served: Dense, NestedStack, SwiGLU and MHA
// children with FP8/FP4 stores; anything else is reported as code 2/3.
#include "model.h"

#include <cmath>
#include <cstring>
#include <map>
#include <stdexcept>
#include <tuple>
#include <utility>

#include "codec.h"

namespace wv {
namespace {

// Little-endian cursor over the descriptor bytes. Callers name the part of
// the descriptor they are in (`part`), so a descriptor that ends early or
// carries an impossible element count is reported with where it happened.
// Every failure is std::invalid_argument (status code 1).
class WireIn {
 public:
  WireIn(const uint8_t* data, size_t size) : at_(data), end_(data + size) {}

  size_t remaining() const { return static_cast<size_t>(end_ - at_); }
  const char* part = "header";
  int nesting = 0;

  int32_t i32() { return scalar<int32_t>(); }
  uint32_t u32() { return scalar<uint32_t>(); }
  float f32() { return scalar<float>(); }
  double f64() { return scalar<double>(); }

  // n values of T into dst
  template <class T>
  void fill(T* dst, size_t n) {
    if (n > remaining() / sizeof(T)) ended();
    take(dst, n * sizeof(T));
  }
  // an i32 element count, then that many values of T
  template <class T>
  std::vector<T> counted() {
    const int32_t n = i32();
    if (n < 0 || static_cast<size_t>(n) > remaining() / sizeof(T))
      throw std::invalid_argument(std::string("model descriptor: bad element count in ") + part);
    std::vector<T> out(static_cast<size_t>(n));
    take(out.data(), out.size() * sizeof(T));
    return out;
  }

 private:
  template <class T>
  T scalar() {
    T v;
    take(&v, sizeof(T));
    return v;
  }
  void take(void* dst, size_t bytes) {
    if (bytes > remaining()) ended();
    if (bytes) std::memcpy(dst, at_, bytes);
    at_ += bytes;
  }
  [[noreturn]] void ended() const {
    throw std::invalid_argument(std::string("model descriptor ends inside ") + part);
  }
  const uint8_t* at_;
  const uint8_t* end_;
};

void require(bool ok, const char* why) {
  if (!ok) throw std::invalid_argument(why);
}

struct StatusError : std::runtime_error {
  int code;
  explicit StatusError(const Status& s) : std::runtime_error(s.message), code(s.code) {}
};
void good(const Status& s) {
  if (!s) throw StatusError(s);
}

// Element counts implied by a child's dimensions: at most 2^26, and no more
// 4-byte values than the bytes left could hold.
size_t payload_count(const WireIn& r, int64_t n, bool allow_empty) {
  require(n >= 0 && (allow_empty || n > 0) && n <= (int64_t(1) << 26) &&
              static_cast<size_t>(n) <= r.remaining() / 4,
          "invalid model payload size");
  return static_cast<size_t>(n);
}

std::vector<float> weights_f32(WireIn& r, int64_t n) {
  std::vector<float> v(payload_count(r, n, false));
  r.fill(v.data(), v.size());
  return v;
}

void read_child(WireIn& r, ModelNode* c) {
  require(++r.nesting <= 64, "model nesting exceeds 64");
  r.part = "a child operation";
  c->kind = r.i32();
  switch (c->kind) {
  case 0: break;
  case 1: {  // Dense: child_wire.hpp:29-55
    c->in = r.i32();
    c->out = r.i32();
    c->act = r.i32();
    c->dtype = r.i32();
    require(c->in > 0 && c->out > 0, "invalid Dense dims");
    c->W = weights_f32(r, (int64_t)c->out * c->in);
    const uint32_t bl = r.u32();
    std::vector<double> bias(payload_count(r, bl, true));
    r.fill(bias.data(), bias.size());
    WeightStore s;
    s.rows = c->out, s.cols = c->in, s.bias = std::move(bias);
    c->stores.push_back(std::move(s));
    break;
  }
  case 4: {  // SwiGLU: child_wire.hpp:95-118
    c->in = r.i32();
    c->inter = r.i32();
    c->dtype = r.i32();
    require(c->in > 0 && c->inter > 0, "invalid SwiGLU dims");
    const int64_t n = (int64_t)c->in * c->inter;
    std::vector<float> packed = weights_f32(r, 3 * n);
    c->W.assign(packed.begin(), packed.begin() + n);
    c->W2.assign(packed.begin() + n, packed.begin() + 2 * n);
    c->W3.assign(packed.begin() + 2 * n, packed.end());
    for (int i = 0; i < 3; ++i) {
      WeightStore s;
      s.rows = i < 2 ? c->inter : c->in;
      s.cols = i < 2 ? c->in : c->inter;
      c->stores.push_back(std::move(s));
    }
    break;
  }
  case 7: {  // MHA: child_wire.hpp:153-192
    const int seq = r.i32();
    MHAConfig& g = c->mha_cfg;
    g.d_model = r.i32();
    g.num_heads = r.i32();
    g.num_kv_heads = r.i32();
    g.head_dim = r.i32();
    const int msl = r.i32();
    g.mask = r.i32();
    g.pos = r.i32();
    c->dtype = r.i32();
    require(g.num_heads > 0 && g.d_model > 0 && g.num_kv_heads >= 0 && g.head_dim >= 0,
            "invalid MHA dims");
    const int hd = g.head_dim > 0 ? g.head_dim : g.d_model / g.num_heads;
    const int kvh = g.num_kv_heads > 0 ? g.num_kv_heads : g.num_heads;
    g.max_seq_len = msl > 0 ? msl : seq;
    const int qd = g.num_heads * hd, kvd = kvh * hd;
    c->W = weights_f32(r, (int64_t)qd * g.d_model);
    c->W2 = weights_f32(r, (int64_t)kvd * g.d_model);
    c->W3 = weights_f32(r, (int64_t)kvd * g.d_model);
    c->W4 = weights_f32(r, (int64_t)g.d_model * qd);
    good(mha_validate(&g));
    const int rows[4] = {qd, kvd, kvd, g.d_model}, cols[4] = {g.d_model, g.d_model, g.d_model, qd};
    for (int i = 0; i < 4; ++i) {
      WeightStore s;
      s.rows = rows[i], s.cols = cols[i];
      c->stores.push_back(std::move(s));
    }
    break;
  }
  case 19: {  // NestedStack: child_wire.hpp:409-421
    const int32_t n = r.i32();
    require(n > 0 && n <= 4096, "invalid nested count");
    c->nested.resize((size_t)n);
    for (auto& ch : c->nested) read_child(r, &ch);
    break;
  }
  default:
    --r.nesting;
    throw StatusError(Status::err(kGap, "gap? model child kind " + std::to_string(c->kind) +
                                            " is outside the quantized Dense path"));
  }
  --r.nesting;
}

// Cameral training controls (model_wire.hpp:195-253): parsed for framing and
// validation; they carry no forward semantics.
void skip_controls(WireIn& r) {
  r.part = "the training controls";
  int32_t n = r.i32();
  require(n >= 0 && n <= 4096, "invalid controls");
  for (int i = 0; i < n; ++i) {
    const int32_t m = r.i32();
    require(m >= 0 && m <= 33, "invalid train mode");
  }
  n = r.i32();
  require(n >= 0 && n <= 4096, "invalid controls");
  for (int i = 0; i < n; ++i) (void)r.f64();
  (void)r.f64(), (void)r.f64(), (void)r.f64();
  const int32_t present = r.i32();
  if (!present) return;
  (void)r.i32();
  (void)r.f64();
  const int32_t when = r.i32();
  require(when >= 0 && when <= 3, "invalid sync timing");
  n = r.i32();
  require(n >= 0 && n <= 4096, "invalid controls");
  for (int i = 0; i < n; ++i) (void)r.f64();
  n = r.i32();
  require(n >= 0 && n <= 4096, "invalid controls");
  for (int g = 0; g < n; ++g) {
    const int32_t cnt = r.i32();
    require(cnt >= 0 && cnt <= 4096, "invalid controls");
    for (int i = 0; i < cnt; ++i) (void)r.i32();
  }
  n = r.i32();
  require(n >= 0 && n <= 4096, "invalid controls");
  for (int i = 0; i < 6 * n; ++i) (void)r.i32();
}

void skip_control_tree(WireIn& r, const ModelNode& c) {
  skip_controls(r);
  for (const auto& ch : c.nested) skip_control_tree(r, ch);
}

void collect(ModelNode& c, std::vector<WeightStore*>* out) {
  for (auto& s : c.stores) out->push_back(&s);
  for (auto& ch : c.nested) collect(ch, out);
}

// Store payload (model_session.cpp:135-162): i32 dtype, rows, cols, f32
// scale, vec<f32> f32, vec<u8> native, vec<f64> bias. The reference's FP8 /
// FP4 stores are FormatNone: f32 empty, scale unused (native_codec.cpp:176,
// 534-549). Scaled stores of this library are an additive extension keyed in
// the dtype word: bits 0-7 the DType id, bits 8-15 the scale scheme (0 is
// the reference format, and the only one a reference reader accepts):
//   1  per tensor: `scale` holds s (finite, > 0), f32 empty;
//   2  per output row: f32 holds rows scales (finite);
//   3  E8M0 per 32 inputs: f32 holds rows * ceil(cols / 32) scales, each an
//      exact power of two 2^e, e in [-127, 127] (2^-127 is the subnormal
//      0x00400000).
// The dequantized weight is decode(code) times the scale (times 2^e for
// scheme 3), as the library's own quantizer produces it.
constexpr int32_t kSchemeShift = 8;

int e8m0_of_pow2(float v) {
  const uint32_t u = bits_of(v);
  if (u == 0x00400000u) return -127;
  const uint32_t ex = (u >> 23) & 0xFFu;
  require((u & 0x807FFFFFu) == 0 && ex >= 1 && ex <= 254, "block scale is not a power of two");
  return (int)ex - 127;
}

// One store payload as it sits on the wire, before it is checked against
// the child that owns it.
struct StoreWire {
  int32_t tag = 0, rows = 0, cols = 0;
  float scale = 0.0f;
  std::vector<float> f32;
  std::vector<uint8_t> native;
  std::vector<double> bias;
  int dtype() const { return tag & 0xFF; }
  int scheme() const { return (tag >> kSchemeShift) & 0xFF; }
};

StoreWire take_store(WireIn& r) {
  r.part = "a weight store";
  StoreWire w;
  w.tag = r.i32();
  w.rows = r.i32();
  w.cols = r.i32();
  w.scale = r.f32();
  w.f32 = r.counted<float>();
  w.native = r.counted<uint8_t>();
  w.bias = r.counted<double>();
  return w;
}

// Number of f32 scale values each scheme carries in the store's f32 field.
size_t scales_carried(int scheme, int rows, int cols) {
  if (scheme == kSchemeRow) return static_cast<size_t>(rows);
  if (scheme == kSchemeBlock32) return static_cast<size_t>(rows) * ((cols + 31) / 32);
  return 0;
}

void install_store(StoreWire&& w, WeightStore* s) {
  const int dt = w.dtype(), scheme = w.scheme();
  require(w.tag >= 0 && (w.tag >> 16) == 0 && dt <= 33 && scheme <= kSchemeBlock32,
          "store header: unknown dtype or scale scheme");
  require(w.rows == s->rows && w.cols == s->cols, "store shape differs from its operation");
  require(std::isfinite(w.scale), "store scale is not finite");
  if (dt != kE4M3 && dt != kE5M2 && dt != kFP4)
    throw StatusError(Status::err(kUnsupported, "model store dtype " + std::to_string(dt) +
                                                    " is outside the FP8/FP4 path"));
  const int64_t elems = static_cast<int64_t>(w.rows) * w.cols;
  const size_t code_bytes = dt == kFP4 ? static_cast<size_t>((elems + 1) / 2)
                                       : static_cast<size_t>(elems);
  require(w.native.size() == code_bytes, "store code bytes do not match its shape");
  require(w.f32.size() == scales_carried(scheme, w.rows, w.cols),
          "store scale count does not match its scheme");
  s->dtype = dt;
  s->scheme = scheme;
  s->scale = w.scale;
  s->native = std::move(w.native);
  s->bias = std::move(w.bias);
  s->blk_exp.clear();
  switch (scheme) {
  case kSchemeTensor:
    require(w.scale > 0.0f, "tensor scale must be positive");
    s->row_scale.assign(static_cast<size_t>(w.rows), w.scale);
    break;
  case kSchemeRow:
    for (float v : w.f32) require(std::isfinite(v), "row scale is not finite");
    s->row_scale = std::move(w.f32);
    break;
  default:  // reference stores (scale unused) and E8M0 blocks: unit row scales
    s->row_scale.assign(static_cast<size_t>(w.rows), 1.0f);
    if (scheme == kSchemeBlock32) {
      s->blk_exp.reserve(w.f32.size());
      for (float v : w.f32) s->blk_exp.push_back(static_cast<uint8_t>(e8m0_of_pow2(v) + 127));
    }
    break;
  }
}

void build(ModelNode& c, int scheme, int terms, hipStream_t st) {
  if (terms != kTerms && (c.kind == 4 || c.kind == 7))
    throw StatusError(Status::err(kUnsupported,
                                  "two activation terms are for Dense children, not SwiGLU or MHA"));
  switch (c.kind) {
  case 1: {
    c.dense = std::make_unique<DenseLayer>();
    const WeightStore& s = c.stores[0];
    if (scheme == kSchemeRef) {
      good(dense_build_from_store(c.in, c.out, c.act, s, c.dense.get(), st));
    } else {
      good(dense_build(c.in, c.out, c.act, s.dtype, scheme, c.W.data(), s.bias.data(),
                       s.bias.size(), c.dense.get(), st));
    }
    c.dense->terms = terms;
    break;
  }
  case 4: {
    c.swiglu = std::make_unique<SwiGLULayer>();
    c.swiglu->in = c.in, c.swiglu->inter = c.inter;
    DenseLayer* parts[3] = {&c.swiglu->gate, &c.swiglu->up, &c.swiglu->down};
    const std::vector<float>* ws[3] = {&c.W, &c.W2, &c.W3};
    for (int i = 0; i < 3; ++i) {
      const WeightStore& s = c.stores[(size_t)i];
      if (scheme == kSchemeRef) good(dense_build_from_store(s.cols, s.rows, kLinear, s, parts[i], st));
      else good(dense_build(s.cols, s.rows, kLinear, s.dtype, scheme, ws[i]->data(), s.bias.data(),
                            s.bias.size(), parts[i], st));
    }
    good(swiglu_finish(c.swiglu.get(), st));
    break;
  }
  case 7: {
    c.mha = std::make_unique<MHALayer>();
    c.mha->cfg = c.mha_cfg;
    DenseLayer* parts[4] = {&c.mha->q, &c.mha->k, &c.mha->v, &c.mha->o};
    const std::vector<float>* ws[4] = {&c.W, &c.W2, &c.W3, &c.W4};
    for (int i = 0; i < 4; ++i) {
      const WeightStore& s = c.stores[(size_t)i];
      if (scheme == kSchemeRef) good(dense_build_from_store(s.cols, s.rows, kLinear, s, parts[i], st));
      else good(dense_build(s.cols, s.rows, kLinear, s.dtype, scheme, ws[i]->data(), s.bias.data(),
                            s.bias.size(), parts[i], st));
      parts[i]->terms = terms;
    }
    break;
  }
  case 19:
    for (auto& ch : c.nested) build(ch, scheme, terms, st);
    break;
  default: break;
  }
  // fp32 copies are no longer needed once the device holds the codes
  c.W.clear(), c.W2.clear(), c.W3.clear(), c.W4.clear();
  c.W.shrink_to_fit(), c.W2.shrink_to_fit(), c.W3.shrink_to_fit(), c.W4.shrink_to_fit();
}

// Flattens NestedStack children into the op sequence (stack.cpp:38-57).
void flatten(ModelNode& c, std::vector<ModelNode*>* ops) {
  if (c.kind == 19) {
    for (auto& ch : c.nested) flatten(ch, ops);
  } else if (c.kind != 0) {
    ops->push_back(&c);
  }
}

struct Tensor {
  std::vector<int> shape;
  float* data = nullptr;  // device
  size_t numel() const {
    size_t n = 1;
    for (int d : shape) n *= (size_t)d;
    return n;
  }
};

// Op outputs from the model's scratch, in op order (reused pass after pass).
struct Arena {
  ModelScratch& sc;
  float* get(size_t n) {
    if (sc.next == sc.bufs.size()) sc.bufs.emplace_back();
    DevBuf& b = sc.bufs[sc.next++];
    if (b.bytes < n * sizeof(float)) good(b.alloc(n * sizeof(float)));
    return b.as<float>();
  }
};

// One op (stack.cpp:58ff child_forward) on device tensors; returns post.
// pre_out (Dense) receives the pre-activation (post itself when the layer
// has no epilogue).
Tensor op_forward(ModelNode& c, const Tensor& in, Arena& ar, Workspace* ws, hipStream_t st,
                  Tensor* pre_out = nullptr) {
  Tensor out;
  switch (c.kind) {
  case 1: {
    require(in.shape.size() == 2, "dense: input shape need [batch,in]");
    require(in.shape[1] == c.in, "dense: input width mismatch");
    const int b = in.shape[0];
    out.shape = {b, c.out};
    out.data = ar.get(out.numel());
    float* pre = c.dense->need_epi() ? ar.get(out.numel()) : nullptr;
    if (pre) good(dense_forward(*c.dense, b, in.data, pre, out.data, ws, st));
    else good(dense_forward(*c.dense, b, in.data, out.data, nullptr, ws, st));
    if (pre_out) {
      pre_out->shape = out.shape;
      pre_out->data = pre ? pre : out.data;
    }
    break;
  }
  case 4: {
    int rows = 0;
    if (in.shape.size() == 2) rows = in.shape[0], require(in.shape[1] == c.in, "swiglu: width != InputDim");
    else if (in.shape.size() == 3) rows = in.shape[0] * in.shape[1], require(in.shape[2] == c.in, "swiglu: last dim != InputDim");
    else require(false, "swiglu: need [batch,in] or [batch,seq,in]");
    out.shape = in.shape;
    out.data = ar.get(out.numel());
    float* h = ar.get((size_t)rows * c.inter);
    good(swiglu_forward(*c.swiglu, rows, in.data, h, out.data, ws, st));
    if (pre_out) {
      pre_out->shape = {rows, c.inter};
      pre_out->data = h;
    }
    break;
  }
  case 7: {
    const MHAConfig& g = c.mha->cfg;
    int b = 1, s = 0;
    if (in.shape.size() == 3) b = in.shape[0], s = in.shape[1], require(in.shape[2] == g.d_model, "mha: last dim != d_model");
    else if (in.shape.size() == 2) s = in.shape[0], require(in.shape[1] == g.d_model, "mha: width != d_model");
    else require(false, "mha: need [batch,seq,d] or [seq,d]");
    out.shape = {b, s, g.d_model};
    out.data = ar.get(out.numel());
    float* attn = ar.get((size_t)b * s * g.q_dim());
    good(mha_forward(*c.mha, b, s, in.data, attn, out.data, ws, st));
    break;
  }
  default: require(false, "unsupported op");
  }
  return out;
}

// A Dense op of a serial chain on the split matrix-core path: `ready` when
// the previous op's reduce already wrote the split of `in` to split_buf(ws);
// with `next`, this op's reduce writes next's split to ws->e, and the two
// split buffers are swapped afterwards (ws->e sized for next beforehand, so
// that nothing reallocates a buffer that holds a split).
Tensor dense_chain_op(ModelNode& c, const Tensor& in, Arena& ar, Workspace* ws, hipStream_t st,
                      bool ready, const DenseLayer* next) {
  require(in.shape.size() == 2, "dense: input shape need [batch,in]");
  require(in.shape[1] == c.in, "dense: input width mismatch");
  const int b = in.shape[0];
  const DenseLayer& L = *c.dense;
  Tensor out;
  out.shape = {b, c.out};
  out.data = ar.get(out.numel());
  float* pre = L.need_epi() ? ar.get(out.numel()) : nullptr;
  good(ensure_split(ws, dense_workspace_bytes(L, b)));
  uint8_t* nsplit = nullptr;
  if (next) {
    const size_t need = dense_workspace_bytes(*next, b);
    if (ws->e.bytes < need) good(ws->e.alloc(need));
    nsplit = ws->e.as<uint8_t>();
  }
  if (pre) good(dense_forward_split(L, b, in.data, ready, ws, pre, out.data, st, nullptr, 0, false, nsplit));
  else good(dense_forward_split(L, b, in.data, ready, ws, out.data, nullptr, st, nullptr, 0, false, nsplit));
  if (next) std::swap(ws->b, ws->e);
  return out;
}

// Runs flattened ops in order, each reading the previous one's post.
Tensor ops_forward(const std::vector<ModelNode*>& ops, const Tensor& in, Arena& ar, Workspace* ws,
                   hipStream_t st) {
  Tensor cur = in;
  // consecutive Dense ops that dense_fuses_next admits skip the split launch
  // of the second (stack.cpp:470-494 runs them in this order)
  bool ready = false;
  for (size_t i = 0; i < ops.size(); ++i) {
    ModelNode* op = ops[i];
    ModelNode* nx = i + 1 < ops.size() ? ops[i + 1] : nullptr;
    const bool dense2 = op->kind == 1 && cur.shape.size() == 2;
    const bool fuse = dense2 && nx && nx->kind == 1 &&
                      dense_fuses_next(*op->dense, *nx->dense, cur.shape[0]);
    if (fuse || ready) {
      cur = dense_chain_op(*op, cur, ar, ws, st, ready, fuse ? nx->dense.get() : nullptr);
      ready = fuse;
    } else {
      cur = op_forward(*op, cur, ar, ws, st);
    }
  }
  return cur;
}

Tensor stack_forward(std::vector<ModelNode>& children, const Tensor& in, Arena& ar, Workspace* ws,
                     hipStream_t st) {
  std::vector<ModelNode*> ops;
  for (auto& c : children) flatten(c, &ops);
  return ops_forward(ops, in, ar, ws, st);
}

}  // namespace

Status model_parse(const uint8_t* data, size_t size, int backend, Model* m) {
  try {
    require(data && size >= 28 && size <= (1ull << 32), "invalid mount arguments");
    int scheme = 0, terms = kTerms;
    WV_TRY(decode_backend(backend, &scheme, &terms));
    WireIn r(data, size);
    require(r.u32() == 0x314e4d57u, "unsupported model descriptor version");
    m->root = r.i32();
    const int count = r.i32();
    require(m->root >= 0 && m->root <= 2 && count > 0 && count <= 4096, "invalid model root/count");
    if (m->root == 1) return Status::err(kGap, "gap? Parallel model root is outside the quantized Dense path");
    for (int& d : m->dims) d = r.i32();
    m->children.resize((size_t)count);
    for (auto& c : m->children) read_child(r, &c);
    skip_controls(r);
    for (auto& c : m->children) skip_control_tree(r, c);
    std::vector<WeightStore*> stores;
    for (auto& c : m->children) collect(c, &stores);
    r.part = "the store list";
    require(r.i32() == (int)stores.size(), "store count mismatch");
    for (WeightStore* s : stores) install_store(take_store(r), s);
    if (m->root == 2) {
      int64_t n = 1;
      for (int d : m->dims) {
        require(d > 0 && d <= 4096 && n <= 4096 / d, "invalid grid dimensions");
        n *= d;
      }
      require(n == count, "grid cell count mismatch");
      m->cells.resize((size_t)count);
      r.part = "the grid cells";
      for (int i = 0; i < count; ++i) {
        GridCell& g = m->cells[(size_t)i];
        g.enabled = r.i32();
        require(!g.enabled || m->children[(size_t)i].kind != 0, "enabled grid cell has no operation");
        g.remote = r.i32() != 0;
        g.tz = r.i32(), g.ty = r.i32(), g.tx = r.i32(), g.tl = r.i32();
        if (g.remote)
          require(g.tz >= 0 && g.tz < m->dims[0] && g.ty >= 0 && g.ty < m->dims[1] && g.tx >= 0 &&
                      g.tx < m->dims[2] && g.tl >= 0 && g.tl < m->dims[3],
                  "invalid remote link");
      }
    }
    require(r.remaining() == 0, "trailing descriptor bytes");
    m->scheme = scheme;
    m->terms = terms;
    return Status::ok();
  } catch (const StatusError& e) {
    return Status::err(e.code, e.what());
  } catch (const std::invalid_argument& e) {
    return Status::err(kInvalid, e.what());
  } catch (const std::exception& e) {
    return Status::err(kInternal, e.what());
  }
}

Status model_build(Model* m, hipStream_t st) {
  try {
    for (auto& c : m->children) build(c, m->scheme, m->terms, st);
    return Status::ok();
  } catch (const StatusError& e) {
    return Status::err(e.code, e.what());
  } catch (const std::invalid_argument& e) {
    return Status::err(kInvalid, e.what());
  } catch (const std::exception& e) {
    return Status::err(kInternal, e.what());
  }
}

Status model_forward_view(Model& m, const std::vector<int>& in_shape, const float* x,
                          std::vector<int>* out_shape, const float** y, hipStream_t st) {
  try {
    m.scratch.next = 0;
    Arena ar{m.scratch};
    Workspace& ws = m.scratch.ws;
    Tensor in;
    in.shape = in_shape;
    in.data = const_cast<float*>(x);
    Tensor out;
    if (m.root == 0) {
      out = stack_forward(m.children, in, ar, &ws, st);
    } else {
      // volume_dense (runtime/forward.cpp:98-156): cells in hop order
      // (z, y, x, l), disabled cells skipped, a remote link reads the post of
      // its target cell recorded earlier in this pass.
      const int L = m.dims[3], C = m.dims[2], R = m.dims[1];
      // per cell when a cell reads a remote link (or holds no op kind,
      // which op_forward rejects)
      bool any = false, remote = false;
      for (size_t i = 0; i < m.children.size(); ++i)
        if (m.cells[i].enabled)
          any = true, remote = remote || m.cells[i].remote || m.children[i].kind == 0;
      require(any, "runtime.forward: grid has no enabled cells with ops");
      std::map<int, Tensor> posts;
      Tensor cur = in;
      if (!remote) {
        // no remote links: every enabled cell reads the previous one's post,
        // so the cells' ops form one chain (fused across cell boundaries
        // like the ops of one stack)
        std::vector<ModelNode*> ops;
        for (size_t i = 0; i < m.children.size(); ++i)
          if (m.cells[i].enabled) flatten(m.children[i], &ops);
        cur = ops_forward(ops, in, ar, &ws, st);
      }
      for (size_t i = 0; remote && i < m.children.size(); ++i) {
        const GridCell& g = m.cells[i];
        if (!g.enabled) continue;
        Tensor src = cur;
        if (g.remote) {
          const int t = ((g.tz * R + g.ty) * C + g.tx) * L + g.tl;
          auto it = posts.find(t);
          require(it != posts.end(), "runtime.forward: remote hop has no recorded activation");
          src = it->second;
        }
        std::vector<ModelNode> one;
        Tensor post;
        ModelNode& c = m.children[i];
        if (c.kind == 19) post = stack_forward(c.nested, src, ar, &ws, st);
        else post = op_forward(c, src, ar, &ws, st);
        posts[(int)i] = post;
        cur = post;
      }
      out = cur;
    }
    *out_shape = out.shape;
    *y = out.data;
    WV_HIP(hipStreamSynchronize(st));
    return Status::ok();
  } catch (const StatusError& e) {
    return Status::err(e.code, e.what());
  } catch (const std::invalid_argument& e) {
    return Status::err(kInvalid, e.what());
  } catch (const std::exception& e) {
    return Status::err(kInternal, e.what());
  }
}

namespace {

// The ops of a Stack model for the segment training calls: Dense and SwiGLU
// (the MHA backward is not part of this library).
std::vector<ModelNode*> train_ops(Model& m) {
  require(m.root == 0, "segment backward expects Stack or Parallel");
  std::vector<ModelNode*> ops;
  for (auto& c : m.children) flatten(c, &ops);
  for (ModelNode* op : ops)
    if (op->kind != 1 && op->kind != 4)
      throw StatusError(Status::err(kGap, "gap? segment backward of MHA children is outside the "
                                          "quantized Dense path of this library"));
  return ops;
}

// Weights of an op in the concatenated dW (stack.cpp:308-330): Dense out*in,
// SwiGLU Gate | Up | Down.
size_t op_grad_w(const ModelNode& op) {
  return op.kind == 1 ? (size_t)op.dense->out * op.dense->in
                      : 3 * (size_t)op.swiglu->gate.out * op.swiglu->gate.in;
}

template <class F>
Status model_guard(F&& fn) {
  try {
    fn();
    return Status::ok();
  } catch (const StatusError& e) {
    return Status::err(e.code, e.what());
  } catch (const std::invalid_argument& e) {
    return Status::err(kInvalid, e.what());
  } catch (const std::exception& e) {
    return Status::err(kInternal, e.what());
  }
}

}  // namespace

Status model_backward(Model& m, const std::vector<int>& in_shape, const float* x,
                      const std::vector<int>& gy_shape, const float* gy, const float** gx,
                      const float** dw, size_t* dw_n, hipStream_t st) {
  return model_guard([&] {
    std::vector<ModelNode*> ops = train_ops(m);
    require(in_shape.size() == 2, "dense: input shape need [batch,in]");
    m.scratch.next = 0;
    Arena ar{m.scratch};
    Workspace& ws = m.scratch.ws;
    // recompute the forward, keeping each op's input and pre-activation
    // (stack.cpp:519-530)
    Tensor cur;
    cur.shape = in_shape;
    cur.data = const_cast<float*>(x);
    std::vector<Tensor> ins, pres;
    for (ModelNode* op : ops) {
      ins.push_back(cur);
      Tensor pre;
      cur = op_forward(*op, cur, ar, &ws, st, &pre);
      pres.push_back(pre);
    }
    require(gy_shape == cur.shape, "segment output gradient shape mismatch");
    size_t total = 0;
    for (ModelNode* op : ops) total += op_grad_w(*op);
    float* dwall = ar.get(total > 0 ? total : 1);
    // backward in reverse (stack.cpp:532-557): op i's input gradient is op
    // i - 1's output gradient; dW slices in op order
    const int b = in_shape[0];
    const float* g = gy;
    size_t off = total;
    for (size_t k = ops.size(); k-- > 0;) {
      off -= op_grad_w(*ops[k]);
      if (ops[k]->kind == 1) {
        DenseLayer& L = *ops[k]->dense;
        float* dpre = ar.get((size_t)b * L.out);
        float* dxk = ar.get((size_t)b * L.in);
        good(dense_backward(L, b, ins[k].data, pres[k].data, nullptr, g, false, dpre, dxk,
                            dwall + off, nullptr, &ws, st));
        g = dxk;
      } else {
        // SwiGLU (swiglu.cpp:156-248): h is the recorded pre, y the op's output
        const SwiGLULayer& L = *ops[k]->swiglu;
        const float* y = k + 1 < ops.size() ? ins[k + 1].data : cur.data;
        float* dxk = ar.get((size_t)b * L.gate.in);
        good(swiglu_backward(L, b, ins[k].data, pres[k].data, y, g, false, dxk, dwall + off,
                             nullptr, &ws, st));
        g = dxk;
      }
    }
    good(hip_status(hipStreamSynchronize(st), "segment backward"));
    *gx = g;
    *dw = dwall;
    *dw_n = total;
  });
}

Status model_forward_pair(Model& m, const std::vector<int>& in_shape, const float* x,
                          std::vector<int>* shape, const float** pre, const float** post,
                          hipStream_t st) {
  return model_guard([&] {
    require(m.root == 0, "segment forward expects Stack or Parallel");
    std::vector<ModelNode*> ops;
    for (auto& c : m.children) flatten(c, &ops);
    m.scratch.next = 0;
    Arena ar{m.scratch};
    Tensor cur;
    cur.shape = in_shape;
    cur.data = const_cast<float*>(x);
    Tensor last_pre = cur;  // no ops: pre = post = input (stack.cpp:476-480)
    for (size_t i = 0; i < ops.size(); ++i) {
      if (i + 1 == ops.size() && ops[i]->kind != 1)
        throw StatusError(Status::err(kGap, "gap? segment forward ending in a SwiGLU / MHA child "
                                            "is outside the quantized Dense path of this library"));
      cur = op_forward(*ops[i], cur, ar, &m.scratch.ws, st, i + 1 == ops.size() ? &last_pre : nullptr);
    }
    good(hip_status(hipStreamSynchronize(st), "segment forward"));
    *shape = cur.shape;
    *pre = last_pre.data;
    *post = cur.data;
  });
}

Status model_dense_proxy(Model& m, int kind, const std::vector<int>& in_shape, const float* x,
                         const float* gy, const float* pre, const float** result, hipStream_t st) {
  return model_guard([&] {
    require(m.root == 0 && m.children.size() == 1 && m.children[0].kind == 1,
            "proxy expects one Dense");
    require(kind == 0 || kind == 1, "invalid Dense proxy arguments");
    DenseLayer& L = *m.children[0].dense;
    require(in_shape.size() == 2 && in_shape[0] > 0, "dense: proxy input shape");
    if (kind == 0) require(in_shape[1] == L.in, "dense: LinearGradIn shape");
    const int b = in_shape[0];
    m.scratch.next = 0;
    Arena ar{m.scratch};
    float* dpre = ar.get((size_t)b * L.out);
    float* dx = ar.get((size_t)b * L.in);
    float* dw = ar.get((size_t)L.out * L.in);
    const float* use_pre = pre;
    if (!use_pre) {  // zeros (dense.cpp:160, :183-187)
      float* z = ar.get((size_t)b * L.out);
      good(hip_status(hipMemsetAsync(z, 0, (size_t)b * L.out * sizeof(float), st), "proxy pre"));
      use_pre = z;
    }
    good(dense_backward(L, b, x, use_pre, nullptr, gy, false, dpre, dx, dw, nullptr,
                        &m.scratch.ws, st, kind == 0));
    good(hip_status(hipStreamSynchronize(st), "dense proxy"));
    *result = kind == 0 ? dx : dw;
  });
}

Status model_apply_sgd(Model& m, const float* dw, size_t n, double lr, hipStream_t st) {
  return model_guard([&] {
    std::vector<ModelNode*> ops = train_ops(m);
    size_t total = 0;
    for (ModelNode* op : ops) total += op_grad_w(*op);
    require(n == total, "segment weight gradient size mismatch");
    size_t off = 0;
    for (ModelNode* op : ops) {
      if (op->kind == 1) good(dense_apply_sgd(op->dense.get(), dw + off, lr, st));
      else good(swiglu_apply_sgd(op->swiglu.get(), dw + off, lr, st));
      off += op_grad_w(*op);
    }
  });
}

Status model_forward(Model& m, const std::vector<int>& in_shape, const float* x,
                     std::vector<int>* out_shape, float* y, size_t y_cap, hipStream_t st) {
  const float* out = nullptr;
  WV_TRY(model_forward_view(m, in_shape, x, out_shape, &out, st));
  size_t n = 1;
  for (int d : *out_shape) n *= (size_t)d;
  if (n > y_cap) return Status::err(kInvalid, "model forward: output buffer too small");
  WV_HIP(hipMemcpyAsync(y, out, n * sizeof(float), hipMemcpyDeviceToDevice, st));
  WV_HIP(hipStreamSynchronize(st));
  return Status::ok();
}

namespace {
// The extended store payload of read_store (scheme 0: the reference format).
void write_store(std::vector<uint8_t>* w, const WeightStore& s) {
  auto put = [&](const void* p, size_t n) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    w->insert(w->end(), b, b + n);
  };
  const int32_t hdr[3] = {s.dtype | (s.scheme << kSchemeShift), s.rows, s.cols};
  put(hdr, sizeof hdr);
  put(&s.scale, 4);
  std::vector<float> f;
  if (s.scheme == kSchemeRow) {
    f = s.row_scale;
  } else if (s.scheme == kSchemeBlock32) {
    f.resize(s.blk_exp.size());
    for (size_t i = 0; i < f.size(); ++i) f[i] = pow2f((int)s.blk_exp[i] - 127);
  }
  const int32_t nf = (int32_t)f.size();
  put(&nf, 4);
  put(f.data(), f.size() * sizeof(float));
  const int32_t nn = (int32_t)s.native.size();
  put(&nn, 4);
  put(s.native.data(), s.native.size());
  const int32_t nb = (int32_t)s.bias.size();
  put(&nb, 4);
  put(s.bias.data(), s.bias.size() * sizeof(double));
}
void collect_layers(const ModelNode& c, std::vector<const WeightStore*>* out) {
  switch (c.kind) {
  case 1: out->push_back(&c.dense->store); break;
  case 4:
    out->push_back(&c.swiglu->gate.store), out->push_back(&c.swiglu->up.store),
        out->push_back(&c.swiglu->down.store);
    break;
  case 7:
    out->push_back(&c.mha->q.store), out->push_back(&c.mha->k.store),
        out->push_back(&c.mha->v.store), out->push_back(&c.mha->o.store);
    break;
  case 19:
    for (const auto& ch : c.nested) collect_layers(ch, out);
    break;
  default: break;
  }
}
}  // namespace

Status model_export(const Model& m, std::vector<uint8_t>* out) {
  std::vector<const WeightStore*> stores;
  for (const auto& c : m.children) collect_layers(c, &stores);
  out->clear();
  const uint32_t magic = 0x3153574eu;
  out->insert(out->end(), reinterpret_cast<const uint8_t*>(&magic),
              reinterpret_cast<const uint8_t*>(&magic) + 4);
  const int32_t n = (int32_t)stores.size();
  out->insert(out->end(), reinterpret_cast<const uint8_t*>(&n), reinterpret_cast<const uint8_t*>(&n) + 4);
  for (const WeightStore* s : stores) write_store(out, *s);
  const int32_t extras = 0;
  out->insert(out->end(), reinterpret_cast<const uint8_t*>(&extras),
              reinterpret_cast<const uint8_t*>(&extras) + 4);
  return Status::ok();
}

}  // namespace wv
