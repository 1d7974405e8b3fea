// Dense / SwiGLU / MHA layers over device-resident quantized weights.
//
// Reference call structure kept: Dense is the hub (src/layers/dense/dense.cpp:
// 10-86); SwiGLU = Gate, Up (Linear, no bias), SiLU product, Down
// (src/layers/swiglu/swiglu.cpp:87-136); MHA = Q/K/V projections on
// [batch*seq, d], attention core, O projection (src/layers/mha/mha.cpp:123-183).
// Unlike the reference, weights are quantized once on the device and stay
// there; activations stay on the device between the layer's kernels.
#include "layers.h"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "codec.h"

namespace wv {

Status check_dtype_scheme(int dtype, int scheme) {
  if (dtype != kE4M3 && dtype != kE5M2 && dtype != kFP4) {
    return Status::err(kUnsupported, "dtype " + std::to_string(dtype) +
                                         " is outside the FP8/FP4 path (supported: 4, 5, 16)");
  }
  if (scheme < kSchemeRef || scheme > kSchemeBlock32)
    return Status::err(kInvalid, "backend (scale scheme) must be 0..3");
  return Status::ok();
}

Status decode_backend(int backend, int* scheme, int* terms) {
  if (backend < 0 || (backend & ~(kBackendTwoTerms | kBackendOneTerm | 0xF)) != 0 ||
      (backend & 0xF) > kSchemeBlock32 ||
      (backend & (kBackendTwoTerms | kBackendOneTerm)) == (kBackendTwoTerms | kBackendOneTerm))
    return Status::err(kInvalid, "backend: scale scheme 0..3, plus 16 for two activation terms "
                                 "or 32 for one");
  *scheme = backend & 0xF;
  *terms = (backend & kBackendOneTerm) ? 1 : (backend & kBackendTwoTerms) ? 2 : kTerms;
  return Status::ok();
}

static Status download_store(DenseLayer* L, const uint8_t* d_raw, hipStream_t st) {
  WeightStore& s = L->store;
  const DeviceWeights& d = L->dev;
  const int64_t n = (int64_t)d.rows * d.cols;
  s.native.resize(d.dtype == kFP4 ? (size_t)((n + 1) / 2) : (size_t)n);
  if (d_raw) WV_TRY(copy_d2h(s.native.data(), d_raw, s.native.size(), st));
  s.row_scale.resize((size_t)d.rows);
  WV_TRY(copy_d2h(s.row_scale.data(), d.d_scale(), (size_t)d.rows * sizeof(float), st));
  if (d.scheme == kSchemeBlock32) {
    // the device rows are nblk (padded) bytes long; the store keeps ceil(cols / 32)
    const int nb = (d.cols + 31) / 32;
    std::vector<uint8_t> padded((size_t)d.rows * d.nblk);
    WV_TRY(copy_d2h(padded.data(), d.d_blk(), padded.size(), st));
    s.blk_exp.resize((size_t)d.rows * nb);
    for (int r = 0; r < d.rows; ++r)
      std::memcpy(s.blk_exp.data() + (size_t)r * nb, padded.data() + (size_t)r * d.nblk, nb);
  } else {
    s.blk_exp.clear();
  }
  s.scale = (d.scheme == kSchemeTensor && !s.row_scale.empty()) ? s.row_scale[0] : 1.0f;
  return Status::ok();
}

static Status upload_bias(DenseLayer* L, const double* bias, size_t bias_len, hipStream_t st) {
  L->store.bias.assign(bias ? bias : nullptr, bias ? bias + bias_len : nullptr);
  L->bias_len = (bias && bias_len > 0) ? (int)bias_len : 0;
  L->bias_dev.reset();
  if (L->bias_len > 0) {
    WV_TRY(L->bias_dev.alloc(bias_len * sizeof(double)));
    WV_TRY(copy_h2d(L->bias_dev.p, bias, bias_len * sizeof(double), st));
    WV_HIP(hipStreamSynchronize(st));
  }
  return Status::ok();
}

Status dense_build(int in, int out, int act, int dtype, int scheme, const float* W_host,
                   const double* bias, size_t bias_len, DenseLayer* L, hipStream_t st) {
  if (!L) return Status::err(kInvalid, "dense: null layer");
  if (in <= 0 || out <= 0) return Status::err(kInvalid, "dense: bad dims");
  if (!act_valid(act)) return Status::err(kInvalid, "dense: bad activation");
  WV_TRY(check_dtype_scheme(dtype, scheme));
  L->in = in, L->out = out, L->act = act;
  L->store.dtype = dtype, L->store.scheme = scheme, L->store.rows = out, L->store.cols = in;
  const int64_t n = (int64_t)in * out;
  DevBuf dW, raw;
  WV_TRY(dW.alloc((size_t)n * sizeof(float)));
  if (W_host) {
    WV_TRY(copy_h2d(dW.p, W_host, (size_t)n * sizeof(float), st));
  } else {
    WV_HIP(hipMemsetAsync(dW.p, 0, (size_t)n * sizeof(float), st));
  }
  WV_TRY(raw.alloc(dtype == kFP4 ? (size_t)((n + 1) / 2) : (size_t)n));
  WV_TRY(quantize_to_device(dW.as<float>(), dtype, scheme, out, in, &L->dev, raw.as<uint8_t>(), st));
  WV_TRY(download_store(L, raw.as<uint8_t>(), st));
  return upload_bias(L, bias, bias_len, st);
}

Status dense_build_from_store(int in, int out, int act, const WeightStore& store, DenseLayer* L,
                              hipStream_t st) {
  if (!L) return Status::err(kInvalid, "dense: null layer");
  if (in <= 0 || out <= 0 || store.rows != out || store.cols != in)
    return Status::err(kInvalid, "dense: store shape mismatch");
  if (!act_valid(act)) return Status::err(kInvalid, "dense: bad activation");
  WV_TRY(check_dtype_scheme(store.dtype, store.scheme));
  const int64_t n = (int64_t)in * out;
  const size_t nbytes = store.dtype == kFP4 ? (size_t)((n + 1) / 2) : (size_t)n;
  if (store.native.size() != nbytes) return Status::err(kInvalid, "dense: native payload length");
  const int nb = (in + 31) / 32;
  if (store.scheme == kSchemeBlock32 && store.blk_exp.size() != (size_t)out * nb)
    return Status::err(kInvalid, "dense: block scale length");
  if ((store.scheme == kSchemeRow || store.scheme == kSchemeTensor) &&
      store.row_scale.size() != (size_t)out)
    return Status::err(kInvalid, "dense: row scale length");
  L->in = in, L->out = out, L->act = act;
  L->store = store;
  DevBuf raw, sc, blk;
  WV_TRY(raw.alloc(nbytes));
  WV_TRY(copy_h2d(raw.p, store.native.data(), nbytes, st));
  const float* d_sc = nullptr;
  if (!store.row_scale.empty()) {
    WV_TRY(sc.alloc(store.row_scale.size() * sizeof(float)));
    WV_TRY(copy_h2d(sc.p, store.row_scale.data(), store.row_scale.size() * sizeof(float), st));
    d_sc = sc.as<float>();
  }
  const uint8_t* d_blk = nullptr;
  if (store.scheme == kSchemeBlock32) {
    WV_TRY(blk.alloc(store.blk_exp.size()));
    WV_TRY(copy_h2d(blk.p, store.blk_exp.data(), store.blk_exp.size(), st));
    d_blk = blk.as<uint8_t>();
  }
  WV_TRY(relayout_to_device(raw.as<uint8_t>(), store.dtype, store.scheme, out, in, d_sc, d_blk,
                            &L->dev, st));
  if (store.row_scale.empty()) L->store.row_scale.assign((size_t)out, 1.0f);
  return upload_bias(L, store.bias.data(), store.bias.size(), st);
}

static FmtArgs format_args(const DenseLayer& L) {
  FmtArgs a;
  a.q = L.fw.q.as<const uint8_t>();
  a.h = L.fw.h.as<const uint8_t>();
  a.s = L.fw.s.as<const uint8_t>();
  a.e = L.fw.e.as<const uint8_t>();
  a.rows = L.out;
  a.cols = L.in;
  a.nsub = L.fw.nsub;
  return a;
}

Status dense_build_format(int in, int out, int act, int format, const float* W_host,
                          const uint8_t* blocks, size_t blocks_len, const double* bias,
                          size_t bias_len, DenseLayer* L, hipStream_t st) {
  if (!L) return Status::err(kInvalid, "dense: null layer");
  if (in <= 0 || out <= 0) return Status::err(kInvalid, "dense: bad dims");
  if (!act_valid(act)) return Status::err(kInvalid, "dense: bad activation");
  const FmtGeom G = fmt_geom(format);
  if (G.qk == 0) {
    if (format > kFmtNone && format <= kFmtLast)
      return Status::err(kGap, "gap? quant format " + std::to_string(format) + " not implemented");
    return Status::err(kInvalid, "dense: quant format out of range");
  }
  if (in % G.qk) return Status::err(kInvalid, "dense: in must be a multiple of the format's block");
  if ((W_host == nullptr) == (blocks == nullptr))
    return Status::err(kInvalid, "dense: give either fp32 weights or packed blocks");
  const int64_t n = (int64_t)in * out;
  const size_t nbytes = (size_t)(n / G.qk) * G.bb;
  if (blocks && blocks_len != nbytes) return Status::err(kInvalid, "dense: packed block length");
  L->in = in, L->out = out, L->act = act, L->format = format;
  FormatWeights& f = L->fw;
  f.format = format, f.rows = out, f.cols = in, f.rpad = (int)round_up(out, 16), f.nsub = in / 32;
  DevBuf packed;
  WV_TRY(packed.alloc(nbytes));
  if (W_host) {
    DevBuf dW;
    WV_TRY(dW.alloc((size_t)n * sizeof(float)));
    WV_TRY(copy_h2d(dW.p, W_host, (size_t)n * sizeof(float), st));
    WV_TRY(format_quantize(format, dW.as<float>(), n, packed.as<uint8_t>(), st));
    WV_HIP(hipStreamSynchronize(st));
  } else {
    WV_TRY(copy_h2d(packed.p, blocks, nbytes, st));
  }
  const size_t subs = (size_t)f.rpad * f.nsub;
  WV_TRY(f.q.alloc(subs * G.qb));
  WV_HIP(hipMemsetAsync(f.q.p, 0, f.q.bytes, st));
  WV_TRY(f.s.alloc(subs * G.sb));
  WV_HIP(hipMemsetAsync(f.s.p, 0, f.s.bytes, st));
  f.h.reset();
  f.e.reset();
  if (G.hb) {
    WV_TRY(f.h.alloc(subs * G.hb));
    WV_HIP(hipMemsetAsync(f.h.p, 0, f.h.bytes, st));
  }
  if (G.eb) {
    WV_TRY(f.e.alloc(subs / 8 * G.eb));
    WV_HIP(hipMemsetAsync(f.e.p, 0, f.e.bytes, st));
  }
  WV_TRY(format_relayout(format, format_args(*L), packed.as<uint8_t>(), out, st));
  f.blocks.resize(nbytes);
  WV_TRY(copy_d2h(f.blocks.data(), packed.p, nbytes, st));
  WV_HIP(hipStreamSynchronize(st));
  L->store = WeightStore{};
  L->store.rows = out, L->store.cols = in;
  return upload_bias(L, bias, bias_len, st);
}

Status dense_export_f32(const DenseLayer& L, float* w, hipStream_t st) {
  if (!w) return Status::err(kInvalid, "dense export: null buffer");
  if (L.format) return format_dequant(L.format, format_args(L), L.out, w, st);
  return launch_dequant(L.dev, w, st);
}

static Status format_forward(const DenseLayer& L, int batch, const float* x, float* pre,
                             float* post, hipStream_t st) {
  FmtArgs a = format_args(L);
  a.x = x;
  a.x_stride = L.in;
  a.pre = pre;
  a.post = post;
  a.out_stride = L.out;
  a.act = L.act;
  a.need_epi = L.need_epi();
  a.bias = L.bias_dev.as<const double>();
  a.bias_len = L.bias_len;
  return launch_format_gemv(L.format, a, batch, st);
}

int gemv_batch_limit() { return 1 << 30; }

static GemvTile tile_for(const DeviceWeights& d, int mats) {
  return gemv_tile(d.dtype, d.kpad, d.rows, mats, cu_count());
}

static GemvArgs gemv_args(const DenseLayer& L, const float* x, int x_stride) {
  GemvArgs a;
  a.codes[0] = L.dev.d_codes();
  a.scale[0] = L.dev.d_scale();
  a.blk[0] = L.dev.d_blk();
  a.pitch = L.dev.pitch;
  a.nblk = L.dev.nblk;
  a.kpad = L.dev.kpad;
  a.cols = L.in;
  a.rows = L.out;
  a.x = x;
  a.x_stride = x_stride;
  a.out_stride = L.out;
  a.act = L.act;
  a.need_epi = L.need_epi() ? 1 : 0;
  a.bias = L.bias_dev.as<const double>();
  a.bias_len = L.bias_len;
  return a;
}

static MxvArgs mxv_args(const DenseLayer& L, const float* x, int x_stride, int batch) {
  MxvArgs a;
  a.codes[0] = L.dev.d_codes();
  a.scale[0] = L.dev.d_scale();
  a.blk[0] = L.dev.d_blk();
  a.pitch = L.dev.pitch;
  a.nblk = L.dev.nblk;
  a.kpad = L.dev.kpad;
  a.cols = L.in;
  a.rows = L.out;
  a.x = x;
  a.x_stride = x_stride;
  a.batch = batch;
  a.out_stride = L.out;
  a.act = L.act;
  a.need_epi = L.need_epi() ? 1 : 0;
  a.bias = L.bias_dev.as<const double>();
  a.bias_len = L.bias_len;
  return a;
}

bool uses_split(int batch) { return batch > kMxvMaxBatch; }

// 1-4-row products on the matrix cores over operand-order weights
// (gemv_mx.hip): large enough to fill the GPU with 16-row workgroups, and
// without weight rows holding non-finite codes (whose products the matrix
// cores would turn into NaN where the reference gives inf).
static bool mx_dense(const DenseLayer& L, int batch) {
  return !L.format && L.dev.nf_count() == 0 && gemv_mx_fits(L.dev.dtype, L.out, L.dev.kpad, 1, batch);
}

static bool mx_pair(const SwiGLULayer& L, int rows) {
  return !L.gate.format && !L.up.format && L.gate.dev.nf_count() == 0 && L.up.dev.nf_count() == 0 &&
         gemv_mx_fits(L.gate.dev.dtype, L.inter, L.gate.dev.kpad, 2, rows);
}

static Status build_frag(DenseLayer* L, hipStream_t st) {
  if (L->dev.codes_frag.p) return Status::ok();
  WV_TRY(build_codes_frag(&L->dev, st));
  return hip_status(hipStreamSynchronize(st), "codes_frag");
}

Status dense_prepare_rows(DenseLayer* L, int batch, hipStream_t st) {
  if (L->format) return Status::ok();
  if ((uses_split(batch) && mxg_block_m(batch) == 16) || mx_dense(*L, batch)) return build_frag(L, st);
  return Status::ok();
}

Status swiglu_prepare_rows(SwiGLULayer* L, int rows, hipStream_t st) {
  if (mx_pair(*L, rows)) {
    WV_TRY(build_frag(&L->gate, st));
    WV_TRY(build_frag(&L->up, st));
  } else {
    WV_TRY(dense_prepare_rows(&L->gate, rows, st));
    WV_TRY(dense_prepare_rows(&L->up, rows, st));
  }
  return dense_prepare_rows(&L->down, rows, st);
}

// The kernel reads x as 16-byte vectors.
static bool mx_vec(const DenseLayer& L, const float* x) {
  return L.in % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

static GemvMxArgs mx_args(const DenseLayer& L, const float* x, int batch) {
  GemvMxArgs a;
  a.nb = batch;
  a.codesf[0] = L.dev.d_codesf();
  a.blkf[0] = L.dev.d_blkf();
  a.scale[0] = L.dev.d_scale();
  a.kpad = L.dev.kpad;
  a.cols = L.in;
  a.rows = L.out;
  a.x = x;
  a.act = L.act;
  a.need_epi = L.need_epi() ? 1 : 0;
  a.bias = L.bias_dev.as<const double>();
  a.bias_len = L.bias_len;
  return a;
}

// Split activations plus, for small batches split along K, the partial sums.
static size_t gemm_ws_bytes(const DenseLayer& L, int batch, int mats) {
  return split_bytes(batch, L.dev.kpad) + mxg_part_bytes(batch, L.dev.kpad, L.out, mats);
}

size_t dense_workspace_bytes(const DenseLayer& L, int batch) {
  if (L.format) return 0;
  return uses_split(batch) ? gemm_ws_bytes(L, batch, 1) : 0;
}

Status ensure_split(Workspace* ws, size_t n) {
  if (!ws) return Status::err(kInvalid, "workspace: null");
  if (ws->b.bytes < n) WV_TRY(ws->b.alloc(n));
  return Status::ok();
}

static MxgArgs mxg_args(const DenseLayer& L, int batch, const uint8_t* split) {
  MxgArgs p;
  p.M = batch;
  p.mpad = (int)round_up(batch, mxg_block_m(batch));
  p.a = split;
  p.as = split + (size_t)kTerms * p.mpad * L.dev.kpad;
  p.codes[0] = L.dev.d_codes();
  p.scale[0] = L.dev.d_scale();
  p.blk[0] = L.dev.d_blk();
  p.blkf[0] = L.dev.d_blkf();
  p.codesf[0] = L.dev.d_codesf();
  p.pitch = L.dev.pitch;
  p.nblk = L.dev.nblk;
  p.kpad = L.dev.kpad;
  p.N = L.out;
  p.out_stride = L.out;
  p.act = L.act;
  p.need_epi = L.need_epi() ? 1 : 0;
  p.bias = L.bias_dev.as<const double>();
  p.bias_len = L.bias_len;
  // the partial sums follow the split terms (gemm_ws_bytes)
  p.part = reinterpret_cast<float*>(const_cast<uint8_t*>(split) + split_bytes(batch, L.dev.kpad));
  // one activation term is built for the large-tile kernels only (more
  // than 32 rows); 5..32 rows of such a layer (a model forward, the
  // allocation-free execute) take the default terms
  p.terms = (L.terms == 1 && mxg_block_m(batch) == 16) ? kTerms : L.terms;
  return p;
}

// The fp32 input of a small-M GEMM, which splits it itself.
static void set_input(MxgArgs& p, const float* x, int stride, int cols) {
  p.x = x;
  p.x_stride = stride;
  p.cols = cols;
  p.x_vec = stride % 4 == 0 && cols % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

// Rows with non-finite codes, recomputed after a matrix-core product of
// `batch` rows of x (row stride x_stride).
static Status fix_nonfinite(const DenseLayer& L, int batch, const float* x, int x_stride,
                            float* pre, float* post, hipStream_t st) {
  if (L.dev.nf_count() == 0) return Status::ok();
  NfArgs a;
  a.rows = L.dev.nf_rows.as<const int>();
  a.n = L.dev.nf_count();
  a.dtype = L.dev.dtype;
  a.codes[0] = L.dev.d_codes();
  a.scale[0] = L.dev.d_scale();
  a.blk[0] = L.dev.d_blk();
  a.pitch = L.dev.pitch;
  a.nblk = L.dev.nblk;
  a.cols = L.in;
  a.x = x;
  a.x_stride = x_stride;
  a.batch = batch;
  a.pre = pre;
  a.post = post;
  a.out_stride = L.out;
  a.act = L.act;
  a.need_epi = L.need_epi() ? 1 : 0;
  a.bias = L.bias_dev.as<const double>();
  a.bias_len = L.bias_len;
  return launch_nf_fix(a, st);
}

Status dense_forward_split(const DenseLayer& L, int batch, const float* x, bool split_ready,
                           Workspace* ws, float* pre, float* post, hipStream_t st,
                           const double* rope_tab, int rope_hd, bool keep_out,
                           uint8_t* next_split) {
  MxgArgs p = mxg_args(L, batch, split_buf(ws));
  p.pre = pre;
  p.post = post;
  p.next = next_split;
  p.keep_out = keep_out ? 1 : 0;
  p.rope_tab = rope_tab;
  p.rope_hd = rope_hd;
  if (mxg_block_m(batch) > 16) {
    if (!split_ready)
      WV_TRY(launch_split(x, L.in, batch, L.in, L.dev.kpad, split_buf(ws), st, L.terms));
  } else {
    set_input(p, x, L.in, L.in);
  }
  WV_TRY(launch_mxg(p, L.dev.dtype, L.dev.scheme == kSchemeBlock32, st));
  return fix_nonfinite(L, batch, x, L.in, pre, post, st);
}

bool dense_fuses_next(const DenseLayer& L, const DenseLayer& next, int batch) {
  return !L.format && !next.format && mxg_block_m(batch) > 16 && L.dev.nf_count() == 0 &&
         L.out % 256 == 0 && next.in == L.out && next.dev.kpad == L.out &&
         next.terms == L.terms && mxg_part_bytes(batch, L.dev.kpad, L.out, 1) > 0;
}

Status dense_forward(const DenseLayer& L, int batch, const float* x, float* pre, float* post,
                     Workspace* ws, hipStream_t st) {
  if (batch <= 0 || !x || !pre) return Status::err(kInvalid, "dense forward: bad args");
  if (L.need_epi() && !post) return Status::err(kInvalid, "dense forward: post needed");
  // packed block formats: the GEMV over every batch row
  if (L.format) return format_forward(L, batch, x, pre, post, st);
  if (mx_dense(L, batch) && L.dev.codes_frag.p && mx_vec(L, x)) {
    GemvMxArgs m = mx_args(L, x, batch);
    m.pre = pre;
    m.post = post;
    return launch_gemv_mx(m, L.dev.dtype, L.dev.scheme == kSchemeBlock32, st);
  }
  if (uses_split(batch)) {
    WV_TRY(ensure_split(ws, gemm_ws_bytes(L, batch, 1)));
    return dense_forward_split(L, batch, x, false, ws, pre, post, st);
  }
  if (batch >= 2 && batch <= kMxvMaxBatch) {
    MxvArgs m = mxv_args(L, x, L.in, batch);
    m.pre = pre;
    m.post = post;
    WV_TRY(launch_mxv(m, L.dev.dtype, L.dev.scheme == kSchemeBlock32, st));
    return fix_nonfinite(L, batch, x, L.in, pre, post, st);
  }
  GemvArgs a = gemv_args(L, x, L.in);
  a.pre = pre;
  a.post = post;
  return launch_gemv(a, L.dev.dtype, L.dev.scheme == kSchemeBlock32, batch, tile_for(L.dev, 1),
                     st);
}

// ---------------------------------------------------------------------------
Status dense_backward(const DenseLayer& L, int batch, const float* x, const float* pre,
                      const float* post, const float* g, bool use_target, float* dpre, float* dx,
                      float* dw, double* loss_part, Workspace* ws, hipStream_t st,
                      bool linear_act) {
  if (batch <= 0 || !x || !pre || !g || !dpre || !dx || !dw || !ws || (use_target && !post))
    return Status::err(kInvalid, "dense backward: bad args");
  if (L.format) return Status::err(kGap, "gap? dense backward over packed block formats");
  const int64_t n = (int64_t)batch * L.out;
  // Linear without a target: d_pre = gy, stored by the products' launch
  const bool direct = !use_target && (linear_act || L.act == kLinear);
  if (!direct)
    WV_TRY(launch_dpre(g, post, pre, linear_act ? kLinear : L.act, use_target ? 1 : 0, n, dpre,
                       loss_part, st));
  const size_t pb = gemvt_part_bytes(L.in, L.out);
  if (ws->d.bytes < pb) WV_TRY(ws->d.alloc(pb));
  GemvtArgs a;
  a.codes = L.dev.d_codes();
  a.scale = L.dev.d_scale();
  a.blk = L.dev.d_blk();
  a.pitch = L.dev.pitch;
  a.nblk = L.dev.nblk;
  a.kpad = L.dev.kpad;
  a.in = L.in;
  a.out = L.out;
  a.dpre = direct ? g : dpre;
  // (d_pre in gy's own buffer already holds it)
  float* dpre_out = direct && dpre != g ? dpre : nullptr;
  return launch_backward_products(a, L.dev.dtype, L.dev.scheme == kSchemeBlock32, batch, x, dw,
                                  ws->d.as<double>(), dx, dpre_out, st);
}

template <class G>
static Status apply_sgd_impl(DenseLayer* L, const G* dw, double lr, hipStream_t st) {
  if (!L || !dw) return Status::err(kInvalid, "dense sgd: bad args");
  if (L->format) return Status::err(kGap, "gap? SGD on packed block formats");
  const int64_t n = (int64_t)L->in * L->out;
  DevBuf next, raw;
  WV_TRY(next.alloc((size_t)n * sizeof(float)));
  WV_TRY(launch_sgd(L->dev, dw, lr, next.as<float>(), st));
  WV_TRY(raw.alloc(L->dev.dtype == kFP4 ? (size_t)((n + 1) / 2) : (size_t)n));
  DeviceWeights fresh;
  WV_TRY(quantize_to_device(next.as<float>(), L->dev.dtype, L->dev.scheme, L->out, L->in, &fresh,
                            raw.as<uint8_t>(), st));
  if (L->dev.codes_frag.p) WV_TRY(build_codes_frag(&fresh, st));
  L->dev = std::move(fresh);
  return download_store(L, raw.as<uint8_t>(), st);
}

Status dense_apply_sgd(DenseLayer* L, const float* dw, double lr, hipStream_t st) {
  return apply_sgd_impl(L, dw, lr, st);
}

Status dense_apply_sgd(DenseLayer* L, const double* dw, double lr, hipStream_t st) {
  return apply_sgd_impl(L, dw, lr, st);
}

std::vector<float> remap_len(const float* src, size_t sn, size_t need) {
  std::vector<float> out(need, 0.0f);
  if (sn == 0 || need == 0) return out;
  if (sn == need) {
    std::memcpy(out.data(), src, need * sizeof(float));
    return out;
  }
  for (size_t i = 0; i < need; ++i) {
    size_t lo = i * sn / need, hi = (i + 1) * sn / need;
    if (hi <= lo) hi = lo + 1;
    if (hi > sn) hi = sn;
    double sum = 0.0;
    for (size_t j = lo; j < hi; ++j) sum += (double)src[j];
    out[i] = (float)(sum / (double)(hi - lo));
  }
  return out;
}

Status store_quantize(int rows, int cols, int dtype, int scheme, const float* W_host,
                      WeightStore* out, hipStream_t st) {
  if (!out) return Status::err(kInvalid, "weights: null store");
  DenseLayer L;
  WV_TRY(dense_build(cols, rows, kLinear, dtype, scheme, W_host, nullptr, 0, &L, st));
  *out = std::move(L.store);
  out->bias.clear();
  return Status::ok();
}

Status store_decode_rows(const StoreView& s, int row0, int nrows, float* host_out,
                         hipStream_t st) {
  if (!host_out || row0 < 0 || nrows < 0 || row0 + nrows > s.rows || s.cols <= 0)
    return Status::err(kInvalid, "weights: decode rows out of range");
  WV_TRY(check_dtype_scheme(s.dtype, s.scheme));
  if (nrows == 0) return Status::ok();
  const int64_t e0 = (int64_t)row0 * s.cols, n = (int64_t)nrows * s.cols;
  const int64_t total = (int64_t)s.rows * s.cols;
  const bool fp4 = s.dtype == kFP4;
  const size_t need = fp4 ? (size_t)((total + 1) / 2) : (size_t)total;
  if (!s.native || s.native_len != need)
    return Status::err(kInvalid, "weights: native payload length");
  const size_t b0 = fp4 ? (size_t)(e0 / 2) : (size_t)e0;
  const size_t b1 = fp4 ? (size_t)((e0 + n + 1) / 2) : (size_t)(e0 + n);
  const int nb = (s.cols + 31) / 32;
  const bool blk = s.scheme == kSchemeBlock32;
  const bool scaled = s.scheme == kSchemeTensor || s.scheme == kSchemeRow;
  if (blk && (!s.blk_exp || s.blk_exp_len != (size_t)s.rows * nb))
    return Status::err(kInvalid, "weights: block scale length");
  if (scaled && (!s.row_scale || s.row_scale_len != (size_t)s.rows))
    return Status::err(kInvalid, "weights: row scale length");
  DevBuf bytes, sc, ex, out;
  WV_TRY(bytes.alloc(b1 - b0));
  WV_TRY(copy_h2d(bytes.p, s.native + b0, b1 - b0, st));
  if (scaled) {
    WV_TRY(sc.alloc((size_t)nrows * sizeof(float)));
    WV_TRY(copy_h2d(sc.p, s.row_scale + row0, (size_t)nrows * sizeof(float), st));
  }
  if (blk) {
    WV_TRY(ex.alloc((size_t)nrows * nb));
    WV_TRY(copy_h2d(ex.p, s.blk_exp + (size_t)row0 * nb, (size_t)nrows * nb, st));
  }
  WV_TRY(out.alloc((size_t)n * sizeof(float)));
  WV_TRY(launch_decode_store(bytes.as<uint8_t>(), s.dtype, e0, n, s.cols,
                             scaled ? sc.as<float>() : nullptr, blk ? ex.as<uint8_t>() : nullptr,
                             nb, out.as<float>(), st));
  WV_TRY(copy_d2h(host_out, out.p, (size_t)n * sizeof(float), st));
  WV_HIP(hipStreamSynchronize(st));
  return Status::ok();
}

bool dense_group_fused(int batch) { return uses_split(batch) && mxg_block_m(batch) > 16; }

Status dense_group_build(const DenseLayer* const* layers, int n, int batch,
                         const float* const* x, float* const* pre, float* const* post,
                         DenseGroup* g) {
  if (n <= 0 || !layers || !x || !pre || !g) return Status::err(kInvalid, "dense group: bad args");
  if (!dense_group_fused(batch)) return Status::err(kInvalid, "dense group: batch too small");
  for (int i = 0; i < n; ++i)
    if (layers[i]->format)
      return Status::err(kUnsupported, "dense group: packed block formats run one by one");
  const DenseLayer& L0 = *layers[0];
  g->layers.clear();
  std::vector<SplitJob> jobs(n);
  std::vector<MxgArgs> tab(n);
  const size_t sb = split_bytes(batch, L0.dev.kpad);
  WV_TRY(g->split.alloc(sb * n));
  bool vec = (L0.in % 4) == 0;
  for (int i = 0; i < n; ++i) {
    const DenseLayer* L = layers[i];
    if (!L || L->in != L0.in || L->out != L0.out || L->act != L0.act ||
        L->dev.dtype != L0.dev.dtype || L->dev.scheme != L0.dev.scheme ||
        L->need_epi() != L0.need_epi() || L->terms != L0.terms)
      return Status::err(kInvalid, "dense group: members differ in shape, dtype, scheme or epilogue");
    if (!x[i] || !pre[i] || (L->need_epi() && (!post || !post[i])))
      return Status::err(kInvalid, "dense group: null member buffer");
    uint8_t* buf = g->split.as<uint8_t>() + sb * i;
    jobs[i].x = x[i];
    jobs[i].buf = buf;
    vec = vec && (reinterpret_cast<uintptr_t>(x[i]) & 15u) == 0;
    g->layers.push_back(L);
    tab[i] = mxg_args(*L, batch, buf);
    tab[i].part = nullptr;  // large tiles: no K split
    tab[i].pre = pre[i];
    tab[i].post = post ? post[i] : nullptr;
  }
  WV_TRY(g->jobs.alloc(sizeof(SplitJob) * n));
  WV_TRY(g->tab.alloc(sizeof(MxgArgs) * n));
  WV_TRY(copy_h2d(g->jobs.p, jobs.data(), sizeof(SplitJob) * n, nullptr));
  WV_TRY(copy_h2d(g->tab.p, tab.data(), sizeof(MxgArgs) * n, nullptr));
  WV_HIP(hipStreamSynchronize(nullptr));
  g->hjobs = jobs;
  g->htab = tab;
  g->n = n;
  g->batch = batch;
  g->dtype = L0.dev.dtype;
  g->terms = L0.terms;
  g->blk = L0.dev.scheme == kSchemeBlock32;
  g->vec = vec;
  g->in = L0.in;
  g->kpad = L0.dev.kpad;
  g->shape = tab[0];
  return Status::ok();
}

// Members whose weights hold non-finite codes get their rows recomputed.
static Status group_fix(const DenseGroup& g, hipStream_t st) {
  for (int i = 0; i < g.n; ++i)
    WV_TRY(fix_nonfinite(*g.layers[(size_t)i], g.batch, g.hjobs[(size_t)i].x, g.in,
                         g.htab[(size_t)i].pre, g.htab[(size_t)i].post, st));
  return Status::ok();
}

static bool group_has_nonfinite(const DenseGroup& g) {
  for (const DenseLayer* L : g.layers)
    if (L->dev.nf_count() > 0) return true;
  return false;
}

Status dense_group_forward(const DenseGroup& g, hipStream_t st) {
  WV_TRY(launch_split_group(g.jobs.as<const SplitJob>(), g.n, g.vec, g.in, g.batch, g.in, g.kpad,
                            st, g.terms));
  WV_TRY(launch_mxg_group(g.tab.as<const MxgArgs>(), g.shape, g.n, g.dtype, g.blk, st));
  return group_fix(g, st);
}

Status dense_chain_build(const DenseGroup* const* groups, int count, DenseChain* c,
                         bool keep_inner) {
  if (count <= 0 || !groups || !c) return Status::err(kInvalid, "dense chain: bad args");
  for (int k = 0; k < count; ++k)
    if (!groups[k] || groups[k]->n <= 0) return Status::err(kInvalid, "dense chain: null group");
  c->groups.assign(groups, groups + count);
  c->tabs.clear();
  c->tabs.resize(count);
  c->fused.assign(count, 0);
  for (int k = 0; k + 1 < count; ++k) {
    const DenseGroup& P = *groups[k];
    const DenseGroup& C = *groups[k + 1];
    if (P.n != C.n || P.batch != C.batch)
      return Status::err(kInvalid, "dense chain: groups differ in members or batch");
    if (P.shape.N != C.in)
      return Status::err(kInvalid, "dense chain: out differs from the next group's in");
    for (int i = 0; i < P.n; ++i) {
      const MxgArgs& a = P.htab[i];
      const bool linked = C.hjobs[i].x == (a.post ? a.post : a.pre) ||
                          (!a.need_epi && C.hjobs[i].x == a.pre);
      if (!linked)
        return Status::err(kInvalid, "dense chain: member input is not the previous member's output");
    }
    // the epilogue split would see the matrix-core values of rows that are
    // recomputed afterwards: such a link runs the consumer's own split
    if (P.shape.N % 256 != 0 || C.kpad != P.shape.N || P.shape.mats != 1 ||
        group_has_nonfinite(P) || P.terms != C.terms)
      continue;
    // The consumer's GEMM reads the split only, so the producer's fp32 output
    // may be left out, unless the consumer has rows with non-finite codes:
    // their recomputation after the consumer's product (group_fix) reads the
    // consumer's fp32 input, which is this output.
    const bool drop_out = !keep_inner && !group_has_nonfinite(C);
    std::vector<MxgArgs> tab = P.htab;
    for (int i = 0; i < P.n; ++i) {
      tab[i].next = C.hjobs[i].buf;
      if (drop_out) tab[i].pre = tab[i].post = nullptr;
    }
    WV_TRY(c->tabs[k].alloc(sizeof(MxgArgs) * P.n));
    WV_TRY(copy_h2d(c->tabs[k].p, tab.data(), sizeof(MxgArgs) * P.n, nullptr));
    WV_HIP(hipStreamSynchronize(nullptr));
    c->fused[k] = 1;
  }
  return Status::ok();
}

Status dense_chain_forward(const DenseChain& c, hipStream_t st) {
  if (c.groups.empty()) return Status::err(kInvalid, "dense chain: empty");
  for (size_t k = 0; k < c.groups.size(); ++k) {
    const DenseGroup& g = *c.groups[k];
    if (k == 0 || !c.fused[k - 1])
      WV_TRY(launch_split_group(g.jobs.as<const SplitJob>(), g.n, g.vec, g.in, g.batch, g.in,
                                g.kpad, st, g.terms));
    const MxgArgs* tab = c.fused[k] ? c.tabs[k].as<const MxgArgs>() : g.tab.as<const MxgArgs>();
    WV_TRY(launch_mxg_group(tab, g.shape, g.n, g.dtype, g.blk, st));
    WV_TRY(group_fix(g, st));
  }
  return Status::ok();
}

// ---------------------------------------------------------------------------
Status swiglu_finish(SwiGLULayer* L, hipStream_t st) {
  std::vector<int> u = L->gate.dev.nf_host;
  u.insert(u.end(), L->up.dev.nf_host.begin(), L->up.dev.nf_host.end());
  std::sort(u.begin(), u.end());
  u.erase(std::unique(u.begin(), u.end()), u.end());
  L->nf_gu_host = u;
  return upload_rows(u, &L->nf_gu, st);
}

Status swiglu_build(int in, int inter, int dtype, int scheme, const float* G, const float* U,
                    const float* D, SwiGLULayer* L, hipStream_t st) {
  if (in <= 0 || inter <= 0)
    return Status::err(kInvalid, "swiglu: need InputDim>0 and IntermediateDim>0");
  L->in = in, L->inter = inter;
  WV_TRY(dense_build(in, inter, kLinear, dtype, scheme, G, nullptr, 0, &L->gate, st));
  WV_TRY(dense_build(in, inter, kLinear, dtype, scheme, U, nullptr, 0, &L->up, st));
  WV_TRY(dense_build(inter, in, kLinear, dtype, scheme, D, nullptr, 0, &L->down, st));
  return swiglu_finish(L, st);
}

// Gate / up rows with non-finite codes, recomputed with the product rule.
static Status swiglu_fix(const SwiGLULayer& L, int rows, const float* x, float* h,
                         hipStream_t st) {
  if (L.nf_gu_host.empty()) return Status::ok();
  NfArgs a;
  a.rows = L.nf_gu.as<const int>();
  a.n = (int)L.nf_gu_host.size();
  a.dtype = L.gate.dev.dtype;
  a.mats = 2;
  a.codes[0] = L.gate.dev.d_codes(), a.codes[1] = L.up.dev.d_codes();
  a.scale[0] = L.gate.dev.d_scale(), a.scale[1] = L.up.dev.d_scale();
  a.blk[0] = L.gate.dev.d_blk(), a.blk[1] = L.up.dev.d_blk();
  a.pitch = L.gate.dev.pitch;
  a.nblk = L.gate.dev.nblk;
  a.cols = L.in;
  a.x = x;
  a.x_stride = L.in;
  a.batch = rows;
  a.pre = h;
  a.out_stride = L.inter;
  return launch_nf_fix(a, st);
}

// The 1-4-row gate+up launch writes the down projection's input split.
static bool mx_fused(const SwiGLULayer& L, int rows) {
  return mx_pair(L, rows) && mx_dense(L.down, rows) && L.down.in == L.inter;
}

size_t swiglu_workspace_bytes(const SwiGLULayer& L, int rows) {
  if (mx_fused(L, rows)) return (size_t)rows * gemv_mx_split_bytes(L.down.dev.kpad);
  if (!uses_split(rows)) return 0;
  const size_t a = gemm_ws_bytes(L.gate, rows, 2), b = gemm_ws_bytes(L.down, rows, 1);
  return a > b ? a : b;
}

Status swiglu_forward(const SwiGLULayer& L, int rows, const float* x, float* h, float* y,
                      Workspace* ws, hipStream_t st) {
  if (rows <= 0 || !x || !h || !y) return Status::err(kInvalid, "swiglu forward: bad args");
  if (mx_pair(L, rows) && L.gate.dev.codes_frag.p && L.up.dev.codes_frag.p && mx_vec(L.gate, x)) {
    GemvMxArgs g = mx_args(L.gate, x, rows);
    g.mats = 2;
    g.codesf[1] = L.up.dev.d_codesf();
    g.blkf[1] = L.up.dev.d_blkf();
    g.scale[1] = L.up.dev.d_scale();
    g.pre = h;
    g.need_epi = 0;
    // the split of h for the down projection, when the session's workspace
    // holds it (never allocated here: this may run under graph capture)
    const size_t nb = (size_t)rows * gemv_mx_split_bytes(L.down.dev.kpad);
    const bool fuse = mx_fused(L, rows) && L.down.dev.codes_frag.p && ws && ws->b.bytes >= nb;
    if (fuse) {
      g.next = split_buf(ws);
      g.next_steps = L.down.dev.kpad / 128;
    }
    const bool blk = L.gate.dev.scheme == kSchemeBlock32;
    WV_TRY(launch_gemv_mx(g, L.gate.dev.dtype, blk, st));
    if (!fuse) return dense_forward(L.down, rows, h, y, nullptr, ws, st);
    GemvMxArgs d = mx_args(L.down, h, rows);
    d.asplit = split_buf(ws);
    d.asplit_steps = L.down.dev.kpad / 128;
    d.pre = y;
    d.post = nullptr;
    return launch_gemv_mx(d, L.down.dev.dtype, L.down.dev.scheme == kSchemeBlock32, st);
  }
  if (rows >= 2 && rows <= kMxvMaxBatch) {
    MxvArgs m = mxv_args(L.gate, x, L.in, rows);
    m.mats = 2;
    m.codes[1] = L.up.dev.d_codes();
    m.scale[1] = L.up.dev.d_scale();
    m.blk[1] = L.up.dev.d_blk();
    m.pre = h;
    m.need_epi = 0;
    WV_TRY(launch_mxv(m, L.gate.dev.dtype, L.gate.dev.scheme == kSchemeBlock32, st));
    WV_TRY(swiglu_fix(L, rows, x, h, st));
    return dense_forward(L.down, rows, h, y, nullptr, ws, st);
  }
  if (uses_split(rows)) {
    WV_TRY(ensure_split(ws, swiglu_workspace_bytes(L, rows)));
    uint8_t* buf = split_buf(ws);
    MxgArgs p = mxg_args(L.gate, rows, buf);
    if (mxg_block_m(rows) > 16) WV_TRY(launch_split(x, L.in, rows, L.in, L.gate.dev.kpad, buf, st));
    else set_input(p, x, L.in, L.in);
    p.mats = 2;
    p.codes[1] = L.up.dev.d_codes();
    p.scale[1] = L.up.dev.d_scale();
    p.blk[1] = L.up.dev.d_blk();
    p.blkf[1] = L.up.dev.d_blkf();
    p.codesf[1] = L.up.dev.d_codesf();
    p.pre = h;
    p.need_epi = 0;
    p.keep_out = 1;  // h is split by the down projection next
    WV_TRY(launch_mxg(p, L.gate.dev.dtype, L.gate.dev.scheme == kSchemeBlock32, st));
    WV_TRY(swiglu_fix(L, rows, x, h, st));
    return dense_forward_split(L.down, rows, h, false, ws, y, nullptr, st);
  }
  GemvArgs a = gemv_args(L.gate, x, L.in);
  a.mats = 2;
  a.codes[1] = L.up.dev.d_codes();
  a.scale[1] = L.up.dev.d_scale();
  a.blk[1] = L.up.dev.d_blk();
  a.pre = h;
  a.post = nullptr;
  a.need_epi = 0;
  WV_TRY(launch_gemv(a, L.gate.dev.dtype, L.gate.dev.scheme == kSchemeBlock32, rows,
                     tile_for(L.gate.dev, 2), st));
  return dense_forward(L.down, rows, h, y, nullptr, ws, st);
}

Status swiglu_backward(const SwiGLULayer& L, int rows, const float* x, const float* h,
                       const float* y, const float* g, bool use_target, float* dx, float* dw,
                       double* loss_part, Workspace* ws, hipStream_t st) {
  if (rows <= 0 || !x || !h || !y || !g || !dx || !dw || !ws)
    return Status::err(kInvalid, "swiglu backward: bad args");
  const int in = L.gate.in, inter = L.gate.out;
  const size_t ri = (size_t)rows * in, rf = (size_t)rows * inter, wf = (size_t)inter * in;
  DevBuf b_dpre_d, b_gh, b_gp, b_up, b_dg, b_du, b_dpre, b_gxg, b_gxu;
  WV_TRY(b_dpre_d.alloc(ri * sizeof(float)));
  WV_TRY(b_gh.alloc(rf * sizeof(float)));
  WV_TRY(b_gp.alloc(rf * sizeof(float)));
  WV_TRY(b_up.alloc(rf * sizeof(float)));
  WV_TRY(b_dg.alloc(rf * sizeof(float)));
  WV_TRY(b_du.alloc(rf * sizeof(float)));
  WV_TRY(b_dpre.alloc(rf * sizeof(float)));
  WV_TRY(b_gxg.alloc(ri * sizeof(float)));
  WV_TRY(b_gxu.alloc(ri * sizeof(float)));
  // Down (Linear): its backward takes gy (or forms the MSE gradient from y)
  // on h; the recomputed Down(h) is y itself (same kernels, same input)
  WV_TRY(dense_backward(L.down, rows, h, y, y, g, use_target, b_dpre_d.as<float>(),
                        b_gh.as<float>(), dw + 2 * wf, loss_part, ws, st));
  // Gate and Up recomputed on x (Linear), then the product rule
  WV_TRY(dense_forward(L.gate, rows, x, b_gp.as<float>(), nullptr, ws, st));
  WV_TRY(dense_forward(L.up, rows, x, b_up.as<float>(), nullptr, ws, st));
  WV_TRY(launch_swiglu_bwd(b_gp.as<float>(), b_up.as<float>(), b_gh.as<float>(),
                           b_du.as<float>(), b_dg.as<float>(), (int64_t)rf, st));
  WV_TRY(dense_backward(L.gate, rows, x, b_gp.as<float>(), nullptr, b_dg.as<float>(), false,
                        b_dpre.as<float>(), b_gxg.as<float>(), dw, nullptr, ws, st));
  WV_TRY(dense_backward(L.up, rows, x, b_up.as<float>(), nullptr, b_du.as<float>(), false,
                        b_dpre.as<float>(), b_gxu.as<float>(), dw + wf, nullptr, ws, st));
  WV_TRY(launch_add_f64(b_gxg.as<float>(), b_gxu.as<float>(), dx, (int64_t)ri, st));
  // the scratch buffers are freed on return: the queued work must be done
  return hip_status(hipStreamSynchronize(st), "swiglu backward");
}

Status swiglu_apply_sgd(SwiGLULayer* L, const float* dw, double lr, hipStream_t st) {
  if (!L || !dw) return Status::err(kInvalid, "swiglu sgd: bad args");
  const size_t wf = (size_t)L->gate.out * L->gate.in;
  WV_TRY(dense_apply_sgd(&L->gate, dw, lr, st));
  WV_TRY(dense_apply_sgd(&L->up, dw + wf, lr, st));
  WV_TRY(dense_apply_sgd(&L->down, dw + 2 * wf, lr, st));
  return swiglu_finish(L, st);
}

// ---------------------------------------------------------------------------
Status mha_validate(MHAConfig* c) {
  if (c->d_model <= 0 || c->num_heads <= 0)
    return Status::err(kInvalid, "mha: need DModel>0 and NumHeads>0");
  if (c->head_dim <= 0) {
    if (c->d_model % c->num_heads != 0)
      return Status::err(kInvalid, "mha: HeadDim unset and DModel%NumHeads!=0");
    c->head_dim = c->d_model / c->num_heads;
  }
  if (c->num_kv_heads <= 0) c->num_kv_heads = c->num_heads;
  if (c->num_heads % c->num_kv_heads != 0)
    return Status::err(kInvalid, "mha: NumHeads not divisible by NumKVHeads");
  if (c->max_seq_len <= 0) c->max_seq_len = 512;
  // The reference passes the mask and position kinds through unchecked
  // (src/interop/c_abi.cpp:805-806, child_wire.hpp:180-181); its attention
  // treats every mask other than 2, 3 and 4 as causal (kernels.cu:470-485)
  // and rotates / adds ALiBi only for position kinds 0, 3 / 2, 3
  // (kernels.cu:550-551). Both are folded to the kind that behaves the same.
  if (c->mask != 2 && c->mask != 3 && c->mask != 4) c->mask = 1;
  if (c->pos < 0 || c->pos > 3) c->pos = 1;
  if (c->rope_theta <= 0) c->rope_theta = 10000.0;
  if (c->softmax != 0 && c->softmax != 1) return Status::err(kInvalid, "mha: unknown Softmax");
  return Status::ok();
}

Status mha_build(const MHAConfig& cfg_in, int dtype, int scheme, const float* Q, const float* K,
                 const float* V, const float* O, MHALayer* L, hipStream_t st) {
  MHAConfig cfg = cfg_in;
  WV_TRY(mha_validate(&cfg));
  L->cfg = cfg;
  const int d = cfg.d_model, qd = cfg.q_dim(), kvd = cfg.kv_dim();
  WV_TRY(dense_build(d, qd, kLinear, dtype, scheme, Q, nullptr, 0, &L->q, st));
  WV_TRY(dense_build(d, kvd, kLinear, dtype, scheme, K, nullptr, 0, &L->k, st));
  WV_TRY(dense_build(d, kvd, kLinear, dtype, scheme, V, nullptr, 0, &L->v, st));
  WV_TRY(dense_build(qd, d, kLinear, dtype, scheme, O, nullptr, 0, &L->o, st));
  return Status::ok();
}

size_t mha_workspace_bytes(const MHALayer& L, int batch, int seq) {
  const size_t t = (size_t)batch * seq;
  return t * ((size_t)L.cfg.q_dim() + 2 * (size_t)L.cfg.kv_dim()) * sizeof(float);
}

static size_t mha_split_bytes(const MHALayer& L, int T) {
  if (!uses_split(T)) return 0;
  size_t n = 0;
  for (const DenseLayer* d : {&L.q, &L.k, &L.v, &L.o}) {
    const size_t b = gemm_ws_bytes(*d, T, 1);
    n = b > n ? b : n;
  }
  return n;
}

static bool mha_rope(const MHAConfig& c) { return (c.pos == 0 || c.pos == 3) && c.head_dim / 2 > 0; }

// The RoPE table covers token positions [0, T); built once (mount) and
// reused, so a forward of at most T tokens queues no trigonometry.
static Status ensure_rope_table(const MHALayer& L, int T, Workspace* ws, hipStream_t st) {
  if (!mha_rope(L.cfg)) return Status::ok();
  // a workspace shared by MHA layers of different head_dim or theta (a model
  // session) rebuilds the table when the layer differs
  if (ws->rope_tokens >= T && ws->rope_hd == L.cfg.head_dim && ws->rope_theta == L.cfg.rope_theta)
    return Status::ok();
  WV_TRY(ws->c.alloc((size_t)T * (L.cfg.head_dim / 2) * 2 * sizeof(double)));
  WV_TRY(build_rope_table(ws->c.as<double>(), T, L.cfg.head_dim, L.cfg.rope_theta, st));
  WV_HIP(hipStreamSynchronize(st));
  ws->rope_tokens = T;
  ws->rope_hd = L.cfg.head_dim;
  ws->rope_theta = L.cfg.rope_theta;
  return Status::ok();
}

Status mha_prepare(const MHALayer& L, int batch, int seq, Workspace* ws) {
  const size_t need = mha_workspace_bytes(L, batch, seq);
  if (ws->a.bytes < need) WV_TRY(ws->a.alloc(need));
  WV_TRY(ensure_rope_table(L, batch * seq, ws, nullptr));
  return ensure_split(ws, mha_split_bytes(L, batch * seq));
}

Status mha_forward(const MHALayer& L, int batch, int seq, const float* x, float* attn, float* y,
                   Workspace* ws, hipStream_t st) {
  const MHAConfig& c = L.cfg;
  if (batch <= 0 || seq <= 0 || !x || !attn || !y || !ws)
    return Status::err(kInvalid, "mha forward: bad args");
  if (seq > c.max_seq_len) return Status::err(kInvalid, "mha: seq > MaxSeqLen");
  const size_t need = mha_workspace_bytes(L, batch, seq);
  if (ws->a.bytes < need) WV_TRY(ws->a.alloc(need));
  const int T = batch * seq;
  float* qb = ws->a.as<float>();
  float* kb = qb + (size_t)T * c.q_dim();
  float* vb = kb + (size_t)T * c.kv_dim();
  // RoPE in the Q and K GEMM epilogues (large tiles): the attention kernel
  // then reads rotated rows
  const bool rope = mha_rope(c);
  // (not when Q or K has rows that are recomputed after the product: the
  // rotation pairs each column with another)
  const bool rope_epi = rope && uses_split(T) && mxg_block_m(T) > 16 && c.head_dim % 8 == 0 &&
                        128 % c.head_dim == 0 && !L.q.need_epi() && !L.k.need_epi() &&
                        L.q.dev.nf_count() == 0 && L.k.dev.nf_count() == 0;
  if (rope) WV_TRY(ensure_rope_table(L, T, ws, st));
  if (uses_split(T)) {
    // Q, K and V read the same activations: above 32 rows they are split
    // once (up to 32 rows each GEMM kernel splits its own K range)
    WV_TRY(ensure_split(ws, mha_split_bytes(L, T)));
    const bool once = mxg_block_m(T) > 16;
    const double* tab = rope_epi ? ws->c.as<const double>() : nullptr;
    const int rhd = rope_epi ? c.head_dim : 0;
    if (once)
      WV_TRY(launch_split(x, c.d_model, T, c.d_model, L.q.dev.kpad, split_buf(ws), st, L.q.terms));
    // (Q, K and V are read by the attention kernel next: kept in the caches)
    WV_TRY(dense_forward_split(L.q, T, x, once, ws, qb, nullptr, st, tab, rhd, true));
    WV_TRY(dense_forward_split(L.k, T, x, once, ws, kb, nullptr, st, tab, rhd, true));
    WV_TRY(dense_forward_split(L.v, T, x, once, ws, vb, nullptr, st, nullptr, 0, true));
  } else {
    WV_TRY(dense_forward(L.q, T, x, qb, nullptr, ws, st));
    WV_TRY(dense_forward(L.k, T, x, kb, nullptr, ws, st));
    WV_TRY(dense_forward(L.v, T, x, vb, nullptr, ws, st));
  }
  AttnArgs a;
  a.q = qb, a.k = kb, a.v = vb, a.out = attn;
  a.tokens = T, a.seq = seq, a.heads = c.num_heads, a.kv_heads = c.num_kv_heads;
  a.hd = c.head_dim, a.msl = c.max_seq_len;
  a.mask = c.mask, a.window = c.window, a.prefix_len = c.prefix_len;
  a.window_causal = (c.window_causal || c.mask == 1) ? 1 : 0;
  a.rope = rope && !rope_epi ? 1 : 0;
  if (a.rope) a.rope_tab = ws->c.as<const double>();
  a.alibi = (c.pos == 2 || c.pos == 3) ? 1 : 0;
  a.sigmoid = c.softmax == 1 ? 1 : 0;
  a.rope_theta = c.rope_theta;
  a.scale = c.scale_override > 0 ? c.scale_override : 1.0 / std::sqrt((double)c.head_dim);
  // The matrix-core attention can also write the O projection's split of
  // its output (three FP6 terms; the QKV split is no longer needed): no
  // split launch between the two.
  const bool fuse_o = uses_split(T) && mxg_block_m(T) > 16 && !L.o.format &&
                      L.o.terms == kTerms && L.o.dev.kpad == c.q_dim() &&
                      attention_writes_split(a);
  if (fuse_o) {
    WV_TRY(ensure_split(ws, dense_workspace_bytes(L.o, T)));
    a.split = split_buf(ws);
    a.split_mpad = (int)round_up(T, mxg_block_m(T));
    WV_TRY(launch_attention(a, st));
    return dense_forward_split(L.o, T, attn, true, ws, y, nullptr, st);
  }
  WV_TRY(launch_attention(a, st));
  return dense_forward(L.o, T, attn, y, nullptr, ws, st);
}

}  // namespace wv
