// Weight rows holding non-finite codes.
//
// E5M2 codes 0x7C-0x7F and 0xFC-0xFF decode to +-inf and NaN in the
// reference (src/core/float_codecs.cpp:160-182); they reach a store through
// the encoder (|w| at or above the E5M2 overflow threshold with scale 1, or a
// non-finite w) or through a stored payload. The reference then sums
// f64(w) * f64(x) serially (src/cuda/kernels.cu:130-144), so such a row's
// output is +-inf or NaN as IEEE arithmetic gives it.
//
// The batch-1 GEMV decodes each code and accumulates in fp32, which yields
// the same non-finite result. The matrix-core paths multiply every weight by
// several activation terms, some of them zero, and inf * 0 = NaN would turn
// an infinite output into NaN. So layers with such rows keep a list of them,
// made at mount, and after a matrix-core product k_nf_fix recomputes those
// rows (all batch rows) with decoded weights and an f64 sum, and applies the
// layer's epilogue (bias / activation, or the SwiGLU product).
#include "codec.h"
#include "act.h"
#include "common.h"
#include "kernels.h"
#include "runtime.h"

namespace wv {
namespace {

constexpr int kThreads = 256;


// flags[r] = 1 when row r of the canonical codes holds a non-finite E5M2
// code (the exponent field all ones). One workgroup per row.
__global__ __launch_bounds__(kThreads) void k_nf_flags(const uint8_t* __restrict__ codes,
                                                      int pitch, int cols,
                                                      int* __restrict__ flags) {
  const uint8_t* row = codes + (size_t)blockIdx.x * pitch;
  int any = 0;
  for (int c = threadIdx.x; c < cols; c += kThreads) any |= (row[c] & 0x7Cu) == 0x7Cu;
  any = __syncthreads_or(any);
  if (threadIdx.x == 0) flags[blockIdx.x] = any;
}

// Element c of row r as the oracle dequantizes it: decode(code) * row
// scale (f32), times 2^(e - 127) for block scales.
__device__ __forceinline__ float dequant(int dtype, const uint8_t* row, const float* scale,
                                         const uint8_t* blk, int nblk, int r, int c) {
  uint8_t q;
  if (dtype == kFP4) q = (row[c >> 1] >> (4 * (c & 1))) & 15u;
  else q = row[c];
  float w = decode(dtype, q) * scale[r];
  if (blk) w *= pow2f((int)blk[(size_t)r * nblk + c / 32] - 127);
  return w;
}

__device__ __forceinline__ double wave_sum(double v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One wave per (listed row, batch row).
__global__ __launch_bounds__(kThreads) void k_nf_fix(NfArgs a) {
  const int w = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (w >= a.n * a.batch) return;  // whole waves; no barrier below
  const int r = a.rows[w / a.batch], b = w % a.batch;
  const float* x = a.x + (size_t)b * a.x_stride;
  double acc[2] = {0.0, 0.0};
  for (int m = 0; m < a.mats; ++m) {
    const uint8_t* row = a.codes[m] + (size_t)r * a.pitch;
    double s = 0.0;
    for (int c = lane; c < a.cols; c += 64)
      s += (double)dequant(a.dtype, row, a.scale[m], a.blk[m], a.nblk, r, c) * (double)x[c];
    acc[m] = wave_sum(s);
  }
  if (lane != 0) return;
  const size_t oi = (size_t)b * a.out_stride + r;
  if (a.mats == 2) {
    // SwiGLU product (kernels.cu:296-304)
    const float g = (float)acc[0], u = (float)acc[1];
    const float gs = (float)act_f64(kSilu, (double)g);
    a.pre[oi] = (float)((double)gs * (double)u);
    return;
  }
  float y = (float)acc[0];
  if (!a.need_epi) {
    a.pre[oi] = y;
    if (a.post && a.post != a.pre) a.post[oi] = y;
    return;
  }
  // bias and activation (kernels.cu:147-161)
  double v = (double)y;
  if (a.bias && r < a.bias_len) {
    v += a.bias[r];
    y = (float)v;
  }
  a.pre[oi] = y;
  a.post[oi] = (float)act_f64(a.act, v);
}

}  // namespace

Status find_nonfinite_rows(DeviceWeights* dw, hipStream_t st) {
  dw->nf_rows.reset();
  dw->nf_host.clear();
  if (dw->dtype != kE5M2) return Status::ok();
  DevBuf flags;
  WV_TRY(flags.alloc((size_t)dw->rows * sizeof(int)));
  k_nf_flags<<<dw->rows, kThreads, 0, st>>>(dw->codes.as<const uint8_t>(), dw->pitch, dw->cols,
                                            flags.as<int>());
  WV_HIP(hipGetLastError());
  std::vector<int> h((size_t)dw->rows);
  WV_TRY(copy_d2h(h.data(), flags.p, h.size() * sizeof(int), st));
  for (int r = 0; r < dw->rows; ++r)
    if (h[(size_t)r]) dw->nf_host.push_back(r);
  return upload_rows(dw->nf_host, &dw->nf_rows, st);
}

Status upload_rows(const std::vector<int>& rows, DevBuf* out, hipStream_t st) {
  out->reset();
  if (rows.empty()) return Status::ok();
  WV_TRY(out->alloc(rows.size() * sizeof(int)));
  WV_TRY(copy_h2d(out->p, rows.data(), rows.size() * sizeof(int), st));
  return hip_status(hipStreamSynchronize(st), "nonfinite rows");
}

Status launch_nf_fix(const NfArgs& a, hipStream_t st) {
  if (a.n <= 0 || a.batch <= 0) return Status::ok();
  const int64_t waves = (int64_t)a.n * a.batch;
  const unsigned grid = (unsigned)((waves + kThreads / 64 - 1) / (kThreads / 64));
  k_nf_fix<<<grid, kThreads, 0, st>>>(a);
  return hip_status(hipGetLastError(), "nonfinite fix");
}

}  // namespace wv
