// Dense backward over the device-resident quantized weights and the
// re-quantizing SGD step: the Dense NormalBP leaf
// (src/interop/c_abi.cpp:119-200, welvet_dense_normalbp_f32).
//
//   k_dpre     d_pre = f32(f64(gy) * act'(f64 pre)) (src/cuda/kernels.cu:48-90).
//              With a target, gy = f32(2/n * (f64 post - f64 target)) and the
//              squared differences are summed per block for the MSE loss
//              (src/runtime/training.cpp:44-69). Not launched for a Linear
//              layer without a target: there d_pre is gy, which k_bwd reads
//              directly and stores as d_pre.
//   k_bwd      both products, which read only d_pre, in one launch:
//              * dX = W^T d_pre (kernels.cu:92-107) from the code rows the
//                forward streams: a workgroup owns 1024 columns and a band of
//                rows, each lane 16 consecutive columns (one 16-byte FP8 or
//                8-byte FP4 load per row, 8 rows in flight per wave), decoded
//                in registers and accumulated in f64. The dequantized f32
//                weight (decode times its scale, one f32 multiply) times
//                f64(d_pre) is exact in f64 (24 + 24 significand bits), so
//                every term equals the reference's; only the order of the f64
//                additions differs (rows by wave, then bands).
//              * dW[o][i]: acc = f32(f64(acc) + f64(d_pre[b][o]) * f64(x[b][i]))
//                over b in order (kernels.cu:109-127), in the workgroups after
//                the dX ones. The f64 product of two floats is exact, so this
//                is bit-exact. The read-bound dX stream and the write-bound dW
//                stream share the launch and overlap in HBM.
//   k_gemvt_reduce  adds the band partials in a fixed order, rounds to f32.
//   k_sgd      w' = f32(f64(w) - lr * f64(dW)), w the dequantized f32 weight
//              (native_codec.cpp:1112-1128, weight_at / set_weight_at); the
//              caller re-quantizes w' with the layer's scheme (scheme 0: the
//              reference encode of every element).
//   k_dequant  the weights as f32 (store.cpp:42-71 export_f32, times the scales).
#include <type_traits>

#include "codec.h"
#include "common.h"
#include "kernels.h"

namespace wv {
namespace {

constexpr int kThreads = 256;
constexpr int kCpl = 16;                // dX columns per lane
constexpr int kTileCols = 64 * kCpl;    // columns per dX workgroup
constexpr int kRowsInFlight = 8;        // code rows loaded ahead per wave
constexpr int kBatchChunk = 2;          // d_pre rows per launch
constexpr int kOuterRows = 4;           // dW rows per workgroup

typedef float v2f __attribute__((ext_vector_type(2)));
typedef const float __attribute__((address_space(4)))* ConstF32;

unsigned grid_for(int64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

// act' in f64: activate_deriv_dev (kernels.cu:48-81), host twin
// activate_deriv_f64 (src/core/activate.cpp:31-63).
__device__ double act_deriv(int act, double x) {
  switch (act) {
  case kLinear: return 1.0;
  case kReLU: return x > 0.0 ? 1.0 : 0.0;
  case kReLU2: return x > 0.0 ? 2.0 * x : 0.0;
  case kLeaky: return x > 0.0 ? 1.0 : 0.01;
  case kSilu: {
    const double sg = 1.0 / (1.0 + exp(-x));
    return sg * (1.0 + x * (1.0 - sg));
  }
  case kGELU: {
    const double k = 0.7978845608028654;
    const double u = k * (x + 0.044715 * x * x * x);
    const double th = tanh(u);
    const double du = k * (1.0 + 3.0 * 0.044715 * x * x);
    return 0.5 * (1.0 + th) + 0.5 * x * (1.0 - th * th) * du;
  }
  case kTanh: {
    const double t = tanh(x);
    return 1.0 - t * t;
  }
  case kSigmoid: {
    const double sg = 1.0 / (1.0 + exp(-x));
    return sg * (1.0 - sg);
  }
  default: return 1.0;
  }
}

__global__ __launch_bounds__(kThreads) void k_dpre(const float* __restrict__ g,
                                                   const float* __restrict__ post,
                                                   const float* __restrict__ pre, int act,
                                                   int use_target, double gscale, int64_t n,
                                                   float* __restrict__ dpre,
                                                   double* __restrict__ loss_part) {
  __shared__ double red[kThreads / 64];
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  double sq = 0.0;
  if (i < n) {
    float gy = g[i];
    if (use_target) {
      const double d = (double)post[i] - (double)g[i];
      gy = (float)(gscale * d);
      sq = d * d;
    }
    dpre[i] = (float)((double)gy * act_deriv(act, (double)pre[i]));
  }
  if (!use_target) return;
  for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = red[0];
    for (int w = 1; w < kThreads / 64; ++w) t += red[w];
    loss_part[blockIdx.x] = t;
  }
}

// Decodes the 16 codes of one lane: 16 bytes (FP8) or 8 bytes (FP4, low
// nibble first). The device codes are canonical, so the conversion
// instructions return the reference decode.
template <int DT>
struct RowCodes {
  typedef typename std::conditional<DT == kFP4, uint2, uint4>::type T;
};

template <int DT>
__device__ __forceinline__ void decode16(const typename RowCodes<DT>::T q, float (&w)[16]) {
  if constexpr (DT == kFP4) {
    const uint32_t d[2] = {q.x, q.y};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v2f v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[h], 1.0f, 0);
      const v2f v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[h], 1.0f, 1);
      const v2f v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[h], 1.0f, 2);
      const v2f v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[h], 1.0f, 3);
      w[8 * h + 0] = v0.x, w[8 * h + 1] = v0.y, w[8 * h + 2] = v1.x, w[8 * h + 3] = v1.y;
      w[8 * h + 4] = v2.x, w[8 * h + 5] = v2.y, w[8 * h + 6] = v3.x, w[8 * h + 7] = v3.y;
    }
  } else {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v2f lo, hi;
      if constexpr (DT == kE4M3) {
        lo = __builtin_amdgcn_cvt_pk_f32_fp8(d[k], false), hi = __builtin_amdgcn_cvt_pk_f32_fp8(d[k], true);
      } else {
        lo = __builtin_amdgcn_cvt_pk_f32_bf8(d[k], false), hi = __builtin_amdgcn_cvt_pk_f32_bf8(d[k], true);
      }
      w[4 * k] = lo.x, w[4 * k + 1] = lo.y, w[4 * k + 2] = hi.x, w[4 * k + 3] = hi.y;
    }
  }
}

struct OuterArgs {
  const float* x = nullptr;  // [batch][in]
  float* dw = nullptr;       // [out][in]
  float* dpre_out = nullptr;  // [batch][out]: d_pre written here when the products read gy
  int batch = 0, cb = 0, vec = 0;
};

// dX part: workgroup `blk` of the first tiles * bands owns 1024 columns
// (lane: 16) and a band of rows; wave w takes rows o0 + w, + 4, ..., 8 rows'
// loads in flight at a time. d_pre rows b0 .. b0 + NB - 1. Lanes past the
// padded row read column 0 (never stored). The 4 waves' sums are added in
// wave order through LDS into the band's partial row.
template <int DT, bool BLK, int NB>
__device__ __forceinline__ void gemvt_tile(const GemvtArgs& a, int blk, int tiles, int bands, int b0,
                                           double* __restrict__ part, double (*red)[NB][kTileCols]) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blk % tiles, band = blk / tiles;
  const int c0 = tile * kTileCols + lane * kCpl;
  const int cc = c0 < a.kpad ? c0 : 0;
  const int o0 = (int)((int64_t)a.out * band / bands), o1 = (int)((int64_t)a.out * (band + 1) / bands);
  typedef typename RowCodes<DT>::T Q;
  const uint8_t* base = a.codes + (DT == kFP4 ? cc / 2 : cc);
  const ConstF32 sc = (ConstF32)a.scale;
  const ConstF32 dp = (ConstF32)(a.dpre + (size_t)b0 * a.out);
  double acc[NB][kCpl];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < kCpl; ++j) acc[b][j] = 0.0;

  for (int o = o0 + wave; o < o1; o += 4 * kRowsInFlight) {
    // the round's scalar operands (row scales, d_pre) first, then the code
    // rows: one wait for each kind
    int ou[kRowsInFlight];
    float rs[kRowsInFlight], gp[NB][kRowsInFlight];
#pragma unroll
    for (int u = 0; u < kRowsInFlight; ++u) {
      ou[u] = o + 4 * u < o1 ? o + 4 * u : o;
      rs[u] = BLK ? 1.0f : sc[ou[u]];
#pragma unroll
      for (int b = 0; b < NB; ++b) gp[b][u] = dp[(size_t)b * a.out + ou[u]];
    }
    Q q[kRowsInFlight];
    uint8_t e[kRowsInFlight];
#pragma unroll
    for (int u = 0; u < kRowsInFlight; ++u) {
      q[u] = *reinterpret_cast<const Q*>(base + (size_t)ou[u] * a.pitch);
      e[u] = BLK ? a.blk[(size_t)ou[u] * a.nblk + cc / 32] : (uint8_t)127;
    }
#pragma unroll
    for (int u = 0; u < kRowsInFlight; ++u) {
      if (o + 4 * u >= o1) break;  // wave-uniform
      const float sf = BLK ? pow2f((int)e[u] - 127) : rs[u];
      float w[kCpl];
      decode16<DT>(q[u], w);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const double g = (double)gp[b][u];
#pragma unroll
        for (int j = 0; j < kCpl; ++j) acc[b][j] = fma((double)(w[j] * sf), g, acc[b][j]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < kCpl; ++j) red[wave][b][lane * kCpl + j] = acc[b][j];
  __syncthreads();
  const size_t cpad = (size_t)tiles * kTileCols;
  for (int t = threadIdx.x; t < NB * kTileCols; t += kThreads) {
    const int b = t / kTileCols, c = t % kTileCols;
    const double v = ((red[0][b][c] + red[1][b][c]) + red[2][b][c]) + red[3][b][c];
    part[((size_t)band * NB + b) * cpad + (size_t)tile * kTileCols + c] = v;
  }
}

// dW part: workgroup g (after the dX workgroups) owns kOuterRows rows from
// (g / cb) * kOuterRows and columns (g % cb) * 1024 ..; thread: 4 columns of
// every row. Per batch row (in order) the x slice and the rows' d_pre values
// are loaded once, then every row's accumulators take their f32 step. With
// vec (in a multiple of 4, x and dW 16-byte aligned) the x loads and dW
// stores are 16 bytes.
__device__ __forceinline__ void outer_rows(const float* __restrict__ dpre, const OuterArgs& oa,
                                           int g, int in, int out) {
  const int r0 = (g / oa.cb) * kOuterRows;
  // Linear without a target: d_pre = f32(f64(gy) * 1), which is gy (a NaN
  // stays a NaN), is not formed by a launch of its own; the first column
  // block of each row group stores it.
  if (oa.dpre_out && g % oa.cb == 0 && (int)threadIdx.x < kOuterRows && r0 + (int)threadIdx.x < out) {
    const size_t r = (size_t)r0 + threadIdx.x;
    for (int b = 0; b < oa.batch; ++b) oa.dpre_out[(size_t)b * out + r] = dpre[(size_t)b * out + r];
  }
  const int c = ((g % oa.cb) * kThreads + (int)threadIdx.x) * 4;
  if (c >= in) return;
  const ConstF32 dp = (ConstF32)dpre;
  float acc[kOuterRows][4];
#pragma unroll
  for (int r = 0; r < kOuterRows; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[r][j] = 0.0f;
  for (int b = 0; b < oa.batch; ++b) {
    const float* xb = oa.x + (size_t)b * in + c;
    float xv[4];
    if (oa.vec) {
      const float4 t = *reinterpret_cast<const float4*>(xb);
      xv[0] = t.x, xv[1] = t.y, xv[2] = t.z, xv[3] = t.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[j] = c + j < in ? xb[j] : 0.0f;
    }
    double gr[kOuterRows];
#pragma unroll
    for (int r = 0; r < kOuterRows; ++r)
      gr[r] = (double)dp[(size_t)b * out + (r0 + r < out ? r0 + r : out - 1)];
#pragma unroll
    for (int r = 0; r < kOuterRows; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[r][j] = (float)((double)acc[r][j] + gr[r] * (double)xv[j]);
  }
#pragma unroll
  for (int r = 0; r < kOuterRows; ++r) {
    if (r0 + r >= out) break;
    float* dst = oa.dw + (size_t)(r0 + r) * in + c;
    if (oa.vec) {
      *reinterpret_cast<float4*>(dst) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c + j < in) dst[j] = acc[r][j];
    }
  }
}

// One launch for both products of the backward (both read only d_pre): the
// first tiles * bands workgroups stream the codes for dX partials, the rest
// write dW, so the read-bound and the write-bound streams overlap in HBM.
template <int DT, bool BLK, int NB>
__global__ __launch_bounds__(kThreads) void k_bwd(GemvtArgs a, int b0, int tiles, int bands,
                                                  double* __restrict__ part, OuterArgs oa) {
  __shared__ double red[4][NB][kTileCols];
  const int gemvt_blocks = tiles * bands;
  if ((int)blockIdx.x < gemvt_blocks) {
    gemvt_tile<DT, BLK, NB>(a, blockIdx.x, tiles, bands, b0, part, red);
  } else {
    outer_rows(a.dpre, oa, (int)blockIdx.x - gemvt_blocks, a.in, a.out);
  }
}

// dX[b][i] = f32(sum of the band partials): workgroup (i / 64, b), wave w
// adds bands w, w + 4, ... in order, then the 4 wave sums in wave order.
__global__ __launch_bounds__(kThreads) void k_gemvt_reduce(const double* __restrict__ part,
                                                           int bands, int nb, int in,
                                                           size_t cpad, float* __restrict__ dx) {
  __shared__ double red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = blockIdx.x * 64 + lane, b = blockIdx.y;
  const int ic = i < in ? i : in - 1;
  const double* src = part + (size_t)b * cpad + ic;
  const size_t stride = (size_t)nb * cpad;  // one band
  double s = 0.0;
  int k = wave;
  for (; k + 28 < bands; k += 32) {
    double v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[(size_t)(k + 4 * u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; k < bands; k += 4) s += src[(size_t)k * stride];
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && i < in)
    dx[(size_t)b * in + i] = (float)(((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane]);
}

// SwiGLU backward product (kernels.cu:307-320): with gp = f64(gate_pre),
// s = f32(SiLU(gp)), ds = f32(SiLU'(gp)), dh = f64(grad_h):
// d_up = f32(dh * f64(s)), d_gate = f32(dh * f64(up) * f64(ds)).
__global__ __launch_bounds__(kThreads) void k_swiglu_bwd(const float* __restrict__ gate_pre,
                                                         const float* __restrict__ up_post,
                                                         const float* __restrict__ grad_h,
                                                         float* __restrict__ d_up,
                                                         float* __restrict__ d_gate, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const double gp = (double)gate_pre[i];
  const float s = (float)(gp / (1.0 + exp(-gp)));  // activate_dev Silu (kernels.cu:33)
  const float ds = (float)act_deriv(kSilu, gp);
  const double dh = (double)grad_h[i], up = (double)up_post[i];
  d_up[i] = (float)(dh * (double)s);
  d_gate[i] = (float)(dh * up * (double)ds);
}

// out = f32(f64(a) + f64(b)) (swiglu.cpp:231-234).
__global__ __launch_bounds__(kThreads) void k_add_f64(const float* __restrict__ a,
                                                      const float* __restrict__ b,
                                                      float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = (float)((double)a[i] + (double)b[i]);
}

struct DequantView {
  int dtype, rows, cols, pitch, nblk;
};

// The dequantized f32 weight of element (o, c): decode times the row scale,
// or times 2^e of its 32-column block (scheme 3), as one f32 multiply.
__device__ __forceinline__ float dequant_at(const DequantView& d, const uint8_t* codes,
                                            const float* scale, const uint8_t* blk, int o, int c) {
  uint8_t q;
  if (d.dtype == kFP4) {
    const uint8_t byte = codes[(size_t)o * d.pitch + c / 2];
    q = (c & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15u);
  } else {
    q = codes[(size_t)o * d.pitch + c];
  }
  const float v = decode(d.dtype, q);
  if (blk) return v * pow2f((int)blk[(size_t)o * d.nblk + c / 32] - 127);
  return v * scale[o];
}

// G: the gradient's element type (f32 from the backward kernels, f64 from a
// caller of WeightStore::apply_sgd); either is widened to f64 exactly.
template <class G>
__global__ __launch_bounds__(kThreads) void k_sgd(DequantView v, const uint8_t* __restrict__ codes,
                                                  const float* __restrict__ scale,
                                                  const uint8_t* __restrict__ blk,
                                                  const G* __restrict__ dw, double lr,
                                                  float* __restrict__ w_next) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= (int64_t)v.rows * v.cols) return;
  const int o = (int)(i / v.cols), c = (int)(i % v.cols);
  const float w = dequant_at(v, codes, scale, blk, o, c);
  w_next[i] = (float)((double)w - lr * (double)dw[i]);
}

__global__ __launch_bounds__(kThreads) void k_dequant(DequantView v, const uint8_t* __restrict__ codes,
                                                      const float* __restrict__ scale,
                                                      const uint8_t* __restrict__ blk,
                                                      float* __restrict__ w) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= (int64_t)v.rows * v.cols) return;
  const int o = (int)(i / v.cols), c = (int)(i % v.cols);
  w[i] = dequant_at(v, codes, scale, blk, o, c);
}

DequantView view_of(const DeviceWeights& d) {
  DequantView v;
  v.dtype = d.dtype, v.rows = d.rows, v.cols = d.cols, v.pitch = d.pitch, v.nblk = d.nblk;
  return v;
}

int gemvt_bands(int in, int out) {
  const int tiles = (in + kTileCols - 1) / kTileCols;
  // about 512 dX workgroups (two per CU beside the dW ones), at least 32
  // rows (8 per wave, one round of loads) per band. Measured at 4096 x 4096:
  // 256 workgroups 29.6 us, 512 workgroups 19.4 us for the fused launch.
  int bands = 512 / tiles;
  const int most = (out + 31) / 32;
  if (bands > most) bands = most;
  return bands < 1 ? 1 : bands;
}

template <int DT, bool BLK>
void launch_bwd_t(const GemvtArgs& a, int b0, int nb, int tiles, int bands, int outer_blocks,
                  double* part, const OuterArgs& oa, hipStream_t st) {
  const unsigned grid = (unsigned)(tiles * bands + outer_blocks);
  if (nb == 1) k_bwd<DT, BLK, 1><<<grid, kThreads, 0, st>>>(a, b0, tiles, bands, part, oa);
  else k_bwd<DT, BLK, 2><<<grid, kThreads, 0, st>>>(a, b0, tiles, bands, part, oa);
}

}  // namespace

int64_t dpre_blocks(int64_t n) { return (n + kThreads - 1) / kThreads; }

Status launch_dpre(const float* g, const float* post, const float* pre, int act, int use_target,
                   int64_t n, float* dpre, double* loss_part, hipStream_t st) {
  if (n <= 0 || !g || !pre || !dpre || (use_target && (!post || !loss_part)))
    return Status::err(kInvalid, "dpre: bad args");
  k_dpre<<<grid_for(n), kThreads, 0, st>>>(g, post, pre, act, use_target, 2.0 / (double)n, n, dpre,
                                          loss_part);
  return hip_status(hipGetLastError(), "dpre launch");
}

size_t gemvt_part_bytes(int in, int out) {
  const size_t cpad = (size_t)(in + kTileCols - 1) / kTileCols * kTileCols;
  return (size_t)gemvt_bands(in, out) * kBatchChunk * cpad * sizeof(double);
}

Status launch_backward_products(const GemvtArgs& a, int dtype, bool blk, int batch,
                                const float* x, float* dw, double* part, float* dx,
                                float* dpre_out, hipStream_t st) {
  if (batch <= 0 || a.in <= 0 || a.out <= 0 || !a.codes || !a.scale || !a.dpre || !part || !dx ||
      !x || !dw || (blk && !a.blk) || a.in > a.kpad)
    return Status::err(kInvalid, "backward: bad args");
  const int tiles = (a.in + kTileCols - 1) / kTileCols;
  const int bands = gemvt_bands(a.in, a.out);
  const size_t cpad = (size_t)tiles * kTileCols;
  OuterArgs oa;
  oa.x = x;
  oa.dw = dw;
  oa.dpre_out = dpre_out;
  oa.batch = batch;
  oa.cb = (a.in + 4 * kThreads - 1) / (4 * kThreads);
  oa.vec = a.in % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(dw) & 15u) == 0;
  const int64_t outer = (int64_t)(a.out + kOuterRows - 1) / kOuterRows * oa.cb;
  if (outer + (int64_t)tiles * bands >= (1ll << 31)) return Status::err(kUnsupported, "backward: too large");
  for (int b0 = 0; b0 < batch; b0 += kBatchChunk) {
    const int nb = batch - b0 < kBatchChunk ? batch - b0 : kBatchChunk;
    // the dW workgroups ride with the first chunk (they cover every batch row)
    const int ob = b0 == 0 ? (int)outer : 0;
    switch (dtype) {
    case kE4M3: blk ? launch_bwd_t<kE4M3, true>(a, b0, nb, tiles, bands, ob, part, oa, st) : launch_bwd_t<kE4M3, false>(a, b0, nb, tiles, bands, ob, part, oa, st); break;
    case kE5M2: blk ? launch_bwd_t<kE5M2, true>(a, b0, nb, tiles, bands, ob, part, oa, st) : launch_bwd_t<kE5M2, false>(a, b0, nb, tiles, bands, ob, part, oa, st); break;
    case kFP4: blk ? launch_bwd_t<kFP4, true>(a, b0, nb, tiles, bands, ob, part, oa, st) : launch_bwd_t<kFP4, false>(a, b0, nb, tiles, bands, ob, part, oa, st); break;
    default: return Status::err(kUnsupported, "backward: dtype");
    }
    WV_HIP(hipGetLastError());
    const dim3 rg((unsigned)((a.in + 63) / 64), (unsigned)nb);
    k_gemvt_reduce<<<rg, kThreads, 0, st>>>(part, bands, nb, a.in, cpad, dx + (size_t)b0 * a.in);
    WV_HIP(hipGetLastError());
  }
  return Status::ok();
}

Status launch_swiglu_bwd(const float* gate_pre, const float* up_post, const float* grad_h,
                         float* d_up, float* d_gate, int64_t n, hipStream_t st) {
  if (n <= 0 || !gate_pre || !up_post || !grad_h || !d_up || !d_gate)
    return Status::err(kInvalid, "swiglu bwd: bad args");
  k_swiglu_bwd<<<grid_for(n), kThreads, 0, st>>>(gate_pre, up_post, grad_h, d_up, d_gate, n);
  return hip_status(hipGetLastError(), "swiglu bwd launch");
}

Status launch_add_f64(const float* a, const float* b, float* out, int64_t n, hipStream_t st) {
  if (n <= 0 || !a || !b || !out) return Status::err(kInvalid, "add: bad args");
  k_add_f64<<<grid_for(n), kThreads, 0, st>>>(a, b, out, n);
  return hip_status(hipGetLastError(), "add launch");
}

template <class G>
static Status sgd_launch(const DeviceWeights& d, const G* dw, double lr, float* w_next,
                         hipStream_t st) {
  if (!dw || !w_next) return Status::err(kInvalid, "sgd: bad args");
  k_sgd<G><<<grid_for((int64_t)d.rows * d.cols), kThreads, 0, st>>>(
      view_of(d), d.d_codes(), d.d_scale(), d.d_blk(), dw, lr, w_next);
  return hip_status(hipGetLastError(), "sgd launch");
}

Status launch_sgd(const DeviceWeights& d, const float* dw, double lr, float* w_next,
                  hipStream_t st) {
  return sgd_launch(d, dw, lr, w_next, st);
}

Status launch_sgd(const DeviceWeights& d, const double* dw, double lr, float* w_next,
                  hipStream_t st) {
  return sgd_launch(d, dw, lr, w_next, st);
}

Status launch_dequant(const DeviceWeights& d, float* w, hipStream_t st) {
  if (!w) return Status::err(kInvalid, "dequant: bad args");
  k_dequant<<<grid_for((int64_t)d.rows * d.cols), kThreads, 0, st>>>(view_of(d), d.d_codes(),
                                                                      d.d_scale(), d.d_blk(), w);
  return hip_status(hipGetLastError(), "dequant launch");
}

}  // namespace wv
