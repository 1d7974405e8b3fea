// The K-split reduction: adds the partial sums that the split products
// (k_mxs for 5-32 rows, the split large-tile k_mxg) wrote, in split order,
// and applies the layer's epilogue: the fp32 row scale, bias and activation
// of the reference's Dense epilogue (src/cuda/kernels.cu:147-161), or for
// the SwiGLU gate+up pair h = f32(f64(silu(g)) * f64(u))
// (src/cuda/kernels.cu:296-304).
#include <hip/hip_runtime.h>

#include "act.h"
#include "common.h"
#include "kernels.h"

namespace wv {
namespace {

constexpr int kRedThreads = 256;

// Thread q owns E consecutive outputs of one activation row and issues the
// loads of up to U splits before adding any (consecutive threads read
// consecutive floats of a plane). One output per thread: with E = 4
// (16-byte loads) the f64 epilogues of a thread run back to back on a
// quarter of the waves, and the C3 16-row SwiGLU step measured 1 us slower.
template <int MATS, int E>
__global__ __launch_bounds__(kRedThreads) void k_mxs_reduce(MxgArgs p, int ksplit, int rows) {
  constexpr int U = 16 / MATS;
  const int nq = p.N / E;
  const int64_t q = (int64_t)blockIdx.x * kRedThreads + threadIdx.x;
  if (q >= (int64_t)p.M * nq) return;
  const int mrow = (int)(q / nq), n0 = E * (int)(q % nq);
  const size_t npad = ((size_t)p.N + rows - 1) / rows * rows;
  const size_t plane = (size_t)p.mpad * npad;  // one (split, matrix) plane
  const float* src = p.part + (size_t)mrow * npad + n0;
  typedef float vec __attribute__((ext_vector_type(E)));
  vec tot[MATS];
#pragma unroll
  for (int m = 0; m < MATS; ++m) tot[m] = vec(0.0f);
#pragma unroll 1
  for (int k0 = 0; k0 < ksplit; k0 += U) {
    vec t[MATS][U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k0 + u < ksplit) {  // uniform
#pragma unroll
        for (int m = 0; m < MATS; ++m)
          t[m][u] = *reinterpret_cast<const vec*>(src + ((size_t)(k0 + u) * MATS + m) * plane);
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k0 + u < ksplit) {
#pragma unroll
        for (int m = 0; m < MATS; ++m) tot[m] += t[m][u];
      }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int n = n0 + e;
    const size_t oi = (size_t)mrow * p.out_stride + n;
    if constexpr (MATS == 2) {
      const float gs = (float)act_f64(kSilu, (double)(tot[0][e] * p.scale[0][n]));
      p.pre[oi] = (float)((double)gs * (double)(tot[1][e] * p.scale[1][n]));
    } else {
      float y = tot[0][e] * p.scale[0][n];
      if (p.need_epi) {
        double v = (double)y;
        if (p.bias && n < p.bias_len) {
          v += p.bias[n];
          y = (float)v;
        }
        p.pre[oi] = y;
        p.post[oi] = (float)act_f64(p.act, v);
      } else {
        p.pre[oi] = y;
        if (p.post && p.post != p.pre) p.post[oi] = y;
      }
    }
  }
}

template <int MATS, int E>
void launch_e(const MxgArgs& p, int ksplit, int rows, hipStream_t st) {
  const int64_t n = (int64_t)p.M * (p.N / E);
  k_mxs_reduce<MATS, E><<<(unsigned)((n + kRedThreads - 1) / kRedThreads), kRedThreads, 0, st>>>(
      p, ksplit, rows);
}

}  // namespace

void launch_mxs_reduce(const MxgArgs& p, int ksplit, int rows, int mats, hipStream_t st) {
  if (mats == 2) launch_e<2, 1>(p, ksplit, rows, st);
  else launch_e<1, 1>(p, ksplit, rows, st);
}

}  // namespace wv
