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
#include "split.h"

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

// The K-split reduce of a Dense layer followed in a serial chain by another
// that also writes the next layer's activation split: the split of post,
// laid out as the split buffer of a layer with the same rows and kpad = N, so
// that no split launch runs between the two products. The sums, epilogue and
// split are those of k_mxs_reduce and k_split, in the same order, so the
// results equal the unfused launches bit for bit. One wave per (16-row block
// rb, 128-wide output chunk kc): the partial planes are read row-contiguous
// (lane l takes columns 4 (l % 32) .. + 3 of rows 2i + l / 32), the finished
// values go out with the same coalesced pattern and into LDS, and the split
// reads them back in operand order (rows at or above M as zeros). One wave
// per workgroup: a chained product has few slices (128 at 256 x 1024), and
// one-wave workgroups spread them over that many CUs.
template <int NT>
__global__ __launch_bounds__(64) void k_reduce_split(MxgArgs p, int ksplit) {
  constexpr bool X6 = act_fp6<NT>();
  constexpr int kWaves = 1;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KC = p.N / 128;
  const int w = blockIdx.x * kWaves + wave;
  if (w >= (p.mpad / 16) * KC) return;  // whole waves; no workgroup barrier below
  const int rb = w / KC, kc = w % KC;
  __shared__ __attribute__((aligned(16))) float stage[kWaves][16][132];
  float(*sl)[132] = stage[wave];  // rows padded by 16 bytes: no bank conflicts
  const size_t npad = ((size_t)p.N + 255) / 256 * 256;
  const size_t plane = (size_t)p.mpad * npad;  // one split's plane
  const int c4 = 4 * (lane & 31), n = kc * 128 + c4;
  v4f tot[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) tot[i] = v4f{0.f, 0.f, 0.f, 0.f};
  const float* src = p.part + (size_t)(rb * 16 + (lane >> 5)) * npad + n;
  // the loads of up to 4 splits in flight together, added in split order
#pragma unroll 1
  for (int k0 = 0; k0 < ksplit; k0 += 4) {
    v4f t[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (k0 + u < ksplit) {  // uniform
#pragma unroll
        for (int i = 0; i < 8; ++i)
          t[u][i] = *reinterpret_cast<const v4f*>(src + (size_t)(k0 + u) * plane + (size_t)(2 * i) * npad);
      }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (k0 + u < ksplit) {
#pragma unroll
        for (int i = 0; i < 8; ++i) tot[i] += t[u][i];
      }
  }
  // the epilogue of k_mxs_reduce per output; the split takes post
  const v4f sc = *reinterpret_cast<const v4f*>(p.scale[0] + n);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 2 * i + (lane >> 5), m = rb * 16 + r;
    const bool live = m < p.M;
    const size_t oi = (size_t)m * p.out_stride + n;
    v4f y = tot[i] * sc, out = y;
    if (p.need_epi) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        double d = (double)y[e];
        if (p.bias && n + e < p.bias_len) {
          d += p.bias[n + e];
          y[e] = (float)d;
        }
        out[e] = (float)act_f64(p.act, d);
      }
      if (live) {
        *reinterpret_cast<v4f*>(p.pre + oi) = y;
        *reinterpret_cast<v4f*>(p.post + oi) = out;
      }
    } else if (live) {
      *reinterpret_cast<v4f*>(p.pre + oi) = y;
      if (p.post && p.post != p.pre) *reinterpret_cast<v4f*>(p.post + oi) = y;
    }
    *reinterpret_cast<v4f*>(&sl[r][c4]) = live ? out : v4f{0.f, 0.f, 0.f, 0.f};
  }
  // The LDS operations of one wave execute in order, so the reads below see
  // this wave's writes.
  const int i16 = lane & 15, g = lane >> 4;
  const GlobalU8 scales =
      (GlobalU8)(p.next + (size_t)kTerms * p.mpad * p.N + (size_t)(rb * KC + kc) * kChunkScaleBytes);
  if constexpr (X6) {
    float v[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = *reinterpret_cast<const float4*>(&sl[i16][32 * g + 4 * q]);
      v[4 * q] = t.x, v[4 * q + 1] = t.y, v[4 * q + 2] = t.z, v[4 * q + 3] = t.w;
    }
    const GlobalU8 chunk = (GlobalU8)(p.next + (size_t)(rb * KC + kc) * NT * kFrag6Bytes);
    split_terms6<1, NT, false>(v, chunk, scales, lane);
  } else {
    float v[2][16];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 t = *reinterpret_cast<const float4*>(&sl[i16][64 * h + 16 * g + 4 * q]);
        v[h][4 * q] = t.x, v[h][4 * q + 1] = t.y, v[h][4 * q + 2] = t.z, v[h][4 * q + 3] = t.w;
      }
    const GlobalU8 chunk = (GlobalU8)(p.next + (size_t)(rb * KC + kc) * NT * kFragBytes);
    split_terms<1, NT, false>(v, chunk, scales, lane);
  }
}

}  // namespace

void launch_reduce_split(const MxgArgs& p, int ksplit, hipStream_t st) {
  const unsigned grid = (unsigned)((int64_t)(p.mpad / 16) * (p.N / 128));
  if (p.terms == 1) k_reduce_split<1><<<grid, 64, 0, st>>>(p, ksplit);
  else if (p.terms == 2) k_reduce_split<2><<<grid, 64, 0, st>>>(p, ksplit);
  else k_reduce_split<kTerms><<<grid, 64, 0, st>>>(p, ksplit);
}

void launch_mxs_reduce(const MxgArgs& p, int ksplit, int rows, int mats, hipStream_t st) {
  if (mats == 2) launch_e<2, 1>(p, ksplit, rows, st);
  else launch_e<1, 1>(p, ksplit, rows, st);
}

}  // namespace wv
