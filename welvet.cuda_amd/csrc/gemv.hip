// Quantized-weight GEMV for small batches (the HBM-streaming path).
//
// One workgroup = 4 waves owns R consecutive weight rows. The K axis is cut
// into 1 KiB-per-wave chunks (64 lanes x 16 bytes: 16 FP8 or 32 FP4 codes per
// lane); waves take chunks round-robin. Each lane keeps its slice of x in
// registers and applies it to all R rows, so x is read once per R rows while
// the weights stream with one 128-bit load per lane per row. Codes are
// decoded in registers by the gfx950 conversion instructions (valid because
// the device copy is canonical, see codec.h) and accumulated in fp32. The R
// partial sums per lane are folded across the wave with a transposing
// butterfly (R/2 + R/4 + ... shuffles instead of 6 per row), then across the
// 4 waves through LDS. The epilogue applies the row scale, the reference
// bias/activation rule (src/cuda/kernels.cu:147-161) or the SwiGLU product
// (kernels.cu:296-304).
#include "codec.h"
#include "common.h"
#include "kernels.h"

namespace wv {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming weight load: non-temporal, so the 16-byte lines do not displace
// x and other reused data from the caches.
__device__ __forceinline__ uint4 load_stream(const uint8_t* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

typedef float v2f __attribute__((ext_vector_type(2)));

__device__ __forceinline__ double act_f64(int act, double x) {
  switch (act) {
  case kReLU: return x < 0.0 ? 0.0 : x;
  case kSilu: return x / (1.0 + exp(-x));
  case kGELU: {
    const double k = 0.7978845608028654;
    return 0.5 * x * (1.0 + tanh(k * (x + 0.044715 * x * x * x)));
  }
  case kTanh: return tanh(x);
  case kSigmoid: return 1.0 / (1.0 + exp(-x));
  case kLeaky: return x < 0.0 ? 0.01 * x : x;
  case kReLU2: return x < 0.0 ? 0.0 : x * x;
  default: return x;
  }
}

// Elements per lane per 16-byte chunk.
template <int DT>
struct Codec {
  static constexpr int KS = DT == kFP4 ? 32 : 16;
};

// Decodes the 16 bytes of q and accumulates sum(dec * xv) into acc.
template <int DT>
__device__ __forceinline__ float dot_chunk(const uint4 q, const float* xv) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float s0 = 0.0f, s1 = 0.0f;
  if constexpr (DT == kFP4) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const v2f v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 0);
      const v2f v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 1);
      const v2f v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 2);
      const v2f v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 3);
      s0 = fmaf(v0.x, xv[8 * d + 0], s0);
      s1 = fmaf(v0.y, xv[8 * d + 1], s1);
      s0 = fmaf(v1.x, xv[8 * d + 2], s0);
      s1 = fmaf(v1.y, xv[8 * d + 3], s1);
      s0 = fmaf(v2.x, xv[8 * d + 4], s0);
      s1 = fmaf(v2.y, xv[8 * d + 5], s1);
      s0 = fmaf(v3.x, xv[8 * d + 6], s0);
      s1 = fmaf(v3.y, xv[8 * d + 7], s1);
    }
  } else {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      v2f lo, hi;
      if constexpr (DT == kE4M3) {
        lo = __builtin_amdgcn_cvt_pk_f32_fp8(w[d], false);
        hi = __builtin_amdgcn_cvt_pk_f32_fp8(w[d], true);
      } else {
        lo = __builtin_amdgcn_cvt_pk_f32_bf8(w[d], false);
        hi = __builtin_amdgcn_cvt_pk_f32_bf8(w[d], true);
      }
      s0 = fmaf(lo.x, xv[4 * d + 0], s0);
      s1 = fmaf(lo.y, xv[4 * d + 1], s1);
      s0 = fmaf(hi.x, xv[4 * d + 2], s0);
      s1 = fmaf(hi.y, xv[4 * d + 3], s1);
    }
  }
  return s0 + s1;
}

// Folds v[0..N) across lanes that differ in bit `d`: the lane with the bit
// clear keeps the lower half, the other the upper half.
template <int N>
__device__ __forceinline__ void fold(float* v, int lane, int d) {
  const bool up = (lane & d) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float send = up ? v[i] : v[i + N / 2];
    const float keep = up ? v[i + N / 2] : v[i];
    v[i] = keep + __shfl_xor(send, d, 64);
  }
}

// Reduces v[0..R) over the 64 lanes; afterwards lane l holds in v[0] the total
// of row (l >> (6 - log2 R)) & (R - 1).
template <int R>
__device__ __forceinline__ void wave_reduce_rows(float* v, int lane) {
  int d = 32;
  if constexpr (R >= 16) { fold<16>(v, lane, d); d >>= 1; }
  if constexpr (R >= 8) { fold<8>(v, lane, d); d >>= 1; }
  if constexpr (R >= 4) { fold<4>(v, lane, d); d >>= 1; }
  if constexpr (R >= 2) { fold<2>(v, lane, d); d >>= 1; }
  for (; d > 0; d >>= 1) v[0] += __shfl_xor(v[0], d, 64);
}

template <int R>
constexpr int log2c() {
  return R >= 16 ? 4 : R >= 8 ? 3 : R >= 4 ? 2 : R >= 2 ? 1 : 0;
}

// MATS = 1: y = W x with the Dense epilogue into pre/post.
// MATS = 2: g = Wg x, u = Wu x, pre = h = f32(f64(f32(SiLU(g))) * f64(u)).
template <int DT, bool BLK, int R, int MATS, bool VECX, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_gemv(GemvArgs a) {
  constexpr int KS = Codec<DT>::KS;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * R;
  const int b = blockIdx.y;
  const float* __restrict__ x = a.x + (size_t)b * a.x_stride;
  const int nchunks = (a.kpad + 64 * KS - 1) / (64 * KS);

  float acc[MATS][R];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  for (int c = wave; c < nchunks; c += WAVES) {
    const int k0 = c * 64 * KS + lane * KS;
    if (k0 >= a.kpad) continue;
    float xv[KS];
    if constexpr (VECX) {
#pragma unroll
      for (int i = 0; i < KS; i += 4) {
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k0 + i < a.cols) t = *reinterpret_cast<const float4*>(x + k0 + i);
        xv[i] = t.x, xv[i + 1] = t.y, xv[i + 2] = t.z, xv[i + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < KS; ++i) xv[i] = (k0 + i < a.cols) ? x[k0 + i] : 0.0f;
    }
    const size_t boff = (size_t)c * 1024 + (size_t)lane * 16;
    uint4 q[MATS][R];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r)
        q[m][r] = load_stream(a.codes[m] + (size_t)(r0 + r) * a.pitch + boff);
    // every weight load of this chunk is in flight before any decode starts
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float p = dot_chunk<DT>(q[m][r], xv);
        if constexpr (BLK) {
          const uint8_t e = a.blk[m][(size_t)(r0 + r) * a.nblk + (k0 >> 5)];
          acc[m][r] = fmaf(p, pow2f((int)e - 127), acc[m][r]);
        } else {
          acc[m][r] += p;
        }
      }
    }
  }

  __shared__ float part[MATS][WAVES][R];
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
    wave_reduce_rows<R>(acc[m], lane);
    constexpr int shift = 6 - log2c<R>();
    if ((lane & ((1 << shift) - 1)) == 0) part[m][wave][(lane >> shift) & (R - 1)] = acc[m][0];
  }
  __syncthreads();
  if (threadIdx.x >= R) return;
  const int o = r0 + threadIdx.x;
  if (o >= a.rows) return;
  float tot[MATS];
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
    float t = part[m][0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += part[m][w][threadIdx.x];
    tot[m] = t * a.scale[m][o];
  }
  const size_t oi = (size_t)b * a.out_stride + o;
  if constexpr (MATS == 2) {
    const float g = (float)act_f64(kSilu, (double)tot[0]);
    a.pre[oi] = (float)((double)g * (double)tot[1]);
  } else {
    float y = tot[0];
    if (a.need_epi) {
      double v = (double)y;
      if (a.bias && o < a.bias_len) {
        v += a.bias[o];
        y = (float)v;
      }
      a.pre[oi] = y;
      a.post[oi] = (float)act_f64(a.act, v);
    } else {
      a.pre[oi] = y;
      if (a.post) a.post[oi] = y;
    }
  }
}

template <int DT, bool BLK, int R, int MATS, int WAVES>
Status launch_t(const GemvArgs& a, int batch, hipStream_t st) {
  const bool vecx = (a.cols % 4 == 0) && (a.x_stride % 4 == 0) &&
                    ((reinterpret_cast<uintptr_t>(a.x) & 15u) == 0);
  dim3 grid((a.rows + R - 1) / R, batch);
  if (vecx) k_gemv<DT, BLK, R, MATS, true, WAVES><<<grid, 64 * WAVES, 0, st>>>(a);
  else k_gemv<DT, BLK, R, MATS, false, WAVES><<<grid, 64 * WAVES, 0, st>>>(a);
  return hip_status(hipGetLastError(), "gemv launch");
}

template <int R, int MATS, int WAVES>
Status launch_r(const GemvArgs& a, int dtype, bool blk, int batch, hipStream_t st) {
  switch (dtype) {
  case kE4M3: return blk ? launch_t<kE4M3, true, R, MATS, WAVES>(a, batch, st) : launch_t<kE4M3, false, R, MATS, WAVES>(a, batch, st);
  case kE5M2: return blk ? launch_t<kE5M2, true, R, MATS, WAVES>(a, batch, st) : launch_t<kE5M2, false, R, MATS, WAVES>(a, batch, st);
  case kFP4: return blk ? launch_t<kFP4, true, R, MATS, WAVES>(a, batch, st) : launch_t<kFP4, false, R, MATS, WAVES>(a, batch, st);
  }
  return Status::err(kUnsupported, "gemv: dtype");
}

template <int MATS, int WAVES>
Status launch_w(const GemvArgs& a, int dtype, bool blk, int batch, int rows, hipStream_t st) {
  switch (rows) {
  case 2: return launch_r<2, MATS, WAVES>(a, dtype, blk, batch, st);
  case 4: return launch_r<4, MATS, WAVES>(a, dtype, blk, batch, st);
  case 16: return launch_r<16, MATS, WAVES>(a, dtype, blk, batch, st);
  default: return launch_r<8, MATS, WAVES>(a, dtype, blk, batch, st);
  }
}

template <int MATS>
Status launch_m(const GemvArgs& a, int dtype, bool blk, int batch, GemvTile t, hipStream_t st) {
  switch (t.waves) {
  case 1: return launch_w<MATS, 1>(a, dtype, blk, batch, t.rows, st);
  case 2: return launch_w<MATS, 2>(a, dtype, blk, batch, t.rows, st);
  default: return launch_w<MATS, 4>(a, dtype, blk, batch, t.rows, st);
  }
}

}  // namespace

GemvTile gemv_tile(int dtype, int kpad, int rows, int mats, int cus) {
  // K chunks of 1 KiB per wave: waves per group = chunks (at most 4), then
  // rows per group so that the grid has >= 8 waves per CU when it can.
  const int ks = dtype == kFP4 ? 32 : 16;
  const int chunks = (kpad + 64 * ks - 1) / (64 * ks);
  GemvTile t;
  t.waves = chunks >= 4 ? 4 : chunks >= 2 ? 2 : 1;
  const long want = 8L * (cus > 0 ? cus : 256);
  t.rows = 16;
  while (t.rows > 2 && ((long)rows + t.rows - 1) / t.rows * t.waves < want) t.rows /= 2;
  if (mats == 2 && t.rows > 8) t.rows = 8;
  return t;
}

Status launch_gemv(const GemvArgs& a, int dtype, bool blk, int batch, GemvTile t, hipStream_t st) {
  if (t.rows != 2 && t.rows != 4 && t.rows != 8 && t.rows != 16)
    return Status::err(kInvalid, "gemv: rows per group must be 2, 4, 8 or 16");
  return a.mats == 2 ? launch_m<2>(a, dtype, blk, batch, t, st)
                     : launch_m<1>(a, dtype, blk, batch, t, st);
}

}  // namespace wv
