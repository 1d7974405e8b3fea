// Quantized-weight GEMV for small batches (the HBM-streaming path).
//
// One workgroup of W waves owns R consecutive weight rows. The K axis is cut
// into chunks of 64 lanes x KB bytes per row (KB 16: 16 FP8 or 32 FP4 codes
// per lane, 1 KiB per wave and row; KB 8: half that); waves take chunks
// round-robin. Each lane keeps its slice of x in registers and applies it to
// all R rows, so x is read once per R rows while the weights stream with one
// KB-byte load per lane per row. All of a chunk's loads are in flight before
// any is used, so the decode and FMAs of a wave's last chunk run after its
// last bytes arrive: half-width chunks (twice the waves) halve that tail. Codes are
// decoded in registers by the gfx950 conversion instructions (valid because
// the device copy is canonical, see codec.h) and accumulated in fp32. The R
// partial sums per lane are folded across the wave with a transposing
// butterfly (R/2 + R/4 + ... shuffles instead of 6 per row), then across the
// 4 waves through LDS. The epilogue applies the row scale, the reference
// bias/activation rule (src/cuda/kernels.cu:147-161) or the SwiGLU product
// (kernels.cu:296-304).
#include "codec.h"
#include "act.h"
#include "common.h"
#include "kernels.h"
#include "wave.h"

namespace wv {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming weight load: non-temporal, so the 16-byte lines do not displace
// x and other reused data from the caches.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// KB bytes of codes per lane: KB / 4 words
template <int KB>
struct Words {
  uint32_t w[KB / 4];
};
template <int KB>
__device__ __forceinline__ Words<KB> load_stream(const uint8_t* p) {
  Words<KB> r;
  if constexpr (KB == 16) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    r.w[0] = v.x, r.w[1] = v.y, r.w[2] = v.z, r.w[3] = v.w;
  } else if constexpr (KB == 8) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    r.w[0] = v.x, r.w[1] = v.y;
  } else {
    static_assert(KB == 4, "4, 8 or 16 bytes per lane");
    r.w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
  }
  return r;
}

typedef float v2f __attribute__((ext_vector_type(2)));
// Pointer into the constant address space (read-only for the kernel's
// lifetime): uniform loads through it compile to scalar loads.
typedef const float __attribute__((address_space(4)))* ConstF32;


// Elements per lane per chunk of KB bytes.
template <int DT, int KB>
struct Codec {
  static constexpr int KS = DT == kFP4 ? 2 * KB : KB;
};

// Decodes the KB bytes of q and returns sum(dec * xv).
template <int DT, int KB>
__device__ __forceinline__ float dot_chunk(const Words<KB>& q, const float* xv) {
  const uint32_t* w = q.w;
  float s0 = 0.0f, s1 = 0.0f;
  if constexpr (DT == kFP4) {
#pragma unroll
    for (int d = 0; d < KB / 4; ++d) {
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
    for (int d = 0; d < KB / 4; ++d) {
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

// One chunk c of K (64 lanes x KB bytes per row): loads first (x slice, then
// the weight rows and block exponents), all in flight before any of them is
// used, then the decode and FMAs into acc. With CLAMP, x reads past cols are
// clamped to the last element and zeroed after the loads (the codes there
// are zero).
template <int DT, bool BLK, int R, int MATS, bool VECX, bool CLAMP, int KB>
__device__ __forceinline__ void gemv_chunk(int c, int lane, int cols, const float* __restrict__ x,
                                           const uint8_t* __restrict__ w0,
                                           const uint8_t* __restrict__ w1,
                                           const uint8_t* __restrict__ e0,
                                           const uint8_t* __restrict__ e1, uint32_t pitch,
                                           uint32_t nblk, float (&acc)[MATS][R]) {
  constexpr int KS = Codec<DT, KB>::KS;
  const int k0 = c * 64 * KS + lane * KS;
  float xr[KS];
  if constexpr (VECX) {
#pragma unroll
    for (int i = 0; i < KS; i += 4) {
      const int k = k0 + i;
      const float4 t = *reinterpret_cast<const float4*>(x + (!CLAMP || k < cols ? k : cols - 4));
      xr[i] = t.x, xr[i + 1] = t.y, xr[i + 2] = t.z, xr[i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < KS; ++i) xr[i] = x[!CLAMP || k0 + i < cols ? k0 + i : cols - 1];
  }
  // 32-bit offsets from the wave-uniform row-group bases: one add per row
  // and loads addressed as scalar base + vector offset
  const uint32_t boff = (uint32_t)c * (64u * KB) + (uint32_t)lane * KB;
  const uint32_t eoff = (uint32_t)k0 >> 5;
  Words<KB> q[MATS][R];
  uint8_t e[MATS][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    q[0][r] = load_stream<KB>(w0 + (r * pitch + boff));
    if constexpr (MATS == 2) q[1][r] = load_stream<KB>(w1 + (r * pitch + boff));
    if constexpr (BLK) {
      e[0][r] = e0[r * nblk + eoff];
      if constexpr (MATS == 2) e[1][r] = e1[r * nblk + eoff];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  float xv[KS];
#pragma unroll
  for (int i = 0; i < KS; ++i) xv[i] = !CLAMP || k0 + i < cols ? xr[i] : 0.0f;
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float p = dot_chunk<DT, KB>(q[m][r], xv);
      if constexpr (BLK) acc[m][r] = fmaf(p, pow2f((int)e[m][r] - 127), acc[m][r]);
      else acc[m][r] += p;
    }
  }
}

// MATS = 1: y = W x with the Dense epilogue into pre/post.
// MATS = 2: g = Wg x, u = Wu x, pre = h = f32(f64(f32(SiLU(g))) * f64(u)).
template <int DT, bool BLK, int R, int MATS, bool VECX, int WAVES, int KB>
__global__ __launch_bounds__(64 * WAVES) void k_gemv(GemvArgs a) {
  constexpr int KS = Codec<DT, KB>::KS;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * R;
  // Every argument the K loop uses is read before its first branch, so the
  // scalar loads of the argument block are issued together and waited on
  // once (otherwise the loop guard is loaded first and the pointers after).
  const int kpad = a.kpad, cols = a.cols;
  const uint32_t nblk = (uint32_t)a.nblk, pitch = (uint32_t)a.pitch;
  const float* __restrict__ x = a.x + (size_t)blockIdx.y * a.x_stride;
  const uint8_t* __restrict__ w0 = a.codes[0] + (size_t)r0 * pitch;
  const uint8_t* __restrict__ w1 = a.codes[MATS - 1] + (size_t)r0 * pitch;
  const uint8_t* __restrict__ e0 = BLK ? a.blk[0] + (size_t)r0 * nblk : nullptr;
  const uint8_t* __restrict__ e1 = BLK ? a.blk[MATS - 1] + (size_t)r0 * nblk : nullptr;

  asm volatile("" ::"s"(kpad), "s"(cols), "s"(nblk), "s"(pitch), "s"(x), "s"(w0), "s"(w1),
               "s"(e0), "s"(e1));
  const int nchunks = (kpad + 64 * KS - 1) / (64 * KS);
  // The R row scales of this group are wave-uniform; they are read through
  // the constant address space so they become scalar loads (own counter, so
  // no vector-memory wait in the K loop covers them), finished long before
  // the epilogue. The scale array is padded to the row padding, a multiple
  // of R.
  float scs[MATS][R];
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
    const ConstF32 sp = (ConstF32)a.scale[m];  // address-space cast: C-style only
#pragma unroll
    for (int r = 0; r < R; ++r) scs[m][r] = sp[r0 + r];
  }

  float acc[MATS][R];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  for (int c = wave; c < nchunks; c += WAVES) {
    // Chunks wholly inside cols (all but a ragged last one) read x without
    // clamps or selects; the test is wave-uniform.
    if ((c + 1) * 64 * KS <= cols) {
      gemv_chunk<DT, BLK, R, MATS, VECX, false, KB>(c, lane, cols, x, w0, w1, e0, e1, pitch, nblk, acc);
    } else if (c * 64 * KS + lane * KS < kpad) {
      gemv_chunk<DT, BLK, R, MATS, VECX, true, KB>(c, lane, cols, x, w0, w1, e0, e1, pitch, nblk, acc);
    }
  }

  __shared__ float part[MATS][WAVES][R];
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
    wave_reduce_rows<R>(acc[m], lane);
    if (lane < R) part[m][wave][reduced_row<R>(lane)] = acc[m][0];
  }
  __syncthreads();
  const int t = threadIdx.x;
  const int o = r0 + t;
  if (t >= R || o >= a.rows) return;
  float tot[MATS];
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
    float sum = part[m][0][t];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum += part[m][w][t];
    float sc = scs[m][0];
#pragma unroll
    for (int r = 1; r < R; ++r) sc = t == r ? scs[m][r] : sc;
    tot[m] = sum * sc;
  }
  const size_t oi = (size_t)blockIdx.y * a.out_stride + o;
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

// Bytes per lane per row and chunk. Measured against 16 (1 KiB per wave and
// row): 4096 x 4096 E4M3 5.04 -> 4.88 us, the 11008 x 4096 FP4 gate+up pair
// 12.2 -> 11.7 us, 4096 x 11008 FP4 8.08 -> 7.53 us.
constexpr int kChunkLaneBytes = 8;

template <int DT, bool BLK, int R, int MATS, int WAVES>
Status launch_t(const GemvArgs& a, int batch, hipStream_t st) {
  const bool vecx = (a.cols % 4 == 0) && (a.x_stride % 4 == 0) &&
                    ((reinterpret_cast<uintptr_t>(a.x) & 15u) == 0);
  dim3 grid((a.rows + R - 1) / R, batch);
  constexpr int KB = kChunkLaneBytes;
  if (vecx) k_gemv<DT, BLK, R, MATS, true, WAVES, KB><<<grid, 64 * WAVES, 0, st>>>(a);
  else k_gemv<DT, BLK, R, MATS, false, WAVES, KB><<<grid, 64 * WAVES, 0, st>>>(a);
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
  // 3, 6 and 8 waves (K axes of 3, 5-6 and 7-8 chunks) come with 8 rows only
  case 3: return launch_r<8, MATS, 3>(a, dtype, blk, batch, st);
  case 6: return launch_r<8, MATS, 6>(a, dtype, blk, batch, st);
  case 8: return launch_r<8, MATS, 8>(a, dtype, blk, batch, st);
  default: return launch_w<MATS, 4>(a, dtype, blk, batch, t.rows, st);
  }
}

}  // namespace

GemvTile gemv_tile(int dtype, int kpad, int rows, int mats, int cus) {
  // K chunks of 64 lanes x kChunkLaneBytes. Waves per group: one per chunk up
  // to 8 chunks (5 -> 6, 7 -> 8), so no wave streams two chunks while
  // another idles; 4 beyond that. Then rows per group so that the grid has
  // >= 8 waves per CU when it can (8 rows with 3, 6 or 8 waves).
  const int ks = dtype == kFP4 ? 2 * kChunkLaneBytes : kChunkLaneBytes;
  const int chunks = (kpad + 64 * ks - 1) / (64 * ks);
  GemvTile t;
  t.waves = chunks <= 4 ? chunks : chunks <= 6 ? 6 : chunks <= 8 ? 8 : 4;
  if (t.waves == 3 || t.waves >= 6) {
    t.rows = 8;
    return t;
  }
  const long want = 8L * (cus > 0 ? cus : 256);
  t.rows = 16;
  while (t.rows > 2 && ((long)rows + t.rows - 1) / t.rows * t.waves < want) t.rows /= 2;
  if (mats == 2 && t.rows > 8) t.rows = 8;
  // the FP4 SwiGLU pair: 4 rows x 4 waves measured 11.44 us against 11.71
  // for 8 x 4 at d_model 4096, d_ff 11008 (two matrices per row halve the
  // rows a wave can keep in flight)
  if (mats == 2 && dtype == kFP4 && t.waves == 4 && t.rows > 4) t.rows = 4;
  return t;
}

Status launch_gemv(const GemvArgs& a, int dtype, bool blk, int batch, GemvTile t, hipStream_t st) {
  if (t.rows != 2 && t.rows != 4 && t.rows != 8 && t.rows != 16)
    return Status::err(kInvalid, "gemv: rows per group must be 2, 4, 8 or 16");
  if ((t.waves == 3 || t.waves == 6 || t.waves == 8) && t.rows != 8)
    return Status::err(kInvalid, "gemv: 3, 6 or 8 waves need 8 rows per group");
  return a.mats == 2 ? launch_m<2>(a, dtype, blk, batch, t, st)
                     : launch_m<1>(a, dtype, blk, batch, t, st);
}

}  // namespace wv
