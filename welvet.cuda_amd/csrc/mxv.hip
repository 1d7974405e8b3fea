// Small-batch quantized GEMV on the CDNA4 scaled matrix cores.
//
// v_mfma_scale_f32_16x16x128_f8f6f4 multiplies FP8/FP4 operands with per-32
// E8M0 block scales, so the stored weight codes (canonical form) go straight
// into the B operand: no VALU decode. The activations are fp32; each batch
// row is split into four E4M3 terms x ~ sum_t a_t * 2^e_t (each term
// quantizes the residual of the previous ones per 32-element block), which
// leaves a relative residual of about 2^-16 per element. The 4 terms of up to
// 4 batch rows fill the 16 A rows of one MFMA, and a lane's 4 accumulator rows
// are exactly the 4 terms of one batch row, so their sum needs no shuffles.
//
// Operand lane layouts of the 16x16x128 instruction (lane l, group g = l/16):
//   B (weights), col n = l%16; FP8: bytes 0-15 -> k = 16g + j, bytes 16-31 ->
//   k = 64 + 16g + j; FP4: nibble j -> k = 32g + j. A rows likewise with row
//   i = l%16. D: col l%16, rows 4g + r. Scale of lane l: row l%16, K block g.
//
// Work split: one workgroup per 16 weight rows, 8 waves cut K into ranges;
// each wave loads its weight bytes (non-temporal, all in flight), quantizes
// its x range into LDS while they arrive, runs the MFMAs, and the partial
// sums of the 8 waves meet in LDS for the epilogue (row scale, bias,
// activation, or the SwiGLU product).
#include "codec.h"
#include "act.h"
#include "common.h"
#include "kernels.h"

namespace wv {
namespace {

constexpr int kW = 8;    // waves per workgroup (K split)
constexpr int kSB = 4;   // K steps of 128 per batch
constexpr int kT = 4;    // activation terms

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef short v2s __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4 load_stream(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}


__device__ __forceinline__ float quad_max(float v) {
  int o = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false);
  v = fmaxf(v, __builtin_bit_cast(float, o));
  o = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false);
  return fmaxf(v, __builtin_bit_cast(float, o));
}

// Weight MFMA format code: 0 E4M3, 1 E5M2, 4 E2M1.
template <int DT>
constexpr int wfmt() {
  return DT == kE4M3 ? 0 : DT == kE5M2 ? 1 : 4;
}

template <int DT, bool BLK, int MATS, int NB, bool VECX>
__global__ __launch_bounds__(64 * kW) void k_mxv(MxvArgs a) {
  constexpr bool FP4 = DT == kFP4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int S = a.kpad / 128;
  const int s_begin = wave * S / kW, s_end = (wave + 1) * S / kW;

  __shared__ __attribute__((aligned(16))) uint8_t lds_a[kW][NB * kT * kSB * 128];
  __shared__ uint8_t lds_s[kW][NB * kT * kSB * 4];
  __shared__ float part[kW][MATS][NB][16];
  uint8_t* la = lds_a[wave];
  uint8_t* ls = lds_s[wave];

  v4f acc[MATS];
#pragma unroll
  for (int m = 0; m < MATS; ++m) acc[m] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int sb = s_begin; sb < s_end; sb += kSB) {
    const int ns = min(kSB, s_end - sb);
    // 1. weight bytes of this batch of K steps: all loads in flight
    u32x4 wq[MATS][kSB][2];
    int wsc[MATS][kSB];
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
      const uint8_t* row = a.codes[m] + (size_t)(n0 + n) * a.pitch;
#pragma unroll
      for (int j = 0; j < kSB; ++j) {
        if (j < ns) {
          const int s = sb + j;
          if constexpr (FP4) {
            wq[m][j][0] = load_stream(row + s * 64 + 16 * g);
            wq[m][j][1] = u32x4{0, 0, 0, 0};
          } else {
            wq[m][j][0] = load_stream(row + s * 128 + 16 * g);
            wq[m][j][1] = load_stream(row + s * 128 + 64 + 16 * g);
          }
          wsc[m][j] = BLK ? (int)a.blk[m][(size_t)(n0 + n) * a.nblk + s * 4 + g] : 127;
        } else {
          wq[m][j][0] = wq[m][j][1] = u32x4{0, 0, 0, 0};
          wsc[m][j] = 127;
        }
      }
    }
    // 2. split x[b][sb*128 .. +ns*128) into kT E4M3 terms in this wave's LDS.
    //    Item = (b, 8 consecutive elements); the 4 lanes of a quad hold one
    //    32-element block.
    const int per_b = ns * 16;
    for (int item = lane; item < NB * per_b; item += 64) {
      const int b = item / per_b, e8 = item % per_b;
      const int kl = e8 * 8, k = sb * 128 + kl;
      const float* xb = a.x + (size_t)b * a.x_stride;
      float r[8];
      if (b >= a.batch) {
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = 0.0f;
      } else if (VECX) {
        const float4 p0 = k < a.cols ? *reinterpret_cast<const float4*>(xb + k) : make_float4(0, 0, 0, 0);
        const float4 p1 = k + 4 < a.cols ? *reinterpret_cast<const float4*>(xb + k + 4) : make_float4(0, 0, 0, 0);
        r[0] = p0.x, r[1] = p0.y, r[2] = p0.z, r[3] = p0.w;
        r[4] = p1.x, r[5] = p1.y, r[6] = p1.z, r[7] = p1.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = k + i < a.cols ? xb[k + i] : 0.0f;
      }
#pragma unroll
      for (int t = 0; t < kT; ++t) {
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(r[i]));
        am = quad_max(am);
        const int e = e8m0_exponent(am, 448.0f);
        // scaled converters: divide by and multiply with 2^e exactly
        const float sc = pow2f(e);
        v2s p0 = {0, 0}, p1 = {0, 0};
        p0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p0, r[0], r[1], sc, false);
        p0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p0, r[2], r[3], sc, true);
        p1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p1, r[4], r[5], sc, false);
        p1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p1, r[6], r[7], sc, true);
        const int w0 = __builtin_bit_cast(int, p0), w1 = __builtin_bit_cast(int, p1);
        const int row = b * kT + t;
        *reinterpret_cast<int2*>(la + row * (kSB * 128) + kl) = make_int2(w0, w1);
        if ((lane & 3) == 0) ls[row * (kSB * 4) + kl / 32] = (uint8_t)(e + 127);
        if (t + 1 < kT) {
          const v2f q0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w0, sc, false);
          const v2f q1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w0, sc, true);
          const v2f q2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w1, sc, false);
          const v2f q3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w1, sc, true);
          r[0] -= q0.x, r[1] -= q0.y, r[2] -= q1.x, r[3] -= q1.y;
          r[4] -= q2.x, r[5] -= q2.y, r[6] -= q3.x, r[7] -= q3.y;
        }
      }
    }
    // LDS writes of this wave are complete before its lanes read them.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // 3. MFMAs
#pragma unroll
    for (int j = 0; j < kSB; ++j) {
      if (j < ns) {
        v8i A = v8i{0, 0, 0, 0, 0, 0, 0, 0};
        int asc = 127;
        if (n < NB * kT) {
          const uint8_t* src = la + n * (kSB * 128) + j * 128 + 16 * g;
          const int4 lo = *reinterpret_cast<const int4*>(src);
          const int4 hi = *reinterpret_cast<const int4*>(src + 64);
          A = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
          asc = ls[n * (kSB * 4) + j * 4 + g];
        }
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
          const v8i B = v8i{(int)wq[m][j][0].x, (int)wq[m][j][0].y, (int)wq[m][j][0].z,
                            (int)wq[m][j][0].w, (int)wq[m][j][1].x, (int)wq[m][j][1].y,
                            (int)wq[m][j][1].z, (int)wq[m][j][1].w};
          acc[m] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc[m], 0, wfmt<DT>(), 0,
                                                                   asc, 0, wsc[m][j]);
        }
      }
    }
    // the next batch overwrites this wave's LDS region
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // lane (n, g): accumulator rows 4g..4g+3 are the terms of batch row g
  if (g < NB) {
#pragma unroll
    for (int m = 0; m < MATS; ++m) part[wave][m][g][n] = (acc[m][0] + acc[m][1]) + (acc[m][2] + acc[m][3]);
  }
  __syncthreads();
  if (threadIdx.x >= NB * 16) return;
  const int b = threadIdx.x >> 4, c = threadIdx.x & 15;
  const int o = n0 + c;
  if (b >= a.batch || o >= a.rows) return;
  float tot[MATS];
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) t += part[w][m][b][c];
    tot[m] = t * a.scale[m][o];
  }
  const size_t oi = (size_t)b * a.out_stride + o;
  if constexpr (MATS == 2) {
    const float gte = (float)act_f64(kSilu, (double)tot[0]);
    a.pre[oi] = (float)((double)gte * (double)tot[1]);
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

template <int DT, bool BLK, int MATS, int NB>
Status launch_t(const MxvArgs& a, hipStream_t st) {
  const bool vecx = (a.cols % 8 == 0) && (a.x_stride % 4 == 0) &&
                    ((reinterpret_cast<uintptr_t>(a.x) & 15u) == 0);
  const unsigned grid = (unsigned)((a.rows + 15) / 16);
  if (vecx) k_mxv<DT, BLK, MATS, NB, true><<<grid, 64 * kW, 0, st>>>(a);
  else k_mxv<DT, BLK, MATS, NB, false><<<grid, 64 * kW, 0, st>>>(a);
  return hip_status(hipGetLastError(), "mxv launch");
}

template <int MATS, int NB>
Status launch_nb(const MxvArgs& a, int dtype, bool blk, hipStream_t st) {
  switch (dtype) {
  case kE4M3: return blk ? launch_t<kE4M3, true, MATS, NB>(a, st) : launch_t<kE4M3, false, MATS, NB>(a, st);
  case kE5M2: return blk ? launch_t<kE5M2, true, MATS, NB>(a, st) : launch_t<kE5M2, false, MATS, NB>(a, st);
  case kFP4: return blk ? launch_t<kFP4, true, MATS, NB>(a, st) : launch_t<kFP4, false, MATS, NB>(a, st);
  }
  return Status::err(kUnsupported, "mxv: dtype");
}

template <int MATS>
Status launch_m(const MxvArgs& a, int dtype, bool blk, hipStream_t st) {
  switch (a.batch) {
  case 1: return launch_nb<MATS, 1>(a, dtype, blk, st);
  case 2: return launch_nb<MATS, 2>(a, dtype, blk, st);
  default: return launch_nb<MATS, 4>(a, dtype, blk, st);
  }
}

}  // namespace

Status launch_mxv(const MxvArgs& a, int dtype, bool blk, hipStream_t st) {
  if (a.batch < 1 || a.batch > kMxvMaxBatch) return Status::err(kInvalid, "mxv: batch must be 1..4");
  if (a.kpad % 256 != 0 || a.pitch <= 0) return Status::err(kInvalid, "mxv: layout");
  return a.mats == 2 ? launch_m<2>(a, dtype, blk, st) : launch_m<1>(a, dtype, blk, st);
}

}  // namespace wv
