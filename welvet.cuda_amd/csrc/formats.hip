// Packed block weight formats (QuantFormat): mount-time quantize and
// relayout, dequantization, and the batch-row GEMV over the resident layout.
//
// The reference reserves the QuantFormat enum (include/welvet/weights.hpp:
// 12-15) and lists the formats (README.md:361-383) without implementing any.
// The packed blocks here are ggml's published layouts (block_q8_0 ..
// block_q6_K of ggml-common.h; quantize_row_*_ref and dequantize_row_* of
// ggml-quants.c), the interchange format a caller mounts and exports.
//
// Resident layout. The packed blocks are split at mount into per-row arrays
// of 32-element sub-blocks, so that a lane's share of one sub-block is one
// aligned 16-byte code load plus small aligned side loads:
//   q  codes: 16 bytes per sub-block, byte l holding element l in the low
//      nibble and element l + 16 in the high one (Q8_0: 32 int8, in order);
//      Q2_K/Q3_K 8 bytes, byte b holding elements b, b + 8, b + 16, b + 24
//      in bits 0-1, 2-3, 4-5, 6-7;
//   h  high bits: Q5_0/Q5_1/Q5_K/Q3_K one dword (bit e = the top bit of
//      element e), Q6_K 8 bytes (bits 2e, 2e + 1 = bits 4-5 of element e);
//   s  scales: Q8_0/Q4_0/Q5_0 f16 d; Q4_1/Q5_1 f16 d then f16 m; Q4_K/Q5_K
//      the super-block's 16-byte header (f16 d, f16 dmin, 12 scale bytes),
//      2 bytes per sub-block; Q3_K likewise (12 scale bytes, f16 d, 2 zero
//      bytes); Q2_K and Q6_K the sub-block's two scale bytes; IQ4_NL f16 d;
//      IQ4_XS the super-block's 8-byte header (f16 d, scales_h, scales_l),
//      1 byte per sub-block;
//   e  per super-block: Q2_K f16 d and dmin, Q6_K f16 d.
// Every array holds exactly the packed bytes of its part (Q3_K: 2 bytes of
// padding per 110), so a GEMV reads the packed size (plus x and y). Rows are
// padded to a multiple of 16 with zero bytes (zero scales: padding rows read
// as 0).
#include "act.h"
#include "common.h"
#include "kernels.h"
#include "wave.h"

namespace wv {

namespace {

constexpr int kThreads = 256;
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint16_t ld16(const uint8_t* p) {
  return (uint16_t)(p[0] | (p[1] << 8));
}
__device__ __forceinline__ void st16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
}
__device__ __forceinline__ float f16f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
// binary32 -> binary16 bits, round to nearest even, overflow to infinity,
// NaN to the quiet NaN 0x7E00, in integer operations on the bit pattern.
// (A plain (_Float16) conversion of d = max * -0.125 is folded by the
// compiler into v_fma_mix with a +0 addend, which turns d = -0 into +0.)
__device__ __forceinline__ uint16_t f16b(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t s = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(s | 0x7E00u);
  if (a >= 0x47800000u) return (uint16_t)(s | 0x7C00u);
  const int e = (int)(a >> 23) - 127;
  if (e < -14) {
    if (e < -25) return (uint16_t)s;
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    const int shift = -e - 1;  // to units of 2^-24
    const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    return (uint16_t)(s | (q + (rem > half || (rem == half && (q & 1u)))));
  }
  uint32_t q = ((uint32_t)(e + 15) << 10) | ((a & 0x7FFFFFu) >> 13);
  const uint32_t rem = a & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
  return (uint16_t)(s | q);
}

// ---- quantizers (ggml-quants.c quantize_row_*_ref), one thread per block.
// Plain f32 arithmetic, no contraction, in the order written: the bytes
// equal those of the C restatement.
template <int FMT>
__device__ void quantize_block(const float* __restrict__ x, uint8_t* __restrict__ y) {
#pragma clang fp contract(off)
  if constexpr (FMT == kQ8_0) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    st16(y, f16b(d));
    for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
  } else if constexpr (FMT == kQ4_0 || FMT == kQ5_0) {
    // d = max / -2^(bits - 1), max the element of largest magnitude
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; ++j) {
      if (amax < fabsf(x[j])) {
        amax = fabsf(x[j]);
        mx = x[j];
      }
    }
    constexpr float kDiv = FMT == kQ4_0 ? -8.0f : -16.0f;
    constexpr float kOff = FMT == kQ4_0 ? 8.5f : 16.5f;
    constexpr int kTop = FMT == kQ4_0 ? 15 : 31;
    const float d = mx / kDiv;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    st16(y, f16b(d));
    uint32_t qh = 0;
    uint8_t* qs = y + (FMT == kQ4_0 ? 2 : 6);
    for (int j = 0; j < 16; ++j) {
      int q0 = (int8_t)(x[j] * id + kOff);
      int q1 = (int8_t)(x[16 + j] * id + kOff);
      q0 = q0 < kTop ? q0 : kTop;
      q1 = q1 < kTop ? q1 : kTop;
      qs[j] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
      qh |= (uint32_t)((q0 >> 4) & 1) << j;
      qh |= (uint32_t)((q1 >> 4) & 1) << (j + 16);
    }
    if constexpr (FMT == kQ5_0) {
      for (int b = 0; b < 4; ++b) y[2 + b] = (uint8_t)(qh >> (8 * b));
    }
  } else {
    // Q4_1 / Q5_1: d = (max - min) / (2^bits - 1), m = min
    float mn = 3.402823466e38f, mx = -3.402823466e38f;
    for (int j = 0; j < 32; ++j) {
      if (x[j] < mn) mn = x[j];
      if (x[j] > mx) mx = x[j];
    }
    const float d = (mx - mn) / (FMT == kQ4_1 ? 15.0f : 31.0f);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    st16(y, f16b(d));
    st16(y + 2, f16b(mn));
    uint32_t qh = 0;
    uint8_t* qs = y + (FMT == kQ4_1 ? 4 : 8);
    for (int j = 0; j < 16; ++j) {
      int q0, q1;
      if constexpr (FMT == kQ4_1) {
        q0 = (int8_t)((x[j] - mn) * id + 0.5f);
        q1 = (int8_t)((x[16 + j] - mn) * id + 0.5f);
        q0 = q0 < 15 ? q0 : 15;
        q1 = q1 < 15 ? q1 : 15;
      } else {
        q0 = (uint8_t)((x[j] - mn) * id + 0.5f);
        q1 = (uint8_t)((x[16 + j] - mn) * id + 0.5f);
      }
      qs[j] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
      qh |= (uint32_t)((q0 >> 4) & 1) << j;
      qh |= (uint32_t)((q1 >> 4) & 1) << (j + 16);
    }
    if constexpr (FMT == kQ5_1) {
      for (int b = 0; b < 4; ++b) y[4 + b] = (uint8_t)(qh >> (8 * b));
    }
  }
}

template <int FMT>
__global__ __launch_bounds__(kThreads) void k_fmt_quantize(const float* __restrict__ W,
                                                           int64_t nblocks,
                                                           uint8_t* __restrict__ out) {
  constexpr FmtGeom G = fmt_geom(FMT);
  const int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (b >= nblocks) return;
  float x[32];
  for (int j = 0; j < 32; ++j) x[j] = W[b * 32 + j];
  quantize_block<FMT>(x, out + b * G.bb);
}

// ---- the library's quantizers of the K and IQ4 formats, one thread per
// block, reading x from memory as it goes (a super-block is 256 values).
// One pass, as stated in oracle/formats.c (same arithmetic in the same
// order, no contraction, so the bytes are equal):
//  - affine (Q2_K, Q4_K, Q5_K): per sub-block scale = (max - mn) / qmax and
//    offset = -mn, mn = min(0, min); integer scales / offsets of d = max
//    scale / lmax and dmin = max offset / lmax; q = round((x + dmin lm) /
//    (d ls)) with the f16-rounded d, dmin;
//  - signed (Q3_K, Q6_K): per sub-block s = m / qdiv, m the element of largest
//    magnitude; integer scales l = round(s / d), d = ms / ldiv; q = round(x /
//    (d l));
//  - IQ4_NL / IQ4_XS: the scale maps the largest-magnitude element to the code
//    book's -127 (IQ4_XS: 6-bit integer sub-block scales of d = ms / -32); each
//    element takes the nearest entry (the first on ties).
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
__device__ __forceinline__ float f16r(float v) { return f16f(f16b(v)); }
__device__ __forceinline__ int qround(float v, int lo, int hi) {
#pragma clang fp contract(off)
  return clampi((int)roundf(fminf(fmaxf(v, (float)lo), (float)hi)), lo, hi);
}
__device__ float signed_amax_n(const float* x, int n) {
  float amax = 0.0f, max = 0.0f;
  for (int j = 0; j < n; ++j) {
    if (amax < fabsf(x[j])) {
      amax = fabsf(x[j]);
      max = x[j];
    }
  }
  return max;
}
__device__ __forceinline__ void or8(uint8_t* p, int v) { *p = (uint8_t)(*p | (uint8_t)v); }

__constant__ int8_t kIq4Book[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                    1,    13,   25,  38,  53,  69,  89,  113};

__device__ int iq4_index(float t) {
#pragma clang fp contract(off)
  int best = 0;
  float err = fabsf(t - (float)kIq4Book[0]);
  for (int k = 1; k < 16; ++k) {
    const float e = fabsf(t - (float)kIq4Book[k]);
    if (e < err) {
      err = e;
      best = k;
    }
  }
  return best;
}

// Affine super-block scales: per sub-block the effective scale ds, offset dmn
// and 1/ds; the integer scales ls, lm; d, dmin before f16 rounding.
template <int NSUB, int SUB, int QMAX, int LMAX>
__device__ void affine_scales(const float* x, int (&ls)[NSUB], int (&lm)[NSUB],
                              float (&dmn)[NSUB], float (&id)[NSUB], float* d, float* dmin) {
#pragma clang fp contract(off)
  float scale[NSUB], off[NSUB];
  float max_scale = 0.0f, max_off = 0.0f;
  for (int j = 0; j < NSUB; ++j) {
    const float* v = x + SUB * j;
    float mn = v[0], mx = v[0];
    for (int i = 1; i < SUB; ++i) {
      mn = v[i] < mn ? v[i] : mn;
      mx = v[i] > mx ? v[i] : mx;
    }
    // the offset is -min(min, 0); comparisons, not fmaxf, so that an all-zero
    // or constant sub-block gives +0 (fmaxf may return either signed zero)
    off[j] = mn < 0.0f ? -mn : 0.0f;
    scale[j] = (mx + off[j]) / (float)QMAX;
    if (scale[j] > max_scale) max_scale = scale[j];
    if (off[j] > max_off) max_off = off[j];
  }
  const float inv_s = max_scale > 0.0f ? (float)LMAX / max_scale : 0.0f;
  const float inv_m = max_off > 0.0f ? (float)LMAX / max_off : 0.0f;
  *d = max_scale / (float)LMAX;
  *dmin = max_off / (float)LMAX;
  const float dd = f16r(*d), dm = f16r(*dmin);
  for (int j = 0; j < NSUB; ++j) {
    ls[j] = qround(inv_s * scale[j], 0, LMAX);
    lm[j] = qround(inv_m * off[j], 0, LMAX);
    const float ds = dd * (float)ls[j];
    dmn[j] = dm * (float)lm[j];
    id[j] = ds > 0.0f ? 1.0f / ds : 0.0f;
  }
}

// Signed super-block scales: integer l and 1/(d l) per sub-block, d.
template <int SUB, int LMIN, int LMAX>
__device__ void signed_scales(const float* x, float qdiv, float ldiv, int (&l)[16],
                              float (&is)[16], float* d) {
#pragma clang fp contract(off)
  float s[16];
  for (int j = 0; j < 16; ++j) s[j] = signed_amax_n(x + SUB * j, SUB) / qdiv;
  const float ms = signed_amax_n(s, 16);
  *d = ms / ldiv;
  const float idd = *d != 0.0f ? 1.0f / *d : 0.0f;
  const float dd = f16r(*d);
  for (int j = 0; j < 16; ++j) {
    l[j] = qround(s[j] * idd, LMIN, LMAX);
    const float ds = dd * (float)l[j];
    is[j] = ds != 0.0f ? 1.0f / ds : 0.0f;
  }
}

// 32 code-book indices of one sub-block at scale ds into qs[16]
__device__ void iq4_sub(const float* x, float ds, uint8_t* qs) {
#pragma clang fp contract(off)
  const float id = ds != 0.0f ? 1.0f / ds : 0.0f;
  for (int j = 0; j < 16; ++j)
    qs[j] = (uint8_t)(iq4_index(x[j] * id) | (iq4_index(x[16 + j] * id) << 4));
}

template <int FMT>
__device__ void quantize_kblock(const float* __restrict__ x, uint8_t* __restrict__ y) {
#pragma clang fp contract(off)
  constexpr FmtGeom G = fmt_geom(FMT);
  for (int i = 0; i < G.bb; ++i) y[i] = 0;
  if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
    constexpr bool K5 = FMT == kQ5_K;
    int ls[8], lm[8];
    float dmn[8], id[8], d, dmin;
    affine_scales<8, 32, K5 ? 31 : 15, 63>(x, ls, lm, dmn, id, &d, &dmin);
    st16(y, f16b(d));
    st16(y + 2, f16b(dmin));
    uint8_t* sc = y + 4;
    for (int j = 0; j < 8; ++j) {
      if (j < 4) {
        or8(sc + j, ls[j] & 63);
        or8(sc + j + 4, lm[j] & 63);
      } else {
        sc[j + 4] = (uint8_t)((ls[j] & 15) | ((lm[j] & 15) << 4));
        or8(sc + j - 4, (ls[j] >> 4) << 6);
        or8(sc + j, (lm[j] >> 4) << 6);
      }
    }
    uint8_t* qh = y + 16;
    uint8_t* qs = y + (K5 ? 48 : 16);
    for (int i = 0; i < 4; ++i)
      for (int l = 0; l < 32; ++l) {
        const int ja = 2 * i, jb = 2 * i + 1;
        const int a = qround((x[64 * i + l] + dmn[ja]) * id[ja], 0, K5 ? 31 : 15);
        const int b = qround((x[64 * i + 32 + l] + dmn[jb]) * id[jb], 0, K5 ? 31 : 15);
        qs[32 * i + l] = (uint8_t)((a & 15) | ((b & 15) << 4));
        if constexpr (K5) or8(qh + l, ((a >> 4) << (2 * i)) | ((b >> 4) << (2 * i + 1)));
      }
  } else if constexpr (FMT == kQ2_K) {
    int ls[16], lm[16];
    float dmn[16], id[16], d, dmin;
    affine_scales<16, 16, 3, 15>(x, ls, lm, dmn, id, &d, &dmin);
    for (int j = 0; j < 16; ++j) y[j] = (uint8_t)(ls[j] | (lm[j] << 4));
    for (int n = 0; n < 2; ++n)
      for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) {
          const int e = 128 * n + 32 * j + l, sb = e / 16;
          or8(y + 16 + 32 * n + l, qround((x[e] + dmn[sb]) * id[sb], 0, 3) << (2 * j));
        }
    st16(y + 80, f16b(d));
    st16(y + 82, f16b(dmin));
  } else if constexpr (FMT == kQ3_K || FMT == kQ6_K) {
    constexpr bool K3 = FMT == kQ3_K;
    int l[16];
    float is[16], d;
    if constexpr (K3) signed_scales<16, -32, 31>(x, -4.0f, -32.0f, l, is, &d);
    else signed_scales<16, -128, 127>(x, -32.0f, -128.0f, l, is, &d);
    for (int n = 0; n < 2; ++n)
      for (int t = 0; t < 4; ++t)
        for (int i = 0; i < 32; ++i) {
          const int e = 128 * n + 32 * t + i, sb = e / 16;
          if constexpr (K3) {
            const int v = qround(x[e] * is[sb], -4, 3) + 4;
            or8(y + 32 + 32 * n + i, (v & 3) << (2 * t));
            or8(y + i, (v >> 2) << (4 * n + t));
          } else {
            const int v = qround(x[e] * is[sb], -32, 31) + 32;
            or8(y + 64 * n + 32 * (t & 1) + i, (v & 15) << (4 * (t >> 1)));
            or8(y + 128 + 32 * n + i, (v >> 4) << (2 * t));
          }
        }
    if constexpr (K3) {
      for (int sidx = 0; sidx < 16; ++sidx) {
        const int v = l[sidx] + 32, g = sidx >> 2, i = sidx & 3;
        or8(y + 96 + (g & 1) * 4 + i, (v & 15) << ((g >> 1) * 4));
        or8(y + 96 + 8 + i, (v >> 4) << (2 * g));
      }
      st16(y + 108, f16b(d));
    } else {
      for (int sidx = 0; sidx < 16; ++sidx) y[192 + sidx] = (uint8_t)(int8_t)l[sidx];
      st16(y + 208, f16b(d));
    }
  } else if constexpr (FMT == kIQ4_NL) {
    const float d = signed_amax_n(x, 32) / -127.0f;
    st16(y, f16b(d));
    iq4_sub(x, f16r(d), y + 2);
  } else if constexpr (FMT == kIQ4_XS) {
    float s[8];
    for (int j = 0; j < 8; ++j) s[j] = signed_amax_n(x + 32 * j, 32) / -127.0f;
    const float ms = signed_amax_n(s, 8);
    const float d = ms / -32.0f;
    const float idd = d != 0.0f ? 1.0f / d : 0.0f;
    const float dd = f16r(d);
    st16(y, f16b(d));
    int sh = 0;
    for (int j = 0; j < 8; ++j) {
      const int l = qround(s[j] * idd, -32, 31);
      const int ls = l + 32;
      or8(y + 4 + j / 2, (ls & 15) << (4 * (j & 1)));
      sh |= (ls >> 4) << (2 * j);
      iq4_sub(x + 32 * j, dd * (float)l, y + 8 + 16 * j);
    }
    st16(y + 2, (uint16_t)sh);
  }
}

template <int FMT>
__global__ __launch_bounds__(kThreads) void k_fmt_quantize_k(const float* __restrict__ W,
                                                             int64_t nblocks,
                                                             uint8_t* __restrict__ out) {
  constexpr FmtGeom G = fmt_geom(FMT);
  const int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (b >= nblocks) return;
  quantize_kblock<FMT>(W + b * G.qk, out + b * G.bb);
}

// ---- relayout: one thread per (row, 32-element sub-block) ----------------
template <int FMT>
__global__ __launch_bounds__(kThreads) void k_fmt_relayout(FmtArgs a, const uint8_t* __restrict__ blocks,
                                                           int rows) {
  constexpr FmtGeom G = fmt_geom(FMT);
  constexpr int SPB = G.qk / 32;  // sub-blocks per block
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= (int64_t)rows * a.nsub) return;
  const int row = (int)(i / a.nsub), t = (int)(i % a.nsub);
  const int sb = t % SPB;
  const uint8_t* B = blocks + ((size_t)row * (a.nsub / SPB) + t / SPB) * G.bb;
  uint8_t* q = const_cast<uint8_t*>(a.q) + ((size_t)row * a.nsub + t) * G.qb;
  uint8_t* s = const_cast<uint8_t*>(a.s) + ((size_t)row * a.nsub + t) * G.sb;
  uint8_t* h = G.hb ? const_cast<uint8_t*>(a.h) + ((size_t)row * a.nsub + t) * G.hb : nullptr;
  if constexpr (FMT == kQ8_0) {
    for (int j = 0; j < 32; ++j) q[j] = B[2 + j];
    s[0] = B[0], s[1] = B[1];
  } else if constexpr (FMT == kQ4_0 || FMT == kQ4_1 || FMT == kQ5_0 || FMT == kQ5_1) {
    constexpr int QS = FMT == kQ4_0 ? 2 : FMT == kQ4_1 ? 4 : FMT == kQ5_0 ? 6 : 8;
    for (int j = 0; j < 16; ++j) q[j] = B[QS + j];
    for (int j = 0; j < G.sb; ++j) s[j] = B[j];
    if constexpr (G.hb) {
      constexpr int QH = FMT == kQ5_0 ? 2 : 4;
      for (int j = 0; j < 4; ++j) h[j] = B[QH + j];
    }
  } else if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
    // sub-block sb = 2i + n: nibble n of qs[32 i + e]; Q5_K: bit sb of qh[e]
    constexpr int QS = FMT == kQ5_K ? 48 : 16;
    const int i4 = sb / 2, n = sb % 2;
    for (int l = 0; l < 16; ++l) {
      const int lo = (B[QS + 32 * i4 + l] >> (4 * n)) & 15;
      const int hi = (B[QS + 32 * i4 + l + 16] >> (4 * n)) & 15;
      q[l] = (uint8_t)(lo | (hi << 4));
    }
    s[0] = B[2 * sb], s[1] = B[2 * sb + 1];  // this sub-block's two header bytes
    if constexpr (FMT == kQ5_K) {
      uint32_t bits = 0;
      for (int e = 0; e < 32; ++e) bits |= (uint32_t)((B[16 + e] >> sb) & 1) << e;
      for (int j = 0; j < 4; ++j) h[j] = (uint8_t)(bits >> (8 * j));
    }
  } else if constexpr (FMT == kIQ4_NL || FMT == kIQ4_XS) {
    // table indices in Q4_0's nibble order; IQ4_XS sub-block sb at qs[16 sb]
    constexpr int QS = FMT == kIQ4_NL ? 2 : 8;
    for (int j = 0; j < 16; ++j) q[j] = B[QS + 16 * sb + j];
    if constexpr (FMT == kIQ4_NL) s[0] = B[0], s[1] = B[1];
    else s[0] = B[sb];  // header byte sb
  } else if constexpr (FMT == kQ2_K || FMT == kQ3_K) {
    // sub-block sb = 4 n + j: bits 2j, 2j + 1 of qs[32 n + l] (Q3_K: minus 4
    // unless bit sb of hmask[l] is set); scales 2 sb, 2 sb + 1
    constexpr int QS = FMT == kQ2_K ? 16 : 32;
    const int n = sb / 4, j = sb % 4;
    for (int b = 0; b < 8; ++b) {
      uint8_t v = 0;
      for (int f = 0; f < 4; ++f) v |= (uint8_t)(((B[QS + 32 * n + b + 8 * f] >> (2 * j)) & 3) << (2 * f));
      q[b] = v;
    }
    if constexpr (FMT == kQ2_K) {
      s[0] = B[2 * sb], s[1] = B[2 * sb + 1];
      if (sb == 0) {
        uint8_t* e = const_cast<uint8_t*>(a.e) + ((size_t)row * (a.nsub / SPB) + t / SPB) * 4;
        for (int k = 0; k < 4; ++k) e[k] = B[80 + k];
      }
    } else {
      uint32_t bits = 0;
      for (int l = 0; l < 32; ++l) bits |= (uint32_t)((B[l] >> sb) & 1) << l;
      for (int k = 0; k < 4; ++k) h[k] = (uint8_t)(bits >> (8 * k));
      // header byte k: scales[k] (k < 12), d (12, 13), zero (14, 15)
      for (int k = 2 * sb; k < 2 * sb + 2; ++k) s[k - 2 * sb] = k < 12 ? B[96 + k] : k < 14 ? B[108 + k - 12] : 0;
    }
  } else {
    // Q6_K: sub-block sb = 4 n + t of half n: low 4 bits from nibble t >> 1
    // of ql[64 n + 32 (t & 1) + e], bits 4-5 from bits 2t, 2t + 1 of
    // qh[32 n + e]; scales sc[2 sb], sc[2 sb + 1]
    const int n = sb / 4, tt = sb % 4;
    for (int l = 0; l < 16; ++l) {
      const int lo = (B[64 * n + 32 * (tt & 1) + l] >> (4 * (tt >> 1))) & 15;
      const int hi = (B[64 * n + 32 * (tt & 1) + l + 16] >> (4 * (tt >> 1))) & 15;
      q[l] = (uint8_t)(lo | (hi << 4));
    }
    for (int j = 0; j < 8; ++j) {
      uint8_t v = 0;
      for (int k = 0; k < 4; ++k) v |= (uint8_t)(((B[128 + 32 * n + 4 * j + k] >> (2 * tt)) & 3) << (2 * k));
      h[j] = v;
    }
    s[0] = B[192 + 2 * sb], s[1] = B[192 + 2 * sb + 1];
    if (sb == 0) {
      uint8_t* e = const_cast<uint8_t*>(a.e) + ((size_t)row * (a.nsub / SPB) + t / SPB) * 2;
      e[0] = B[208], e[1] = B[209];
    }
  }
}

// IQ4_NL / IQ4_XS code book (ggml's kvalues_iq4nl) plus 128, as bytes:
// {1, 24, 45, 63, 79, 93, 106, 118, 129, 141, 153, 166, 181, 197, 217, 241}
constexpr uint32_t kIqT0 = 0x3F2D1801u, kIqT1 = 0x766A5D4Fu, kIqT2 = 0xA6998D81u, kIqT3 = 0xF1D9C5B5u;
// the table entries (value + 128) of the four indices (0..15) in the bytes of
// idx: two byte permutes and a blend on bit 3 of each index
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t idx) {
  const uint32_t sel = idx & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(kIqT1, kIqT0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(kIqT3, kIqT2, sel);
  const uint32_t mask = ((idx >> 3) & 0x01010101u) * 0xFFu;
  return (hi & mask) | (lo & ~mask);
}

// ---- decode of one lane's sub-block into 32 f32 code values ---------------
// c[e] = the integer the format multiplies by its scale for element e (the
// offset of the symmetric formats already removed).
template <int FMT>
__device__ __forceinline__ void decode_codes(const uint4 w0, const uint4 w1, uint32_t hb0,
                                             uint32_t hb1, float* c) {
  const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  if constexpr (FMT == kQ8_0) {
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int b = 0; b < 4; ++b) c[4 * d + b] = (float)(int8_t)(w[d] >> (8 * b));
  } else if constexpr (FMT == kIQ4_NL || FMT == kIQ4_XS) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = iq4_lookup(w[d] & 0x0F0F0F0Fu), hi = iq4_lookup((w[d] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        c[4 * d + b] = (float)((int)((lo >> (8 * b)) & 0xFFu) - 128);
        c[4 * d + b + 16] = (float)((int)((hi >> (8 * b)) & 0xFFu) - 128);
      }
    }
  } else if constexpr (FMT == kQ2_K || FMT == kQ3_K) {
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      int v = (int)((w[(e & 7) >> 2] >> (8 * (e & 3) + 2 * (e >> 3))) & 3);
      if constexpr (FMT == kQ3_K) v += 4 * (int)((hb0 >> e) & 1) - 4;
      c[e] = (float)v;
    }
  } else {
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int e = 4 * d + b;
        int lo = (int)((w[d] >> (8 * b)) & 15), hi = (int)((w[d] >> (8 * b + 4)) & 15);
        if constexpr (FMT == kQ5_0 || FMT == kQ5_1 || FMT == kQ5_K) {
          lo |= (int)((hb0 >> e) & 1) << 4;
          hi |= (int)((hb0 >> (e + 16)) & 1) << 4;
        }
        if constexpr (FMT == kQ6_K) {
          lo |= (int)((e < 16 ? (hb0 >> (2 * e)) : 0) & 3) << 4;
          hi |= (int)((hb1 >> (2 * e)) & 3) << 4;
        }
        constexpr int off = FMT == kQ4_0 ? 8 : FMT == kQ5_0 ? 16 : FMT == kQ6_K ? 32 : 0;
        c[e] = (float)(lo - off);
        c[e + 16] = (float)(hi - off);
      }
  }
}

// scale and min of Q4_K/Q5_K sub-block j from the 12 packed scale bytes
// (get_scale_min_k4)
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// Q3_K scale s (0..15) minus 32 from the 12 packed scale bytes: the low
// (groups 0, 1) or high (2, 3) nibble of byte i (even group) or 4 + i (odd
// group), and bits 2g, 2g + 1 of byte 8 + i for bits 4-5 (g = s / 4,
// i = s % 4)
__device__ __forceinline__ int scale_q3k(int s, const uint8_t* q) {
  const int g = s >> 2, i = s & 3;
  const int lo = (q[(g & 1) * 4 + i] >> ((g >> 1) * 4)) & 0xF;
  const int hi = (q[8 + i] >> (2 * g)) & 3;
  return (lo | (hi << 4)) - 32;
}
// the same from the header dwords a0 (scale bytes 0-3), a1 (4-7), tw (8-11)
__device__ __forceinline__ int scale_q3k_regs(int s, uint32_t a0, uint32_t a1, uint32_t tw) {
  const int g = s >> 2, i = s & 3;
  const uint32_t src = (g & 1) ? a1 : a0;
  const int lo = (int)((src >> (8 * i + 4 * (g >> 1))) & 0xFu);
  const int hi = (int)((tw >> (8 * i + 2 * g)) & 3u);
  return (lo | (hi << 4)) - 32;
}

// scale_min_k4 from the header's dwords 1-3 (scale bytes 0-11 at header bytes
// 4-15) with selects only, no indexed register array: byte k + 4 of the
// header is byte k of the scales.
__device__ __forceinline__ void scale_min_k4_regs(int j, uint32_t h1, uint32_t h2, uint32_t h3,
                                                  int* sc, int* m) {
  const int sh = 8 * (j & 3);
  const int b1 = (int)((h1 >> sh) & 0xFF);  // scales[j & 3]
  const int b2 = (int)((h2 >> sh) & 0xFF);  // scales[4 + (j & 3)]
  const int b3 = (int)((h3 >> sh) & 0xFF);  // scales[8 + (j & 3)]
  if (j < 4) {
    *sc = b1 & 63;
    *m = b2 & 63;
  } else {
    *sc = (b3 & 0xF) | ((b1 >> 6) << 4);
    *m = (b3 >> 4) | ((b2 >> 6) << 4);
  }
}

// ---- dequantization of the resident layout ------------------------------
// The 32 dequantized values of sub-block t of a row (the oracle's
// arithmetic, products not contracted into FMAs).
template <int FMT>
__device__ __forceinline__ void dequant_sub(const FmtArgs& a, int row, int t, float (&y)[32]) {
#pragma clang fp contract(off)
  constexpr FmtGeom G = fmt_geom(FMT);
  const uint8_t* q = a.q + ((size_t)row * a.nsub + t) * G.qb;
  const uint8_t* s = a.s + ((size_t)row * a.nsub + t) * G.sb;
  uint4 w0 = make_uint4(0, 0, 0, 0), w1 = make_uint4(0, 0, 0, 0);
  if constexpr (G.qb == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(q);
    w0.x = v.x, w0.y = v.y;
  } else {
    w0 = *reinterpret_cast<const uint4*>(q);
  }
  if constexpr (FMT == kQ8_0) w1 = *reinterpret_cast<const uint4*>(q + 16);
  uint32_t hb0 = 0, hb1 = 0;
  if constexpr (G.hb >= 4) hb0 = *reinterpret_cast<const uint32_t*>(a.h + ((size_t)row * a.nsub + t) * G.hb);
  if constexpr (G.hb == 8) hb1 = *reinterpret_cast<const uint32_t*>(a.h + ((size_t)row * a.nsub + t) * G.hb + 4);
  float c[32];
  decode_codes<FMT>(w0, w1, hb0, hb1, c);
  if constexpr (FMT == kQ8_0 || FMT == kQ4_0 || FMT == kQ5_0) {
    const float d = f16f(ld16(s));
#pragma unroll
    for (int e = 0; e < 32; ++e) y[e] = c[e] * d;
  } else if constexpr (FMT == kQ4_1 || FMT == kQ5_1) {
    const float d = f16f(ld16(s)), m = f16f(ld16(s + 2));
#pragma unroll
    for (int e = 0; e < 32; ++e) y[e] = c[e] * d + m;
  } else if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
    const uint8_t* hd = a.s + ((size_t)row * a.nsub + (t & ~7)) * G.sb;  // super-block header
    int sc, m;
    scale_min_k4(t & 7, hd + 4, &sc, &m);
    const float d1 = f16f(ld16(hd)) * (float)sc, m1 = f16f(ld16(hd + 2)) * (float)m;
#pragma unroll
    for (int e = 0; e < 32; ++e) y[e] = d1 * c[e] - m1;
  } else if constexpr (FMT == kIQ4_NL) {
    const float d = f16f(ld16(s));
#pragma unroll
    for (int e = 0; e < 32; ++e) y[e] = d * c[e];
  } else if constexpr (FMT == kIQ4_XS) {
    const uint8_t* hd = a.s + ((size_t)row * a.nsub + (t & ~7));  // super-block header
    const int ib = t & 7, sh = ld16(hd + 2);
    const int ls = ((hd[4 + ib / 2] >> (4 * (ib & 1))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
    const float dl = f16f(ld16(hd)) * (float)(ls - 32);
#pragma unroll
    for (int e = 0; e < 32; ++e) y[e] = dl * c[e];
  } else if constexpr (FMT == kQ2_K) {
    const uint8_t* e = a.e + ((size_t)row * (a.nsub / 8) + t / 8) * 4;
    const float d = f16f(ld16(e)), dmin = f16f(ld16(e + 2));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float dl = d * (float)(s[h] & 15), ml = dmin * (float)(s[h] >> 4);
#pragma unroll
      for (int k = 16 * h; k < 16 * h + 16; ++k) y[k] = dl * c[k] - ml;
    }
  } else if constexpr (FMT == kQ3_K) {
    const uint8_t* hd = a.s + ((size_t)row * a.nsub + (t & ~7)) * G.sb;  // super-block header
    const float d = f16f(ld16(hd + 12));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float dl = d * (float)scale_q3k(2 * (t & 7) + h, hd);
#pragma unroll
      for (int k = 16 * h; k < 16 * h + 16; ++k) y[k] = dl * c[k];
    }
  } else {
    const float d = f16f(ld16(a.e + ((size_t)row * (a.nsub / 8) + t / 8) * 2));
    const float s0 = d * (float)(int8_t)s[0], s1 = d * (float)(int8_t)s[1];
#pragma unroll
    for (int e = 0; e < 16; ++e) y[e] = s0 * c[e];
#pragma unroll
    for (int e = 16; e < 32; ++e) y[e] = s1 * c[e];
  }
}

// f32 [rows][cols] from the resident arrays (WeightStore::export_f32's
// role): one thread per (row, sub-block)
template <int FMT>
__global__ __launch_bounds__(kThreads) void k_fmt_dequant(FmtArgs a, int rows, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= (int64_t)rows * a.nsub) return;
  const int row = (int)(i / a.nsub), t = (int)(i % a.nsub);
  float y[32];
  dequant_sub<FMT>(a, row, t, y);
  float* o = out + (size_t)row * a.cols + 32 * (size_t)t;
#pragma unroll
  for (int e = 0; e < 32; ++e) o[e] = y[e];
}


__device__ __forceinline__ uint4 load_stream(const uint8_t* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- GEMV: one workgroup of WAVES waves owns R rows; lane l of wave w takes
// sub-block 64 c + l of every row for chunks c = w, w + WAVES, ..; its 32 x
// values are loaded once per chunk and applied to all R rows. Per row it
// loads the 16-byte code (32 for Q8_0) and the small side arrays, forms the
// dot product of the unsigned codes with x in f32 and applies the
// sub-block's scale once: d * (sum(c x) - off * sum(x)) for the symmetric
// formats, d * sum(c x) + m * sum(x) for the affine ones. Codes become floats
// by byte conversions of masked dwords (v_cvt_f32_ubyte), about 2.4 VALU
// operations per 4-bit element with the FMA; the high bits of the 5- and
// 6-bit formats are spread into bits 4-5 of each byte first. The R per-lane
// partial sums are reduced across the wave with the transposing butterfly
// and then across the waves in LDS; the epilogue is the Dense one
// (kernels.cu:147-161: bias and activation in f64).

// byte b of v as a float
__device__ __forceinline__ float ub(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }
// bits 0-3 of x to bit 0 of bytes 0-3 (x * (1 + 2^7 + 2^14 + 2^21) puts bit
// k at 8k with no other term on those bits)
__device__ __forceinline__ uint32_t spread1(uint32_t x) { return (x * 0x00204081u) & 0x01010101u; }
// 2-bit fields 0-3 of x to bits 0-1 of bytes 0-3
__device__ __forceinline__ uint32_t spread2(uint32_t x) {
  x = (x | (x << 12)) & 0x000F000Fu;
  return (x | (x << 6)) & 0x03030303u;
}

// sum over the low-nibble elements (0..15) and the high-nibble ones (16..31)
// of code * x; HB high bits per element from h0 (elements 0-15 for HB = 2)
// and h1 (elements 16-31, HB = 2)
template <int HB>
__device__ __forceinline__ void dot_sub(const uint4 w, uint32_t h0, uint32_t h1,
                                        const float* xv, float& plo, float& phi) {
  const uint32_t W[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t lo = W[d] & 0x0F0F0F0Fu, hi = (W[d] >> 4) & 0x0F0F0F0Fu;
    if constexpr (HB == 1) {
      lo |= spread1((h0 >> (4 * d)) & 0xFu) << 4;
      hi |= spread1((h0 >> (16 + 4 * d)) & 0xFu) << 4;
    } else if constexpr (HB == 2) {
      lo |= spread2((h0 >> (8 * d)) & 0xFFu) << 4;
      hi |= spread2((h1 >> (8 * d)) & 0xFFu) << 4;
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      plo = fmaf(ub(lo, b), xv[4 * d + b], plo);
      phi = fmaf(ub(hi, b), xv[16 + 4 * d + b], phi);
    }
  }
}

// Q2_K / Q3_K: 8 code bytes (byte b: elements b + 8f in bits 2f, 2f + 1);
// Q3_K adds the high bit of element e (bit e of h) as bit 2 of its code
template <bool Q3>
__device__ __forceinline__ void dot_sub2(uint32_t w0, uint32_t w1, uint32_t h, const float* xv,
                                         float& plo, float& phi) {
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    uint32_t u0 = (w0 >> (2 * f)) & 0x03030303u, u1 = (w1 >> (2 * f)) & 0x03030303u;
    if constexpr (Q3) {
      u0 |= spread1((h >> (8 * f)) & 0xFu) << 2;
      u1 |= spread1((h >> (8 * f + 4)) & 0xFu) << 2;
    }
    float& p = f < 2 ? plo : phi;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      p = fmaf(ub(u0, b), xv[8 * f + b], p);
      p = fmaf(ub(u1, b), xv[8 * f + 4 + b], p);
    }
  }
}

// IQ4_NL / IQ4_XS: sum over the 32 elements of (table value + 128) * x
__device__ __forceinline__ float dot_iq4(const uint4 w, const float* xv) {
  const uint32_t W[4] = {w.x, w.y, w.z, w.w};
  float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t lo = iq4_lookup(W[d] & 0x0F0F0F0Fu), hi = iq4_lookup((W[d] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      p0 = fmaf(ub(lo, b), xv[4 * d + b], p0);
      p1 = fmaf(ub(hi, b), xv[16 + 4 * d + b], p1);
    }
  }
  return p0 + p1;
}

// Q8_0: int8 codes q; (q + 128) as unsigned bytes, the 128 taken off with
// sum(x) by the caller
__device__ __forceinline__ float dot_q8(const uint4 w0, const uint4 w1, const float* xv) {
  const uint32_t W[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const uint32_t u = W[d] ^ 0x80808080u;
    p0 = fmaf(ub(u, 0), xv[4 * d], p0);
    p1 = fmaf(ub(u, 1), xv[4 * d + 1], p1);
    p0 = fmaf(ub(u, 2), xv[4 * d + 2], p0);
    p1 = fmaf(ub(u, 3), xv[4 * d + 3], p1);
  }
  return p0 + p1;
}

template <int FMT, int R, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_fmt_gemv(FmtArgs a) {
  constexpr FmtGeom G = fmt_geom(FMT);
  constexpr int HB = FMT == kQ6_K ? 2 : G.hb ? 1 : 0;  // nibble formats
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * R;
  const int nsub = a.nsub;
  const float* __restrict__ x = a.x + (size_t)blockIdx.y * a.x_stride;
  const int nchunks = (nsub + 63) / 64;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;

  for (int ch = wave; ch < nchunks; ch += WAVES) {
    const int t = ch * 64 + lane;
    if (t < nsub) {
      float xv[32];
#pragma unroll
      for (int i = 0; i < 32; i += 4) {
        const float4 v = *reinterpret_cast<const float4*>(x + 32 * (size_t)t + i);
        xv[i] = v.x, xv[i + 1] = v.y, xv[i + 2] = v.z, xv[i + 3] = v.w;
      }
      uint4 w0[R], w1[R];
      uint32_t h0[R], h1[R], sv[R], hd[R][4];
      uint32_t ev[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const size_t sub = (size_t)(r0 + r) * nsub + t;
        w1[r] = make_uint4(0, 0, 0, 0);
        if constexpr (G.qb == 8) {
          typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(a.q + sub * 8));
          w0[r] = make_uint4(v.x, v.y, 0u, 0u);
        } else {
          w0[r] = load_stream(a.q + sub * G.qb);
        }
        if constexpr (FMT == kQ8_0) w1[r] = load_stream(a.q + sub * G.qb + 16);
        h0[r] = h1[r] = 0;
        if constexpr (G.hb >= 4) h0[r] = *reinterpret_cast<const uint32_t*>(a.h + sub * G.hb);
        if constexpr (G.hb == 8) h1[r] = *reinterpret_cast<const uint32_t*>(a.h + sub * G.hb + 4);
        if constexpr (FMT == kIQ4_XS) {
          const uint2 v = *reinterpret_cast<const uint2*>(a.s + ((size_t)(r0 + r) * nsub + (t & ~7)));
          hd[r][0] = v.x, hd[r][1] = v.y, hd[r][2] = hd[r][3] = 0;
          sv[r] = 0;
        } else if constexpr (FMT == kQ4_K || FMT == kQ5_K || FMT == kQ3_K) {
          const uint4 v = *reinterpret_cast<const uint4*>(a.s + ((size_t)(r0 + r) * nsub + (t & ~7)) * G.sb);
          hd[r][0] = v.x, hd[r][1] = v.y, hd[r][2] = v.z, hd[r][3] = v.w;
          sv[r] = 0;
        } else if constexpr (G.sb == 4) {
          sv[r] = *reinterpret_cast<const uint32_t*>(a.s + sub * 4);
        } else {
          sv[r] = *reinterpret_cast<const uint16_t*>(a.s + sub * 2);
        }
        ev[r] = 0;
        if constexpr (FMT == kQ6_K)
          ev[r] = *reinterpret_cast<const uint16_t*>(a.e + ((size_t)(r0 + r) * (nsub / 8) + t / 8) * 2);
        if constexpr (FMT == kQ2_K)
          ev[r] = *reinterpret_cast<const uint32_t*>(a.e + ((size_t)(r0 + r) * (nsub / 8) + t / 8) * 4);
      }
      __builtin_amdgcn_sched_barrier(0);
      float sx_lo = 0.0f, sx_hi = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        sx_lo += xv[e] + xv[e + 1];
        sx_hi += xv[16 + e] + xv[17 + e];
      }
      const float sx = sx_lo + sx_hi;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float v;
        if constexpr (FMT == kQ8_0) {
          v = f16f((uint16_t)sv[r]) * fmaf(-128.0f, sx, dot_q8(w0[r], w1[r], xv));
        } else if constexpr (FMT == kIQ4_NL) {
          v = f16f((uint16_t)sv[r]) * fmaf(-128.0f, sx, dot_iq4(w0[r], xv));
        } else if constexpr (FMT == kIQ4_XS) {
          const int ib = t & 7;
          const uint32_t sh = hd[r][0] >> 16;
          const int ls = (int)(((hd[r][1] >> (8 * (ib >> 1) + 4 * (ib & 1))) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
          v = f16f((uint16_t)hd[r][0]) * (float)(ls - 32) * fmaf(-128.0f, sx, dot_iq4(w0[r], xv));
        } else if constexpr (FMT == kQ2_K || FMT == kQ3_K) {
          float plo = 0.0f, phi = 0.0f;
          dot_sub2<FMT == kQ3_K>(w0[r].x, w0[r].y, h0[r], xv, plo, phi);
          if constexpr (FMT == kQ2_K) {
            // (d * sc) * sum(q x) - (dmin * m) * sum(x) per 16-element half
            const float d = f16f((uint16_t)ev[r]), dmin = f16f((uint16_t)(ev[r] >> 16));
            const float s0 = (float)(sv[r] & 15u), s1 = (float)((sv[r] >> 8) & 15u);
            const float m0 = (float)((sv[r] >> 4) & 15u), m1 = (float)((sv[r] >> 12) & 15u);
            v = fmaf(d, fmaf(s1, phi, s0 * plo), -dmin * fmaf(m1, sx_hi, m0 * sx_lo));
          } else {
            // codes 0..7 with offset 4, signed 6-bit scale per 16-element half
            const int j = t & 7;
            const float s0 = (float)scale_q3k_regs(2 * j, hd[r][0], hd[r][1], hd[r][2]);
            const float s1 = (float)scale_q3k_regs(2 * j + 1, hd[r][0], hd[r][1], hd[r][2]);
            const float lo = fmaf(-4.0f, sx_lo, plo), hi = fmaf(-4.0f, sx_hi, phi);
            v = f16f((uint16_t)hd[r][3]) * fmaf(s1, hi, s0 * lo);
          }
        } else {
          float plo = 0.0f, phi = 0.0f;
          dot_sub<HB>(w0[r], h0[r], h1[r], xv, plo, phi);
          if constexpr (FMT == kQ4_0 || FMT == kQ5_0) {
            constexpr float off = FMT == kQ4_0 ? -8.0f : -16.0f;
            v = f16f((uint16_t)sv[r]) * fmaf(off, sx, plo + phi);
          } else if constexpr (FMT == kQ4_1 || FMT == kQ5_1) {
            v = fmaf(f16f((uint16_t)(sv[r] >> 16)), sx, f16f((uint16_t)sv[r]) * (plo + phi));
          } else if constexpr (FMT == kQ4_K || FMT == kQ5_K) {
            int sc, m;
            scale_min_k4_regs(t & 7, hd[r][1], hd[r][2], hd[r][3], &sc, &m);
            const float d1 = f16f((uint16_t)hd[r][0]) * (float)sc;
            const float m1 = f16f((uint16_t)(hd[r][0] >> 16)) * (float)m;
            v = fmaf(d1, plo + phi, -m1 * sx);
          } else {
            // Q6_K: codes 0..63, offset 32, one int8 scale per 16 elements
            const float lo = fmaf(-32.0f, sx_lo, plo), hi = fmaf(-32.0f, sx_hi, phi);
            v = f16f(ev[r]) * fmaf((float)(int8_t)(sv[r] >> 8), hi, (float)(int8_t)sv[r] * lo);
          }
        }
        acc[r] += v;
      }
    }
  }

  // every lane is active here (the DPP moves need that)
  __shared__ float part[WAVES][R];
  wave_reduce_rows<R>(acc, lane);
  if (lane < R) part[wave][reduced_row<R>(lane)] = acc[0];
  __syncthreads();
  const int tr = threadIdx.x;
  const int o = r0 + tr;
  if (tr >= R || o >= a.rows) return;
  float y = part[0][tr];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) y += part[w][tr];
  const size_t oi = (size_t)blockIdx.y * a.out_stride + o;
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
    if (a.post && a.post != a.pre) a.post[oi] = y;
  }
}

// Batches of 2 rows and more on the matrix cores, each weight decoded once
// for up to 16 batch rows. Workgroup (blockIdx.x, blockIdx.y): weight rows
// r0 = 16 blockIdx.x .. +15 against batch rows j0 = 16 blockIdx.y .. +15; its
// W waves take the groups of 4 sub-blocks (128 columns) round-robin. In a
// group, lane (i, g) (i = lane % 16, g = lane / 16) dequantizes sub-block
// 4q + g of weight row r0 + i to its exact f32 values (dequant_sub, the
// oracle's arithmetic) and loads the same 32 columns of batch row j0 + i;
// v_mfma_f32_16x16x4_f32 number m takes value m of every lane: A[i][g] the
// weight, B[g][i] the input, so the 32 products add the group's 128 columns
// (the four sub-blocks through the instruction's k = g). Lane (i, g) ends
// with D[4g + r][i]: weight row r0 + 4g + r, batch row j0 + i. The waves'
// sums are added in wave order through LDS, then the epilogue of k_fmt_gemv.
// Batch rows from which the matrix-core kernel runs. Measured at 4096 x
// 4096 (Q4_K, Q8_0, Q4_0, Q6_K): batch 8 14-16 us against 17-29 us for the
// per-row kernel, batch 16 20 us against 28-52 us; at batch 2-4 the per-row
// kernel is as fast or faster (the matrix core's 16 batch columns cost the
// same for 2 rows as for 16).
constexpr int kFmtMfmaBatch = 8;

template <int FMT, int W>
__global__ __launch_bounds__(64 * W) void k_fmt_mfma(FmtArgs a, int batch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int r0 = blockIdx.x * 16, j0 = blockIdx.y * 16;
  const int row = r0 + i;  // < rpad, a multiple of 16: in bounds
  const bool xlive = j0 + i < batch;
  const float* __restrict__ xr = a.x + (size_t)(xlive ? j0 + i : 0) * a.x_stride;
  const int groups = (a.nsub + 3) / 4;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  for (int q = wave; q < groups; q += W) {
    const int t = 4 * q + g;
    float w[32], xv[32];
    if (t < a.nsub) {
      dequant_sub<FMT>(a, row, t, w);
#pragma unroll
      for (int e = 0; e < 32; e += 4) {
        const float4 v = xlive ? *reinterpret_cast<const float4*>(xr + 32 * (size_t)t + e)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
        xv[e] = v.x, xv[e + 1] = v.y, xv[e + 2] = v.z, xv[e + 3] = v.w;
      }
    } else {  // past the last sub-block (cols not a multiple of 128)
#pragma unroll
      for (int e = 0; e < 32; ++e) w[e] = xv[e] = 0.0f;
    }
    // every lane is active from here (the matrix core reads all 64)
#pragma unroll
    for (int m = 0; m < 32; ++m) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w[m], xv[m], acc, 0, 0, 0);
  }

  __shared__ v4f part[W][64];
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  v4f y = part[0][lane];
#pragma unroll
  for (int w = 1; w < W; ++w) y += part[w][lane];
  const int j = j0 + i;
  if (j >= batch) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int o = r0 + 4 * g + r;
    if (o >= a.rows) break;
    const size_t oi = (size_t)j * a.out_stride + o;
    float v = y[r];
    if (a.need_epi) {
      double d = (double)v;
      if (a.bias && o < a.bias_len) {
        d += a.bias[o];
        v = (float)d;
      }
      a.pre[oi] = v;
      a.post[oi] = (float)act_f64(a.act, d);
    } else {
      a.pre[oi] = v;
      if (a.post && a.post != a.pre) a.post[oi] = v;
    }
  }
}

template <int FMT>
Status mfma_f(const FmtArgs& a, int batch, hipStream_t st) {
  constexpr int W = 8;
  const dim3 grid((unsigned)((a.rows + 15) / 16), (unsigned)((batch + 15) / 16));
  k_fmt_mfma<FMT, W><<<grid, 64 * W, 0, st>>>(a, batch);
  return hip_status(hipGetLastError(), "format matrix-core gemv launch");
}

template <int FMT, int R>
Status gemv_w(const FmtArgs& a, int batch, int waves, hipStream_t st) {
  const dim3 grid((unsigned)((a.rows + R - 1) / R), (unsigned)batch);
  switch (waves) {
  case 1: k_fmt_gemv<FMT, R, 1><<<grid, 64, 0, st>>>(a); break;
  case 2: k_fmt_gemv<FMT, R, 2><<<grid, 128, 0, st>>>(a); break;
  default: k_fmt_gemv<FMT, R, 4><<<grid, 256, 0, st>>>(a); break;
  }
  return hip_status(hipGetLastError(), "format gemv launch");
}

template <int FMT>
Status gemv_f(const FmtArgs& a, int batch, hipStream_t st) {
  if (batch >= kFmtMfmaBatch) return mfma_f<FMT>(a, batch, st);
  // one wave per 64-sub-block chunk up to 4; then rows per group so that the
  // grid has >= 8 waves per CU when it can
  const int chunks = (a.nsub + 63) / 64;
  const int waves = chunks <= 1 ? 1 : chunks == 2 ? 2 : 4;
  const long groups8 = ((long)a.rows + 7) / 8 * batch;
  if (groups8 * waves >= 8L * 256) return gemv_w<FMT, 8>(a, batch, waves, st);
  return gemv_w<FMT, 4>(a, batch, waves, st);
}

template <int FMT>
Status quantize_f(const float* W, int64_t n, uint8_t* out, hipStream_t st) {
  constexpr FmtGeom G = fmt_geom(FMT);
  const int64_t nb = n / G.qk;
  if (nb == 0) return Status::ok();
  const unsigned grid = (unsigned)((nb + kThreads - 1) / kThreads);
  if constexpr (FMT == kQ8_0 || FMT == kQ4_0 || FMT == kQ4_1 || FMT == kQ5_0 || FMT == kQ5_1)
    k_fmt_quantize<FMT><<<grid, kThreads, 0, st>>>(W, nb, out);
  else
    k_fmt_quantize_k<FMT><<<grid, kThreads, 0, st>>>(W, nb, out);
  return hip_status(hipGetLastError(), "format quantize launch");
}

template <int FMT>
Status relayout_f(const FmtArgs& a, const uint8_t* blocks, int rows, hipStream_t st) {
  const int64_t n = (int64_t)rows * a.nsub;
  if (n == 0) return Status::ok();
  k_fmt_relayout<FMT><<<(unsigned)((n + kThreads - 1) / kThreads), kThreads, 0, st>>>(a, blocks, rows);
  return hip_status(hipGetLastError(), "format relayout launch");
}

template <int FMT>
Status dequant_f(const FmtArgs& a, int rows, float* out, hipStream_t st) {
  const int64_t n = (int64_t)rows * a.nsub;
  if (n == 0) return Status::ok();
  k_fmt_dequant<FMT><<<(unsigned)((n + kThreads - 1) / kThreads), kThreads, 0, st>>>(a, rows, out);
  return hip_status(hipGetLastError(), "format dequant launch");
}

}  // namespace

Status format_quantize(int fmt, const float* W, int64_t n, uint8_t* out, hipStream_t st) {
  const FmtGeom G = fmt_geom(fmt);
  if (G.qk == 0 || n % G.qk) return Status::err(kInvalid, "format quantize: element count");
  switch (fmt) {
  case kQ8_0: return quantize_f<kQ8_0>(W, n, out, st);
  case kQ4_0: return quantize_f<kQ4_0>(W, n, out, st);
  case kQ4_1: return quantize_f<kQ4_1>(W, n, out, st);
  case kQ5_0: return quantize_f<kQ5_0>(W, n, out, st);
  case kQ5_1: return quantize_f<kQ5_1>(W, n, out, st);
  case kQ2_K: return quantize_f<kQ2_K>(W, n, out, st);
  case kQ3_K: return quantize_f<kQ3_K>(W, n, out, st);
  case kQ4_K: return quantize_f<kQ4_K>(W, n, out, st);
  case kQ5_K: return quantize_f<kQ5_K>(W, n, out, st);
  case kQ6_K: return quantize_f<kQ6_K>(W, n, out, st);
  case kIQ4_NL: return quantize_f<kIQ4_NL>(W, n, out, st);
  case kIQ4_XS: return quantize_f<kIQ4_XS>(W, n, out, st);
  default: return Status::err(kUnsupported, "format quantize: no quantizer for this format");
  }
}

Status format_relayout(int fmt, const FmtArgs& a, const uint8_t* blocks, int rows, hipStream_t st) {
  switch (fmt) {
  case kQ8_0: return relayout_f<kQ8_0>(a, blocks, rows, st);
  case kQ4_0: return relayout_f<kQ4_0>(a, blocks, rows, st);
  case kQ4_1: return relayout_f<kQ4_1>(a, blocks, rows, st);
  case kQ5_0: return relayout_f<kQ5_0>(a, blocks, rows, st);
  case kQ5_1: return relayout_f<kQ5_1>(a, blocks, rows, st);
  case kQ2_K: return relayout_f<kQ2_K>(a, blocks, rows, st);
  case kQ3_K: return relayout_f<kQ3_K>(a, blocks, rows, st);
  case kQ4_K: return relayout_f<kQ4_K>(a, blocks, rows, st);
  case kQ5_K: return relayout_f<kQ5_K>(a, blocks, rows, st);
  case kQ6_K: return relayout_f<kQ6_K>(a, blocks, rows, st);
  case kIQ4_NL: return relayout_f<kIQ4_NL>(a, blocks, rows, st);
  case kIQ4_XS: return relayout_f<kIQ4_XS>(a, blocks, rows, st);
  default: return Status::err(kGap, "gap? quant format not implemented");
  }
}

Status format_dequant(int fmt, const FmtArgs& a, int rows, float* out, hipStream_t st) {
  switch (fmt) {
  case kQ8_0: return dequant_f<kQ8_0>(a, rows, out, st);
  case kQ4_0: return dequant_f<kQ4_0>(a, rows, out, st);
  case kQ4_1: return dequant_f<kQ4_1>(a, rows, out, st);
  case kQ5_0: return dequant_f<kQ5_0>(a, rows, out, st);
  case kQ5_1: return dequant_f<kQ5_1>(a, rows, out, st);
  case kQ2_K: return dequant_f<kQ2_K>(a, rows, out, st);
  case kQ3_K: return dequant_f<kQ3_K>(a, rows, out, st);
  case kQ4_K: return dequant_f<kQ4_K>(a, rows, out, st);
  case kQ5_K: return dequant_f<kQ5_K>(a, rows, out, st);
  case kQ6_K: return dequant_f<kQ6_K>(a, rows, out, st);
  case kIQ4_NL: return dequant_f<kIQ4_NL>(a, rows, out, st);
  case kIQ4_XS: return dequant_f<kIQ4_XS>(a, rows, out, st);
  default: return Status::err(kGap, "gap? quant format not implemented");
  }
}

Status launch_format_gemv(int fmt, const FmtArgs& a, int batch, hipStream_t st) {
  if (a.nsub <= 0 || a.rows <= 0 || batch <= 0) return Status::err(kInvalid, "format gemv: shape");
  if ((reinterpret_cast<uintptr_t>(a.x) & 15u) || (a.x_stride % 4))
    return Status::err(kInvalid, "format gemv: x must be 16-byte aligned with a stride of 4k");
  switch (fmt) {
  case kQ8_0: return gemv_f<kQ8_0>(a, batch, st);
  case kQ4_0: return gemv_f<kQ4_0>(a, batch, st);
  case kQ4_1: return gemv_f<kQ4_1>(a, batch, st);
  case kQ5_0: return gemv_f<kQ5_0>(a, batch, st);
  case kQ5_1: return gemv_f<kQ5_1>(a, batch, st);
  case kQ2_K: return gemv_f<kQ2_K>(a, batch, st);
  case kQ3_K: return gemv_f<kQ3_K>(a, batch, st);
  case kQ4_K: return gemv_f<kQ4_K>(a, batch, st);
  case kQ5_K: return gemv_f<kQ5_K>(a, batch, st);
  case kQ6_K: return gemv_f<kQ6_K>(a, batch, st);
  case kIQ4_NL: return gemv_f<kIQ4_NL>(a, batch, st);
  case kIQ4_XS: return gemv_f<kIQ4_XS>(a, batch, st);
  default: return Status::err(kGap, "gap? quant format not implemented");
  }
}

}  // namespace wv
