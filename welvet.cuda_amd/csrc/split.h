// The activation split shared by the matrix-core GEMMs and the K-split
// reduce: operand-order fragments of 16 rows x 128 K of fp32 activations as
// E4M3 or FP6 (E2M3) terms with E8M0 block exponents, the layout the scaled
// f8f6f4 instructions read.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "codec.h"
#include "common.h"

namespace wv {

constexpr int kFragBytes = 2048;                  // one 16 x 128 E4M3 operand
constexpr int kFrag6Bytes = 1536;                 // one 16 x 128 FP6 (E2M3) operand
constexpr int kChunkScaleBytes = 256;             // one exponent dword per lane

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef short v2s __attribute__((ext_vector_type(2)));
// fp32 input rows in the global address space (global, not flat, loads)
typedef const __attribute__((address_space(1))) float* GlobalF;
typedef __attribute__((address_space(1))) uint8_t* GlobalU8;
typedef __attribute__((address_space(3))) uint8_t* LdsU8;

// Three-term splits hold FP6 (E2M3) terms: 0.75 byte per term and element
// instead of 1, and FP4 weights times FP6 terms run at the FP4/FP6 rate of
// the matrix cores. Two- and one-term splits hold E4M3 terms (two FP6 terms
// would sit at 7.8e-4 of the 1e-3 bound).
template <int NT>
constexpr bool act_fp6() {
  return NT == kTerms;
}

// The terms of one (16-row block, 128-wide K chunk) operand slice: lane l
// (row l % 16, group g = l / 16) holds its 32 values v[h][j], k = 64h + 16g +
// j. A 32-element block is held by lanes l and l ^ 16, which exchange their
// amax. Per term and half the lane stores its 16 codes with one 16-byte
// store at chunk + t * kFragBytes + h * 1024 + 16 l; the block exponents are
// gathered to the lanes that pass them to the instruction (row l % 16, block
// l / 16) and stored as one dword per lane at scales + 4 l (byte t: term t).
// AS: the address space of the destination (1 global, 3 LDS).
template <int AS, int NT = kTerms, bool STREAM = false>
__device__ __forceinline__ void split_terms(float (&v)[2][16],
                                            __attribute__((address_space(AS))) uint8_t* chunk,
                                            __attribute__((address_space(AS))) uint8_t* scales,
                                            int lane) {
  typedef __attribute__((address_space(AS))) i32x4 I4;
  typedef __attribute__((address_space(AS))) uint32_t U32;
  __attribute__((address_space(AS))) uint8_t* dst = chunk + lane * 16;
  const int i16 = lane & 15;
  // exponent of block b = l / 16 for row i16 comes from lane 32 (b & 1) + i16,
  // half b >> 1
  const int src = ((lane >> 4) & 1) * 32 + i16;
  uint32_t sword = 0x7F000000u;  // byte 3 unused
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int e[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float am = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) am = fmaxf(am, fabsf(v[h][j]));
      am = fmaxf(am, __shfl_xor(am, 16, 64));
      e[h] = e8m0_exponent(am, 448.0f);
      // scaled converters: divide by and multiply with 2^e exactly
      const float sc = pow2f(e[h]);
      int wq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v2s w = {0, 0};
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, v[h][4 * q], v[h][4 * q + 1], sc, false);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, v[h][4 * q + 2], v[h][4 * q + 3], sc, true);
        const int w4 = __builtin_bit_cast(int, w);
        wq[q] = w4;
        if (t + 1 < NT) {
          const v2f q0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w4, sc, false);
          const v2f q1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w4, sc, true);
          v[h][4 * q] -= q0.x, v[h][4 * q + 1] -= q0.y;
          v[h][4 * q + 2] -= q1.x, v[h][4 * q + 3] -= q1.y;
        }
      }
      const i32x4 codes = i32x4{wq[0], wq[1], wq[2], wq[3]};
      if constexpr (AS == 1 && STREAM)  // read by a later launch: streaming store
        __builtin_nontemporal_store(codes, reinterpret_cast<I4*>(dst + t * kFragBytes + h * 1024));
      else
        *reinterpret_cast<I4*>(dst + t * kFragBytes + h * 1024) = codes;
    }
    const int e0 = __shfl(e[0], src, 64), e1 = __shfl(e[1], src, 64);
    sword |= (uint32_t)(((lane >> 5) ? e1 : e0) + 127) << (8 * t);
  }
  if constexpr (AS == 1 && STREAM)
    __builtin_nontemporal_store(sword, reinterpret_cast<U32*>(scales + lane * 4));
  else
    *reinterpret_cast<U32*>(scales + lane * 4) = sword;
}

// FP6 terms of one (16-row block, 128-wide K chunk) operand slice. The
// f8f6f4 instruction's FP6 operand gives lane l (row l % 16, g = l / 16) the
// 32 values k = 32 g + p of one 32-element block, packed element p of the
// lane's six dwords; the converter packs its two 16-value inputs interleaved
// (element 2i from the first, 2i + 1 from the second). So the block's amax is
// the lane's own. Per term: e, the smallest exponent with amax <= 7.5 * 2^e
// (at least -126, so that 2^e is a normal float); the E2M3 codes of
// v * 2^-e, rounded to nearest-even by the converter (scale 2^e); the
// residual v - dec(code) * 2^e for the next term. The lane stores dwords 0-3 of its
// operand at chunk + t * kFrag6Bytes + 16 l, dwords 4-5 at chunk + t *
// kFrag6Bytes + 1024 + 8 l (both planes fully coalesced), and its exponents
// as one dword at scales + 4 l (byte t: term t).
template <int AS, int NT = kTerms, bool STREAM = false>
__device__ __forceinline__ void split_terms6(float (&v)[32],
                                             __attribute__((address_space(AS))) uint8_t* chunk,
                                             __attribute__((address_space(AS))) uint8_t* scales,
                                             int lane) {
  typedef __attribute__((address_space(AS))) i32x4 I4;
  typedef __attribute__((address_space(AS))) i32x2 I2;
  typedef __attribute__((address_space(AS))) uint32_t U32;
  uint32_t sword = 0x7F7F7F7Fu;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float am = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) am = fmaxf(am, fabsf(v[j]));
    int e = e8m0_exponent(am, 7.5f);
    e = e < -126 ? -126 : e;
    // the converters divide by and multiply with the power of two exactly
    // (the same bits as an explicit multiply by 2^-e and an unscaled convert)
    const float sc = pow2f(e);
    v16f lo, hi;
#pragma unroll
    for (int i = 0; i < 16; ++i) lo[i] = v[2 * i], hi[i] = v[2 * i + 1];
    const auto code = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(lo, hi, sc);
    if (t + 1 < NT) {
      const auto d = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(code, sc);
#pragma unroll
      for (int j = 0; j < 32; ++j) v[j] -= d[j];
    }
    const i32x4 c0 = i32x4{(int)code[0], (int)code[1], (int)code[2], (int)code[3]};
    const i32x2 c1 = i32x2{(int)code[4], (int)code[5]};
    I4* d0 = reinterpret_cast<I4*>(chunk + t * kFrag6Bytes + lane * 16);
    I2* d1 = reinterpret_cast<I2*>(chunk + t * kFrag6Bytes + 1024 + lane * 8);
    if constexpr (AS == 1 && STREAM) {
      __builtin_nontemporal_store(c0, d0);
      __builtin_nontemporal_store(c1, d1);
    } else {
      *d0 = c0;
      *d1 = c1;
    }
    sword = (sword & ~(0xFFu << (8 * t))) | ((uint32_t)(e + 127) << (8 * t));
  }
  if constexpr (AS == 1 && STREAM)
    __builtin_nontemporal_store(sword, reinterpret_cast<U32*>(scales + lane * 4));
  else
    *reinterpret_cast<U32*>(scales + lane * 4) = sword;
}

}  // namespace wv
