// Cross-lane reductions of a 64-lane wave, shared by the GEMV kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace wv {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Value of lane (lane ^ D). Distances inside a 16-lane row are DPP moves
// (VALU, no LDS round trip): quad_perm for 1 and 2, row_shl/row_shr:4 with
// a select for 4, row_ror:8 for 8; 16 and 32 cross rows and use bpermute.
// A DPP move must run with every lane active: a disabled source lane reads
// as out of bounds. So both moves for distance 4 execute unconditionally and
// a select picks between them; they may not sit in the arms of a branch.
template <int D>
__device__ __forceinline__ float xor_lane(float v, int lane) {
  if constexpr (D == 1) {
    return dpp<0xB1>(v);
  } else if constexpr (D == 2) {
    return dpp<0x4E>(v);
  } else if constexpr (D == 4) {
    const float from_above = dpp<0x104>(v);  // row_shl:4, lane i reads i + 4
    const float from_below = dpp<0x114>(v);  // row_shr:4, lane i reads i - 4
    return (lane & 4) ? from_below : from_above;
  } else if constexpr (D == 8) {
    return dpp<0x128>(v);
  } else {
    return __shfl_xor(v, D, 64);
  }
}

// Folds v[0..N) across lanes that differ in bit D: the lane with the bit
// clear keeps the lower half, the other the upper half.
template <int N, int D>
__device__ __forceinline__ void fold(float* v, int lane) {
  const bool up = (lane & D) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float send = up ? v[i] : v[i + N / 2];
    const float keep = up ? v[i + N / 2] : v[i];
    v[i] = keep + xor_lane<D>(send, lane);
  }
}

template <int R>
constexpr int log2c() {
  return R >= 32 ? 5 : R >= 16 ? 4 : R >= 8 ? 3 : R >= 4 ? 2 : R >= 2 ? 1 : 0;
}

// Reduces v[0..R) (R <= 32) over the 64 lanes with a transposing butterfly (R/2 + R/4
// + ... exchanges instead of 6 per row), folding the low lane bits first so
// the multi-value steps are DPP moves. Afterwards lanes 0..R-1 hold in v[0]
// the totals of rows reduced_row<R>(lane).
template <int R>
__device__ __forceinline__ void wave_reduce_rows(float* v, int lane) {
  constexpr int L = log2c<R>();
  // fold j halves the values over lane bit j: 2^L values -> 1
  if constexpr (L >= 5) fold<32, 1>(v, lane);
  if constexpr (L >= 4) fold<16, (1 << (L - 4))>(v, lane);
  if constexpr (L >= 3) fold<8, (1 << (L - 3))>(v, lane);
  if constexpr (L >= 2) fold<4, (1 << (L - 2))>(v, lane);
  if constexpr (L >= 1) fold<2, (1 << (L - 1))>(v, lane);
  // the lane bits above the folded ones: plain sums
  if constexpr (L < 1) v[0] += xor_lane<1>(v[0], lane);
  if constexpr (L < 2) v[0] += xor_lane<2>(v[0], lane);
  if constexpr (L < 3) v[0] += xor_lane<4>(v[0], lane);
  if constexpr (L < 4) v[0] += xor_lane<8>(v[0], lane);
  if constexpr (L < 5) v[0] += xor_lane<16>(v[0], lane);
  v[0] += xor_lane<32>(v[0], lane);
}

// Row whose total lane `lane` holds after wave_reduce_rows<R>: lane bit b
// decided row bit (L - 1 - b).
template <int R>
__device__ __forceinline__ int reduced_row(int lane) {
  constexpr int L = log2c<R>();
  int row = 0;
#pragma unroll
  for (int b = 0; b < L; ++b) row |= ((lane >> b) & 1) << (L - 1 - b);
  return row;
}

}  // namespace wv
