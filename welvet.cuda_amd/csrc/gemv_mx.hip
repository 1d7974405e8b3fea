// Quantized GEMV for 1-4 batch rows on the CDNA4 scaled matrix cores, over
// the weights in matrix-core operand order (DeviceWeights::codes_frag).
//
//   y[b][n] = rowscale[n] * sum_k x[b][k] * dec(W[n][k]) * blockscale[n][k/32]
//
// Weights. Per 16-row block and K chunk of 128 the operand a wave passes to
// v_mfma_scale_f32_16x16x128_f8f6f4 is stored contiguously (1 KiB for FP4,
// 2 x 1 KiB for FP8), so every weight load of a wave reads 1 KiB in one
// piece and a workgroup's 16 rows are one contiguous run. The matrix core
// takes the stored codes and their E8M0 block scales directly: nothing is
// decoded on the VALU.
//
// Activations. x is split into three E4M3 terms per 16-element piece: term t
// quantizes the residual of terms 0..t-1 with its own E8M0 exponent (the
// smallest with the piece's amax <= 448 * 2^e). The terms sit in the rows of
// the A operand, so one MFMA applies all three to a weight fragment. A lane's
// scale covers one 32-element block of one row, so the two 16-element halves
// of a block go to different rows, each with its own exponent: row 3h + t
// holds term t of the pieces that are half h of their block. Piece p of a
// chunk (k = 16p .. 16p + 15) is held by lane group p & 3 at byte 16 (p >> 2)
// (the FP8 operand layout: bytes 0-15 -> k = 16g + j, 16-31 -> k = 64 + 16g
// + j), so row 3h + t carries data only in lane groups g with g & 1 == h; its
// scale for block b is the exponent of piece 2b + h. The six accumulator
// rows (lanes g = 0: rows 0-3, g = 1: rows 4-5) add up to the product. More
// batch rows take six A rows each (rows 6b .. 6b + 5 for batch row b), so two
// rows share one MFMA per weight fragment and three or four take two.
//
// Work split. One workgroup per 16 weight rows (per matrix); its W waves cut
// K into ranges of at most NSW chunks. A wave issues the loads of its input
// first, then every weight load of its range; it splits its slice of x into
// its own LDS region while the weights arrive (or, with a pre-split input,
// loads the terms a producer wrote), runs one MFMA per chunk and matrix, and
// the partial sums of the waves meet in LDS for the epilogue (row scale,
// bias, activation, or the SwiGLU product). The SwiGLU gate+up launch can
// also write the three-term split of its output h for the down projection:
// each workgroup's 16 outputs are exactly one piece.
//
// Non-finite inputs. A wave whose slice of x holds inf or NaN (or whose
// pre-split pieces carry the 0xFF exponent that marks a non-finite piece)
// computes its partial sums on the VALU instead, from the weight codes read
// again and decoded exactly, so such inputs give the IEEE result of the fp32
// GEMV.
#include <type_traits>

#include "codec.h"
#include "act.h"
#include "common.h"
#include "kernels.h"
#include "wave.h"

namespace wv {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTermsMx = 3;
constexpr int kChunkCodeBytes = kTermsMx * 4 * 32;  // codes of one chunk's terms
constexpr int kChunkExpBytes = kTermsMx * 8;       // exponents: term x piece
constexpr uint8_t kNonFinite = 0xFF;               // exponent byte of a non-finite piece

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <int DT>
constexpr int wfmt() {
  return DT == kE4M3 ? 0 : DT == kE5M2 ? 1 : 4;
}

__device__ __forceinline__ u32x4 load_stream(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ float pair_max(float v) {  // lanes l, l ^ 1
  const int o = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false);
  return fmaxf(v, __builtin_bit_cast(float, o));
}

__device__ __forceinline__ bool finite_amax(float am) {
  return am <= 3.40282347e38f;  // false for inf and NaN
}

// Term t of 8 values with scale 2^e: the E4M3 codes of v / 2^e (two words)
// and v - dec(codes) * 2^e left in v. The scaled converters divide by and
// multiply with the scale exactly (same bits as an explicit multiply by the
// power of two, then the plain converter).
__device__ __forceinline__ int2 term8(float (&v)[8], float sc, bool residual) {
  v2s w0 = {0, 0}, w1 = {0, 0};
  w0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w0, v[0], v[1], sc, false);
  w0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w0, v[2], v[3], sc, true);
  w1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w1, v[4], v[5], sc, false);
  w1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w1, v[6], v[7], sc, true);
  const int c0 = __builtin_bit_cast(int, w0), c1 = __builtin_bit_cast(int, w1);
  if (residual) {
    const v2f d0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(c0, sc, false);
    const v2f d1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(c0, sc, true);
    const v2f d2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(c1, sc, false);
    const v2f d3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(c1, sc, true);
    v[0] -= d0.x, v[1] -= d0.y, v[2] -= d1.x, v[3] -= d1.y;
    v[4] -= d2.x, v[5] -= d2.y, v[6] -= d3.x, v[7] -= d3.y;
  }
  return make_int2(c0, c1);
}

// Exact partial sum of one lane's operand slice (row n of the fragment,
// its K positions) against x, for the non-finite fallback: FP4 nibble j ->
// k = 32 g + j; FP8 byte j -> k = 16 g + j (j < 16), 64 + 16 g + j - 16.
// Exact sum of one lane's operand slice against x for the non-finite
// fallback, one 4-byte word at a time (a rolled loop: this path must not add
// register pressure to the matrix-core path). FP4 word d holds nibbles 8d ..
// 8d + 7 (k = 32 g + 8d + j); FP8 word d < 4 holds k = 16 g + 4d + j, word
// d >= 4 k = 64 + 16 g + 4 (d - 4) + j. Each word is scaled by the exponent
// of its block (lanes e_lo for FP4 and FP8 words 0-3, e_hi for FP8 words 4-7).
template <int DT>
__device__ float exact_slice(const uint8_t* w, const float* x, int k0, int g, int cols,
                             float s_lo, float s_hi) {
  constexpr int WORDS = DT == kFP4 ? 4 : 8;
  float s = 0.0f;
#pragma unroll 1
  for (int d = 0; d < WORDS; ++d) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(w + (d < 4 ? 4 * d : 1024 + 4 * (d - 4)));
    float p = 0.0f;
    if constexpr (DT == kFP4) {
      const int k = k0 + 32 * g + 8 * d;
      float q[8];
      const v2f a0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, 1.0f, 0);
      const v2f a1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, 1.0f, 1);
      const v2f a2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, 1.0f, 2);
      const v2f a3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, 1.0f, 3);
      q[0] = a0[0], q[1] = a0[1], q[2] = a1[0], q[3] = a1[1];
      q[4] = a2[0], q[5] = a2[1], q[6] = a3[0], q[7] = a3[1];
#pragma unroll
      for (int j = 0; j < 8; ++j) p = fmaf(q[j], k + j < cols ? x[k + j] : 0.0f, p);
      s = fmaf(p, s_lo, s);
    } else {
      const int k = k0 + (d < 4 ? 16 * g + 4 * d : 64 + 16 * g + 4 * (d - 4));
      const v2f a0 = DT == kE4M3 ? __builtin_amdgcn_cvt_pk_f32_fp8(v, false)
                                 : __builtin_amdgcn_cvt_pk_f32_bf8(v, false);
      const v2f a1 = DT == kE4M3 ? __builtin_amdgcn_cvt_pk_f32_fp8(v, true)
                                 : __builtin_amdgcn_cvt_pk_f32_bf8(v, true);
      const float q[4] = {a0[0], a0[1], a1[0], a1[1]};
#pragma unroll
      for (int j = 0; j < 4; ++j) p = fmaf(q[j], k + j < cols ? x[k + j] : 0.0f, p);
      s = fmaf(p, d < 4 ? s_lo : s_hi, s);
    }
  }
  return s;
}

// NB batch rows (1..4). Row r = 6 b + 3 h + t of the A operand rows of all
// MFMAs (MFMA j takes rows 16 j .. 16 j + 15) holds term t of half h of
// batch row b, so NMF = ceil(6 NB / 16) MFMAs per weight fragment: one for
// 1-2 rows, two for 3-4. Accumulator lane (n, g) of MFMA j holds rows
// 16 j + 4 g .. + 3 of column n: all four of one batch row, or, when
// 16 j + 4 g = 4 mod 6, two of batch row (16 j + 4 g) / 6 and two of the
// next.
// PRE: the input is a pre-split image per batch row (a.asplit); otherwise the
// waves split a.x themselves. NEXT (MATS == 2): write the split of h to
// a.next.
template <int DT, bool BLK, int MATS, int NB, int W, int NSW, bool PRE, bool NEXT, bool ALIGNED = false>
__global__ __launch_bounds__(64 * W) void k_gemv_mx(GemvMxArgs a) {
  constexpr bool FP4 = DT == kFP4;
  constexpr int NMF = (6 * NB + 15) / 16;  // MFMAs per weight fragment
  constexpr int XI = NSW * 16;             // split items (8 values) per batch row
  constexpr int XR = (NB * XI + 63) / 64;  // split rounds of 64 items
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int S = a.kpad / 128;
  const int s0 = wave * S / W, s1 = (wave + 1) * S / W, ns = s1 - s0;
  const int rb = blockIdx.x, n0 = 16 * rb;
  // bytes of one batch row's pre-split image
  const size_t img = (size_t)(PRE ? a.asplit_steps : a.next_steps) * (kChunkCodeBytes + kChunkExpBytes);

  __shared__ __attribute__((aligned(16))) uint8_t lds_c[W][NSW][NB][kChunkCodeBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_e[W][NSW][NB][kChunkExpBytes];
  // the waves' partial sums: one batch row in a buffer of their own; more
  // rows in each wave's staging region, dead once its MFMAs are issued
  constexpr int PARTF = MATS * NMF * 4 * 16 * 2;  // floats per wave (NB > 1)
  static_assert(NB == 1 || PARTF * 4 + NB * 48 <= NSW * NB * kChunkCodeBytes, "partials fit the staging");
  __shared__ float part[NB == 1 ? W : 1][MATS][16][2];
  auto part_w = [&](int w) { return reinterpret_cast<float*>(&lds_c[w][0][0][0]); };

  // 1. the input: this wave's chunks of the pre-split images (16-byte pieces:
  // 24 per chunk of codes, then the exponents), or x for the split below
  constexpr int PU = NSW * (kChunkCodeBytes / 16);  // code pieces per batch row
  constexpr int EU = NSW * (kChunkExpBytes / 4);    // exponent dwords per batch row
  constexpr int PR = (NB * PU + 63) / 64;
  u32x4 pc[PRE ? PR : 1];
  uint32_t pe[PRE ? (NB * EU + 63) / 64 : 1];
  float4 xv[PRE ? 1 : XR][2];
  if constexpr (PRE) {
    const int SA = a.asplit_steps;
    const int valid = (a.cols + 15) / 16;  // pieces ever written
#pragma unroll
    for (int r = 0; r < PR; ++r) {
      // batch row b, chunk i, 16-byte piece v of its codes
      const int u = r * 64 + lane, b = NB == 1 ? 0 : u / PU, i = (u - b * PU) / 24, v = (u - b * PU) % 24;
      // v = 2 (4 t + g) + hi: piece 8 s + g + 4 hi of term t
      const int s = s0 + (i < ns ? i : 0), pc_piece = 8 * s + ((v >> 1) & 3) + 4 * (v & 1);
      // every load unconditional (from a clamped address, then selected):
      // a branch around a load makes the compiler wait for all loads at the join
      const u32x4 t = *reinterpret_cast<const u32x4*>(a.asplit + (b < NB ? b : 0) * img +
                                                      (size_t)s * kChunkCodeBytes + 16 * v);
      const bool live = b < NB && i < ns && pc_piece < valid;  // NB == 1: i < ns covers the tail
      pc[r] = live ? t : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int r = 0; r < (int)(sizeof(pe) / 4); ++r) {
      const int u = r * 64 + lane, b = NB == 1 ? 0 : u / EU, i = (u - b * EU) / (kChunkExpBytes / 4),
                v = (u - b * EU) % (kChunkExpBytes / 4);
      const uint32_t t = *reinterpret_cast<const uint32_t*>(
          a.asplit + (b < NB ? b : 0) * img + (size_t)SA * kChunkCodeBytes +
          (size_t)(s0 + (i < ns ? i : 0)) * kChunkExpBytes + 4 * v);
      pe[r] = b < NB && i < ns ? t : 0x7F7F7F7Fu;
    }
  } else {
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int it = r * 64 + lane, b = NB == 1 ? 0 : it / XI, i = (it - b * XI) >> 4, q = it & 15;
      const int k = (s0 + i) * 128 + 8 * q;
      // x 16-byte aligned and cols % 4 == 0 (launch_gemv_mx checks): the
      // two float4 of an item are wholly inside or outside [0, cols)
      const bool live0 = b < NB && i < ns && k < a.cols, live1 = b < NB && i < ns && k + 4 < a.cols;
      const float* xb = a.x + (size_t)(b < NB ? b : 0) * a.cols;
      const float4 t0 = *reinterpret_cast<const float4*>(xb + (live0 ? k : 0));
      const float4 t1 = *reinterpret_cast<const float4*>(xb + (live1 ? k + 4 : 0));
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
      xv[r][0] = live0 ? t0 : z;
      xv[r][1] = live1 ? t1 : z;
    }
  }

  // the epilogue's row scales (and bias) early, so the epilogue waits for no
  // global load (wave 0 computes it: lane l for row n0 + l % 16)
  float rs[MATS];
#pragma unroll
  for (int m = 0; m < MATS; ++m) rs[m] = wave == 0 ? a.scale[m][n0 + n] : 1.0f;
  const int ob = n0 + n;
  const double bias = wave == 0 && MATS == 1 && a.bias && ob < a.bias_len ? a.bias[ob] : 0.0;

  // 2. every weight load of this wave's range in flight
  constexpr int H = FP4 ? 1 : 2;
  // exponent dwords (groups of 4 chunks) that NSW consecutive chunks from
  // any start touch: (s0 + NSW - 1) / 4 - s0 / 4 <= (NSW + 2) / 4
  // (ALIGNED: every range is NSW chunks from a multiple of 4, NSW / 4 groups)
  constexpr int EG = ALIGNED ? NSW / 4 : (NSW + 2) / 4 + 1;
  u32x4 wl[MATS][NSW], wh[MATS][FP4 ? 1 : NSW];
  uint32_t we[MATS][BLK ? EG : 1];
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
    const uint8_t* f = a.codesf[m] + (size_t)rb * S * (H * 1024) + lane * 16;
#pragma unroll
    for (int i = 0; i < NSW; ++i) {
      // chunks past the range load the range's last one again (cache hits;
      // no MFMA uses them)
      const int s = s0 + i < s1 ? s0 + i : s1 - 1;
      wl[m][i] = load_stream(f + (size_t)s * (H * 1024));
      if constexpr (!FP4) wh[m][i] = load_stream(f + (size_t)s * (H * 1024) + 1024);
    }
    if constexpr (BLK) {
      const int groups = (S + 3) / 4;
#pragma unroll
      for (int j = 0; j < EG; ++j) {
        const int grp = s0 / 4 + j, gc = grp < groups ? grp : groups - 1;
        const uint32_t t = *reinterpret_cast<const uint32_t*>(a.blkf[m] + (((size_t)rb * groups + gc) * 64 + lane) * 4);
        we[m][j] = grp < groups ? t : 0x7F7F7F7Fu;
      }
    }
  }

  // 3. the split of this wave's slice of x (three E4M3 terms per piece)
  bool bad = false;
  if constexpr (!PRE) {
    bool nonfinite = false;
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int it = r * 64 + lane, b = NB == 1 ? 0 : it / XI, i = (it - b * XI) >> 4, q = it & 15, p = q >> 1;
      // staged item: one batch row stages chunks i < NSW (the last round's
      // tail is past them)
      const bool staged = NB == 1 ? i < NSW : b < NB;
      float v[8] = {xv[r][0].x, xv[r][0].y, xv[r][0].z, xv[r][0].w,
                    xv[r][1].x, xv[r][1].y, xv[r][1].z, xv[r][1].w};
      const int cb = (p & 3) * 32 + 16 * (p >> 2) + 8 * (q & 1);
      uint32_t eb = 0;
      // fmaxf passes over NaN, so inf and NaN are caught by the plain sum
      // (a finite sum that overflows only sends the wave to the exact path)
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += v[j];
      nonfinite |= !finite_amax(fabsf(sum));
#pragma unroll
      for (int t = 0; t < kTermsMx; ++t) {
        float am = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) am = fmaxf(am, fabsf(v[j]));
        am = pair_max(am);
        const int e = e8m0_exponent(am, 448.0f);
        const int2 c = term8(v, pow2f(e), t + 1 < kTermsMx);
        if (staged) *reinterpret_cast<int2*>(&lds_c[wave][i][b][t * 128 + cb]) = c;
        eb |= (uint32_t)(e + 127) << (8 * t);
      }
      if ((q & 1) == 0 && staged) {
#pragma unroll
        for (int t = 0; t < kTermsMx; ++t) lds_e[wave][i][b][t * 8 + p] = (uint8_t)(eb >> (8 * t));
      }
    }
    bad = __ballot(nonfinite) != 0;
    // LDS writes of this wave complete before its lanes read them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    // the pre-split chunks into this wave's LDS; exponent bytes of pieces
    // that were never written read as 127 (their codes as zero)
    const int valid = (a.cols + 15) / 16;
    bool marked = false;
#pragma unroll
    for (int r = 0; r < PR; ++r) {
      const int u = r * 64 + lane, b = NB == 1 ? 0 : u / PU, i = (u - b * PU) / 24, v = (u - b * PU) % 24;
      if (NB == 1 ? i < NSW : b < NB) *reinterpret_cast<u32x4*>(&lds_c[wave][i][b][16 * v]) = pc[r];
    }
#pragma unroll
    for (int r = 0; r < (int)(sizeof(pe) / 4); ++r) {
      const int u = r * 64 + lane, b = NB == 1 ? 0 : u / EU, i = (u - b * EU) / (kChunkExpBytes / 4),
                v = (u - b * EU) % (kChunkExpBytes / 4);
      uint32_t w = pe[r];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int piece = 8 * (s0 + i) + ((4 * v + c) & 7);
        const uint32_t e = (w >> (8 * c)) & 0xFFu;
        if (piece >= valid) w = (w & ~(0xFFu << (8 * c))) | (127u << (8 * c));
        else marked |= b < NB && i < ns && e == kNonFinite;
      }
      if (NB == 1 ? i < NSW : b < NB) *reinterpret_cast<uint32_t*>(&lds_e[wave][i][b][4 * v]) = w;
    }
    bad = __ballot(marked) != 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // 4. NMF MFMAs per chunk and matrix, or the exact VALU sums. Lane (n, g)
  // of MFMA j sums into batch row bl[j] (its rows 0-3, or rows 0-1 when
  // two[j]) and bl[j] + 1 (rows 2-3 when two[j]).
  float plo[MATS][NMF], phi[MATS][NMF];
  if (!bad) {
    // A row 16 j + n: batch row ab[j], half ah[j], term at[j]; rows past
    // 6 NB are zero
    int ab[NMF], ah[NMF], at[NMF];
    bool arow[NMF], adata[NMF];
#pragma unroll
    for (int j = 0; j < NMF; ++j) {
      const int r = 16 * j + n;
      ab[j] = r / 6, ah[j] = (r % 6) / 3, at[j] = r % 3;
      arow[j] = ab[j] < NB, adata[j] = arow[j] && (g & 1) == ah[j];
      if (NB == 1 || !arow[j]) ab[j] = 0;
    }
    // A fragments from LDS, read one chunk ahead of their MFMAs
    auto read_a = [&](int i, v8i (&A)[NMF], int (&asc)[NMF]) {
#pragma unroll
      for (int j = 0; j < NMF; ++j) {
        A[j] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
        asc[j] = 127;
        if (arow[j]) {
          if (adata[j]) {
            const uint8_t* c = &lds_c[wave][i][ab[j]][at[j] * 128 + g * 32];
            const int4 lo = *reinterpret_cast<const int4*>(c);
            const int4 hi = *reinterpret_cast<const int4*>(c + 16);
            A[j] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
          }
          asc[j] = lds_e[wave][i][ab[j]][at[j] * 8 + 2 * g + ah[j]];
        }
      }
    };
    v8i A[2][NMF];
    int asc[2][NMF];
    read_a(0, A[0], asc[0]);
    v4f acc[MATS][NMF];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < NMF; ++j) acc[m][j] = v4f{0.f, 0.f, 0.f, 0.f};
    static_for<0, NSW>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if (i < ns) {
        if constexpr (i + 1 < NSW) read_a(i + 1, A[(i + 1) & 1], asc[(i + 1) & 1]);
        const int s = s0 + i;
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
          v8i B;
          if constexpr (FP4) B = v8i{(int)wl[m][i].x, (int)wl[m][i].y, (int)wl[m][i].z, (int)wl[m][i].w, 0, 0, 0, 0};
          else B = v8i{(int)wl[m][i].x, (int)wl[m][i].y, (int)wl[m][i].z, (int)wl[m][i].w,
                       (int)wh[m][i].x, (int)wh[m][i].y, (int)wh[m][i].z, (int)wh[m][i].w};
          int wsc = 127;
          if constexpr (BLK) wsc = (int)((we[m][(s >> 2) - (s0 >> 2)] >> (8 * (s & 3))) & 0xFFu);
#pragma unroll
          for (int j = 0; j < NMF; ++j)
            acc[m][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[i & 1][j], B, acc[m][j], 0, wfmt<DT>(),
                                                                         0, asc[i & 1][j], 0, wsc);
        }
      }
    });
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < NMF; ++j) {
        const bool two = (16 * j + 4 * g) % 6 == 4;  // rows 2-3 start the next batch row
        const float lo = acc[m][j][0] + acc[m][j][1], hi = acc[m][j][2] + acc[m][j][3];
        plo[m][j] = two ? lo : lo + hi;
        phi[m][j] = two ? hi : 0.0f;
      }
  } else {
    // the weights are read again here, so the registers above are dead on
    // this path; each batch row's exact sum lands in the slot the epilogue
    // reads first for it
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
#pragma unroll
      for (int j = 0; j < NMF; ++j) plo[m][j] = phi[m][j] = 0.0f;
      const uint8_t* f = a.codesf[m] + (size_t)rb * S * (H * 1024) + lane * 16;
#pragma unroll 1
      for (int b = 0; b < NB; ++b) {
        float s_ = 0.0f;
#pragma unroll 1
        for (int s = s0; s < s1; ++s) {
          float s_lo = 1.0f, s_hi = 1.0f;
          if constexpr (BLK) {
            // lane (n, g) takes the exponent of block g of chunk s; its FP4
            // nibbles are block g, its FP8 bytes blocks g / 2 (bytes 0-15) and
            // 2 + g / 2 (bytes 16-31), whose exponents other lanes take
            const int groups = (S + 3) / 4;
            const int e = a.blkf[m][(((size_t)rb * groups + (s >> 2)) * 64 + lane) * 4 + (s & 3)];
            if constexpr (FP4) {
              s_lo = pow2f(e - 127);
            } else {
              s_lo = pow2f(__shfl(e, n + 16 * (g >> 1), 64) - 127);
              s_hi = pow2f(__shfl(e, n + 16 * (2 + (g >> 1)), 64) - 127);
            }
          }
          s_ += exact_slice<DT>(f + (size_t)s * (H * 1024), a.x + (size_t)b * a.cols, 128 * s, g, a.cols,
                                s_lo, s_hi);
        }
        // the four lane groups of row n
        s_ += __shfl_xor(s_, 16, 64);
        s_ += __shfl_xor(s_, 32, 64);
        if constexpr (NB == 1) {
          plo[m][0] = g == 0 ? s_ : 0.0f;  // the lanes of group 1 store a zero
        } else {
          // batch row b's first rows sit in group G = 6 b / 4 (MFMA G / 4,
          // lane group G % 4), in its upper slot when 6 b % 4 == 2
#pragma unroll
          for (int j = 0; j < NMF; ++j) {
            if (4 * j + g == 6 * b / 4) {
              if ((6 * b) % 4 == 2) phi[m][j] = s_;
              else plo[m][j] = s_;
            }
          }
        }
      }
    }
  }
  if constexpr (NB == 1) {
    if (g < 2) {
#pragma unroll
      for (int m = 0; m < MATS; ++m) part[wave][m][n][g] = plo[m][0];
    }
  } else {
    float* pw = part_w(wave);
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < NMF; ++j)
        *reinterpret_cast<float2*>(&pw[((m * NMF + j) * 4 + g) * 32 + 2 * n]) = make_float2(plo[m][j], phi[m][j]);
  }
  __syncthreads();

  // 5. epilogue in wave 0: lane (n, g) computes row n0 + n of batch row g
  // (one batch row: the four lane groups alike, so that the 16-lane DPP
  // maxima below run with every lane active); lanes of batch rows < NB store
  if (wave != 0) return;
  const int o = n0 + n;
  const int bq = NB == 1 ? 0 : (g < NB ? g : NB - 1);
  const bool store = NB == 1 ? g == 0 : g < NB;
  float tot[MATS];
#pragma unroll
  for (int m = 0; m < MATS; ++m) {
    if constexpr (NB == 1) {
      float sum = part[0][m][n][0] + part[0][m][n][1];
#pragma unroll
      for (int w = 1; w < W; ++w) sum += part[w][m][n][0] + part[w][m][n][1];
      tot[m] = sum * rs[m];
    } else {
      // rows 6 bq .. 6 bq + 5: groups G1 = 6 bq / 4 (upper slot when it
      // starts with the previous batch row) and G1 + 1 (lower slot)
      const int G1 = 6 * bq / 4;
      const int i1 = ((m * NMF + G1 / 4) * 4 + G1 % 4) * 32 + 2 * n + ((6 * bq) % 4 == 2 ? 1 : 0);
      const int G2 = G1 + 1;
      const int i2 = ((m * NMF + G2 / 4) * 4 + G2 % 4) * 32 + 2 * n;
      float sum = part_w(0)[i1] + part_w(0)[i2];
#pragma unroll
      for (int w = 1; w < W; ++w) sum += part_w(w)[i1] + part_w(w)[i2];
      tot[m] = sum * rs[m];
    }
  }
  const size_t ob_out = (size_t)bq * a.rows + o;
  if constexpr (MATS == 2) {
    const float gt = (float)act_f64(kSilu, (double)tot[0]);
    const float h = (float)((double)gt * (double)tot[1]);
    if (store && o < a.rows) a.pre[ob_out] = h;
    if constexpr (NEXT) {
      // the three-term split of this piece (outputs n0 .. n0 + 15 of batch
      // row bq) for the next product
      float v = o < a.rows ? h : 0.0f;
      auto piece_max = [&](float t) {
        t = fmaxf(t, xor_lane<1>(t, lane));
        t = fmaxf(t, xor_lane<2>(t, lane));
        t = fmaxf(t, xor_lane<4>(t, lane));
        return fmaxf(t, xor_lane<8>(t, lane));
      };
      const float am0 = piece_max(finite_amax(fabsf(v)) ? fabsf(v) : __builtin_inff());  // NaN as inf
      const bool fin = finite_amax(am0);
      const int s = rb >> 3, p = rb & 7;
      uint8_t* codes = a.next + bq * img + (size_t)s * kChunkCodeBytes + (p & 3) * 32 + 16 * (p >> 2);
      uint8_t* exps = a.next + bq * img + (size_t)a.next_steps * kChunkCodeBytes + (size_t)s * kChunkExpBytes + p;
      // the terms' 16 code bytes each meet in LDS (a region this wave alone
      // uses now), then lanes 0-2 of the batch row store 16 bytes each
      uint8_t* gather = (NB == 1 ? reinterpret_cast<uint8_t*>(&part[0][0][0][0])
                                 : reinterpret_cast<uint8_t*>(part_w(0) + PARTF)) + bq * 48;
      // one batch row: fin is the same in every lane, and the DPP maxima
      // inside the branch run with every lane active. More rows: every lane
      // runs the terms (of zeros where its piece is not finite), the stores
      // are selected.
      if (NB == 1 && !fin) {
        if (lane == 0) {
#pragma unroll
          for (int t = 0; t < kTermsMx; ++t) exps[t * 8] = kNonFinite;
        }
      } else {
        if (!fin) v = 0.0f;
        float am = fin ? am0 : 0.0f;
#pragma unroll
        for (int t = 0; t < kTermsMx; ++t) {
          if (t > 0) am = piece_max(fabsf(v));
          const int e = e8m0_exponent(am, 448.0f);
          const float sc = pow2f(e);
          v2s w = {0, 0};
          w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, v, 0.0f, sc, false);
          const int code = __builtin_bit_cast(int, w) & 0xFF;
          if (store) gather[t * 16 + n] = (uint8_t)code;
          if (t + 1 < kTermsMx) v -= __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(code, sc, false)[0];
          if (store && n == 0) exps[t * 8] = fin ? (uint8_t)(e + 127) : kNonFinite;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // a non-finite piece keeps whatever codes it had: its 0xFF exponents
        // send the reader to the exact path over h
        if (store && fin && n < kTermsMx)
          *reinterpret_cast<int4*>(codes + n * 128) = *reinterpret_cast<const int4*>(gather + n * 16);
      }
    }
  } else {
    if (!store || o >= a.rows) return;
    float y = tot[0];
    if (a.need_epi) {
      double v = (double)y;
      if (a.bias && o < a.bias_len) {
        v += bias;
        y = (float)v;
      }
      a.pre[ob_out] = y;
      a.post[ob_out] = (float)act_f64(a.act, v);
    } else {
      a.pre[ob_out] = y;
      if (a.post && a.post != a.pre) a.post[ob_out] = y;
    }
  }
}

// Waves per workgroup and chunks per wave for kpad / 128 = S chunks (chunks
// past a wave's range are loaded again and not used, so the step count
// tracks S / W closely). A wave holds all its weight operands in registers,
// so 16 waves (128 VGPRs each) take 8 chunks only of one FP4 matrix, 4 of
// one FP8 matrix or of two FP4 matrices; two FP8 matrices run 8 waves
// (S <= 32) only. The staged terms take W x NSW x NB x 408 bytes of LDS, so
// 16 waves of 8 chunks run at most 3 batch rows.
constexpr int max_chunks(int dtype, int mats, int nb) {
  return dtype == kFP4 ? (mats == 1 ? (nb <= 3 ? 128 : 96) : 64) : (mats == 1 ? 64 : 32);
}

template <int DT, bool BLK, int MATS, int NB, int W, int NSW, bool PRE, bool NEXT, bool ALIGNED = false>
Status launch_t(const GemvMxArgs& a, hipStream_t st) {
  static_assert(W * NSW * NB * (kChunkCodeBytes + kChunkExpBytes) + (NB == 1 ? W * MATS * 128 : 0) <= 160 * 1024,
                "LDS of one workgroup");
  const unsigned grid = (unsigned)((a.rows + 15) / 16);
  k_gemv_mx<DT, BLK, MATS, NB, W, NSW, PRE, NEXT, ALIGNED><<<grid, 64 * W, 0, st>>>(a);
  return hip_status(hipGetLastError(), "gemv_mx launch");
}

template <int DT, bool BLK, int MATS, int NB, bool PRE, bool NEXT>
Status launch_shape(const GemvMxArgs& a, hipStream_t st) {
  const int S = a.kpad / 128;
  // 32 chunks over 8 waves: each range is one exponent group
  if constexpr (BLK)
    if (S == 32) return launch_t<DT, BLK, MATS, NB, 8, 4, PRE, NEXT, true>(a, st);
  if (S <= 32) return launch_t<DT, BLK, MATS, NB, 8, 4, PRE, NEXT>(a, st);
  if constexpr (DT == kFP4 || MATS == 1)
    if (S <= 64) return launch_t<DT, BLK, MATS, NB, 16, 4, PRE, NEXT>(a, st);
  if constexpr (DT == kFP4 && MATS == 1) {
    if (S <= 96) return launch_t<DT, BLK, MATS, NB, 16, 6, PRE, NEXT>(a, st);
    if constexpr (NB <= 3) return launch_t<DT, BLK, MATS, NB, 16, 8, PRE, NEXT>(a, st);
  }
  return Status::err(kUnsupported, "gemv_mx: K");
}

template <int DT, bool BLK, int NB>
Status launch_nb(const GemvMxArgs& a, hipStream_t st) {
  if (a.mats == 2) {
    return a.next ? launch_shape<DT, BLK, 2, NB, false, true>(a, st)
                  : launch_shape<DT, BLK, 2, NB, false, false>(a, st);
  }
  return a.asplit ? launch_shape<DT, BLK, 1, NB, true, false>(a, st)
                  : launch_shape<DT, BLK, 1, NB, false, false>(a, st);
}

template <int DT, bool BLK>
Status launch_dt(const GemvMxArgs& a, hipStream_t st) {
  switch (a.nb) {
  case 1: return launch_nb<DT, BLK, 1>(a, st);
  case 2: return launch_nb<DT, BLK, 2>(a, st);
  case 3: return launch_nb<DT, BLK, 3>(a, st);
  case 4: return launch_nb<DT, BLK, 4>(a, st);
  }
  return Status::err(kUnsupported, "gemv_mx: batch rows");
}

}  // namespace

bool gemv_mx_fits(int dtype, int rows, int kpad, int mats, int nb) {
  if (dtype != kE4M3 && dtype != kE5M2 && dtype != kFP4) return false;
  const int S = kpad / 128;
  // whole-GPU grids only (one workgroup per 16 rows per CU or more), and K
  // ranges that the instantiated shapes cover
  return mats >= 1 && mats <= 2 && nb >= 1 && nb <= kGemvMxMaxRows && (rows + 15) / 16 >= 256 &&
         S >= 16 && S <= max_chunks(dtype, mats, nb) && kpad % 128 == 0;
}

size_t gemv_mx_split_bytes(int kpad) {
  const size_t S = (size_t)kpad / 128;
  return S * (kChunkCodeBytes + kChunkExpBytes);
}

Status launch_gemv_mx(const GemvMxArgs& a, int dtype, bool blk, hipStream_t st) {
  if (!gemv_mx_fits(dtype, a.rows, a.kpad, a.mats, a.nb) || !a.codesf[0] || !a.scale[0] || !a.pre ||
      (a.mats == 2 && (!a.codesf[1] || !a.scale[1])) || (blk && (!a.blkf[0] || (a.mats == 2 && !a.blkf[1]))) ||
      !a.x || (a.asplit && (a.mats != 1 || a.asplit_steps < a.kpad / 128)) ||
      // the split of x reads 16-byte vectors
      (!a.asplit && (a.cols % 4 != 0 || (reinterpret_cast<uintptr_t>(a.x) & 15u) != 0)) ||
      (a.next && (a.mats != 2 || a.next_steps < (a.rows + 127) / 128)) ||
      (a.mats == 1 && a.need_epi && !a.post))
    return Status::err(kInvalid, "gemv_mx: arguments");
  switch (dtype) {
  case kE4M3: return blk ? launch_dt<kE4M3, true>(a, st) : launch_dt<kE4M3, false>(a, st);
  case kE5M2: return blk ? launch_dt<kE5M2, true>(a, st) : launch_dt<kE5M2, false>(a, st);
  case kFP4: return blk ? launch_dt<kFP4, true>(a, st) : launch_dt<kFP4, false>(a, st);
  }
  return Status::err(kUnsupported, "gemv_mx: dtype");
}

}  // namespace wv
