// Batched quantized GEMM on the CDNA4 scaled matrix cores.
//
//   C[m][n] = rowscale[n] * sum_k x[m][k] * dec(W[n][k]) * blockscale[n][k/32]
//
// x (fp32) is first split into kTerms E4M3 terms with per-32 E8M0 scales
// (k_split: each term quantizes the residual of the previous ones, so
// x ~ sum_t a_t 2^e_t with a relative residual of ~2^-12 for three terms).
// The terms act as extra K: every term is multiplied by the same weight tile
// and accumulated into the same fp32 accumulator by
// v_mfma_scale_f32_16x16x128_f8f6f4, which takes the stored FP8/FP4 weight
// codes and their E8M0 block scales directly.
//
// Tiling: a 256-thread workgroup computes a BM x 64 tile of C; per 128-wide K
// step it stages the A terms, the weight codes and both scale sets in LDS
// (rows padded by 16 bytes so 16-byte fragment reads are bank-conflict free),
// then each wave runs its MFMAs. Operand layout of the instruction (lane l,
// group g = l/16): FP8 bytes 0-15 -> k = 16g + j, bytes 16-31 -> k = 64 + 16g
// + j; FP4 nibble j -> k = 32g + j; scale of lane l: row l%16, block g;
// D: col l%16, rows 4g + r.
#include "codec.h"
#include "common.h"
#include "kernels.h"

namespace wv {
namespace {

constexpr int kBN = 64;
constexpr int kThreads = 256;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
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

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Maximum over the 8 lanes l ^ {1, 2, 4} (one 32-element block of 4 per
// lane). DPP moves read every lane, so all 64 lanes must be active; both
// row shifts for distance 4 run unconditionally and a select picks one.
__device__ __forceinline__ float max8(float v, int lane) {
  v = fmaxf(v, dpp_f<0xB1>(v));  // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4E>(v));  // quad_perm [2,3,0,1]
  const float up = dpp_f<0x104>(v), down = dpp_f<0x114>(v);  // row_shl:4, row_shr:4
  return fmaxf(v, (lane & 4) ? down : up);
}

// One thread per 4 consecutive elements of a row (one float4 load: a wave
// reads 1 KiB contiguous); the 8 lanes of a 32-element block find its amax
// with DPP. Each term stores one dword of 4 E4M3 codes per lane (a wave
// writes 256 contiguous bytes) and lane 0 of the block its E8M0 exponent.
// Rows >= M (padding up to mpad) and columns >= cols get zero codes.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void k_split(const float* __restrict__ x, int x_stride,
                                                    int M, int cols, int mpad, int kpad,
                                                    uint8_t* __restrict__ a,
                                                    uint8_t* __restrict__ as,
                                                    const SplitJob* __restrict__ jobs) {
  if (jobs) {  // grouped: member blockIdx.y
    const SplitJob j = jobs[blockIdx.y];
    x = j.x;
    a = j.buf;
    as = j.buf + (size_t)kTerms * mpad * kpad;
  }
  const int per_row = kpad / 4;
  const int64_t item = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (item >= (int64_t)mpad * per_row) return;  // whole 8-lane blocks exit together
  const int lane = threadIdx.x & 63;
  const int m = (int)(item / per_row), k = (int)(item % per_row) * 4;
  float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (m < M) {
    const float* row = x + (size_t)m * x_stride;
    if (VEC && k + 4 <= cols) {
      const float4 v = *reinterpret_cast<const float4*>(row + k);
      r[0] = v.x, r[1] = v.y, r[2] = v.z, r[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) r[i] = k + i < cols ? row[k + i] : 0.0f;
    }
  }
  const int nblk = kpad / 32;
#pragma unroll
  for (int t = 0; t < kTerms; ++t) {
    float am = fmaxf(fmaxf(fabsf(r[0]), fabsf(r[1])), fmaxf(fabsf(r[2]), fabsf(r[3])));
    am = max8(am, lane);
    const int e = e8m0_exponent(am, 448.0f);
    const float inv = pow2f(-e), sc = pow2f(e);
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(r[0] * inv, r[1] * inv, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(r[2] * inv, r[3] * inv, w, true);
    *reinterpret_cast<int*>(a + ((size_t)t * mpad + m) * kpad + k) = w;
    if ((lane & 7) == 0) as[((size_t)t * mpad + m) * nblk + k / 32] = (uint8_t)(e + 127);
    if (t + 1 < kTerms) {
      const v2f q0 = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
      const v2f q1 = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
      r[0] -= q0.x * sc, r[1] -= q0.y * sc, r[2] -= q1.x * sc, r[3] -= q1.y * sc;
    }
  }
}

template <int DT>
constexpr int wfmt() {
  return DT == kE4M3 ? 0 : DT == kE5M2 ? 1 : 4;
}

// BM x 64 tile; waves WAVES_M x WAVES_N; each wave SM x SN MFMA tiles of 16x16.
template <int DT, bool BLK, int MATS, int BM>
__global__ __launch_bounds__(kThreads) void k_mxg(MxgArgs p) {
  constexpr bool FP4 = DT == kFP4;
  constexpr int WAVES_M = BM >= 32 ? 2 : 1;
  constexpr int WAVES_N = 4 / WAVES_M;
  constexpr int WM = BM / WAVES_M, WN = kBN / WAVES_N;
  constexpr int SM = WM / 16, SN = WN / 16;
  constexpr int AROW = 128 + 16;                 // padded LDS row of A (bytes)
  constexpr int BROW = (FP4 ? 64 : 128) + 16;    // padded LDS row of W
  constexpr int WBYTES = FP4 ? 64 : 128;         // code bytes per row per K step

  __shared__ __attribute__((aligned(16))) uint8_t sa[kTerms * BM * AROW];
  __shared__ __attribute__((aligned(16))) uint8_t sb[MATS * kBN * BROW];
  __shared__ uint8_t ssa[kTerms * BM * 4];
  __shared__ uint8_t ssb[MATS * kBN * 4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int i16 = lane & 15, g = lane >> 4;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * kBN;
  const int S = p.kpad / 128;
  const int nblk_a = p.kpad / 32;

  v4f acc[MATS][SM][SN];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int a = 0; a < SM; ++a)
#pragma unroll
      for (int b = 0; b < SN; ++b) acc[m][a][b] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < S; ++s) {
    // stage A terms: kTerms*BM rows x 8 chunks of 16 B
    for (int c = tid; c < kTerms * BM * 8; c += kThreads) {
      const int t = c / (BM * 8), row = (c / 8) % BM, j = c % 8;
      const uint4 v = *reinterpret_cast<const uint4*>(
          p.a + ((size_t)t * p.mpad + m0 + row) * p.kpad + (size_t)s * 128 + j * 16);
      *reinterpret_cast<uint4*>(sa + (t * BM + row) * AROW + j * 16) = v;
    }
    for (int c = tid; c < kTerms * BM; c += kThreads) {
      const int t = c / BM, row = c % BM;
      *reinterpret_cast<uint32_t*>(ssa + c * 4) = *reinterpret_cast<const uint32_t*>(
          p.as + ((size_t)t * p.mpad + m0 + row) * nblk_a + s * 4);
    }
    // stage weight codes: MATS*64 rows x (WBYTES/16) chunks
    constexpr int WCH = WBYTES / 16;
    for (int c = tid; c < MATS * kBN * WCH; c += kThreads) {
      const int m = c / (kBN * WCH), row = (c / WCH) % kBN, j = c % WCH;
      const uint4 v = *reinterpret_cast<const uint4*>(
          p.codes[m] + (size_t)(n0 + row) * p.pitch + (size_t)s * WBYTES + j * 16);
      *reinterpret_cast<uint4*>(sb + (m * kBN + row) * BROW + j * 16) = v;
    }
    if constexpr (BLK) {
      for (int c = tid; c < MATS * kBN; c += kThreads) {
        const int m = c / kBN, row = c % kBN;
        *reinterpret_cast<uint32_t*>(ssb + c * 4) = *reinterpret_cast<const uint32_t*>(
            p.blk[m] + (size_t)(n0 + row) * p.nblk + s * 4);
      }
    }
    __syncthreads();
    v8i bf[MATS][SN];
    int bsc[MATS][SN];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int b = 0; b < SN; ++b) {
        const int row = wn * WN + b * 16 + i16;
        const uint8_t* src = sb + (m * kBN + row) * BROW + 16 * g;
        const int4 lo = *reinterpret_cast<const int4*>(src);
        int4 hi = make_int4(0, 0, 0, 0);
        if constexpr (!FP4) hi = *reinterpret_cast<const int4*>(src + 64);
        bf[m][b] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        bsc[m][b] = BLK ? (int)ssb[(m * kBN + row) * 4 + g] : 127;
      }
#pragma unroll
    for (int t = 0; t < kTerms; ++t) {
#pragma unroll
      for (int a = 0; a < SM; ++a) {
        const int row = wm * WM + a * 16 + i16;
        const uint8_t* src = sa + (t * BM + row) * AROW + 16 * g;
        const int4 lo = *reinterpret_cast<const int4*>(src);
        const int4 hi = *reinterpret_cast<const int4*>(src + 64);
        const v8i af = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        const int asc = ssa[(t * BM + row) * 4 + g];
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
          for (int b = 0; b < SN; ++b)
            acc[m][a][b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                af, bf[m][b], acc[m][a][b], 0, wfmt<DT>(), 0, asc, 0, bsc[m][b]);
      }
    }
    __syncthreads();
  }

  // epilogue: lane holds rows 4g + r of each 16x16 tile, column i16
#pragma unroll
  for (int a = 0; a < SM; ++a)
#pragma unroll
    for (int b = 0; b < SN; ++b) {
      const int n = n0 + wn * WN + b * 16 + i16;
      if (n >= p.N) continue;
      float sc[MATS];
#pragma unroll
      for (int m = 0; m < MATS; ++m) sc[m] = p.scale[m][n];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int mrow = m0 + wm * WM + a * 16 + 4 * g + r;
        if (mrow >= p.M) continue;
        const size_t oi = (size_t)mrow * p.out_stride + n;
        if constexpr (MATS == 2) {
          const float gv = acc[0][a][b][r] * sc[0], uv = acc[1][a][b][r] * sc[1];
          const float gs = (float)act_f64(kSilu, (double)gv);
          p.pre[oi] = (float)((double)gs * (double)uv);
        } else {
          float y = acc[0][a][b][r] * sc[0];
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
            if (p.post) p.post[oi] = y;
          }
        }
      }
    }
}

// Large-M tile: 128 activation rows x 128 weight rows (64 per matrix when
// MATS = 2) per workgroup, 4 waves of 64 x 64 (x 3 terms: 48 MFMAs per wave
// per 128-wide K step).
//
// Operands move global -> LDS with the gfx950 direct-to-LDS loads
// (global_load_lds_dwordx4: lane i of a wave writes 16 bytes at
// base + 16 i), double-buffered: while the MFMAs of step s run, step s+1 is
// copied into the other buffer, with no register staging. LDS rows are
// unpadded (128 bytes: A terms and FP8 codes; 64 bytes: FP4 codes) and the
// 16-byte chunks of row r are stored at chunk j ^ ((r >> 1) & 7) (FP4:
// j ^ ((r >> 2) & 3)), which makes the 16-lane groups of a fragment read hit
// 16 distinct 16-byte bank groups.
//
// Tiles are ordered so that each XCD (workgroups are dealt round-robin to the
// 8 XCDs) works on a contiguous band of activation rows against all weight
// tiles: its L2 holds that band of A and the whole weight matrix.
constexpr int kBM2 = 128;

typedef __attribute__((address_space(3))) void* LdsPtr;
typedef const __attribute__((address_space(1))) void* GlobalPtr;

// The copy size of the builtin must be a literal.
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds((GlobalPtr)src, (LdsPtr)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds((GlobalPtr)src, (LdsPtr)lds_base, 4, 0, 0);
}

// A grouped member's argument block, read field by field through the constant
// address space: scalar loads into SGPRs (copying the struct as a whole
// would go through a private-memory temporary).
typedef const __attribute__((address_space(4))) MxgArgs* ConstArgs;
__device__ __forceinline__ MxgArgs load_args(ConstArgs t) {
  MxgArgs p;
  p.a = t->a;
  p.as = t->as;
  p.M = t->M;
  p.mpad = t->mpad;
  p.codes[0] = t->codes[0];
  p.codes[1] = t->codes[1];
  p.scale[0] = t->scale[0];
  p.scale[1] = t->scale[1];
  p.blk[0] = t->blk[0];
  p.blk[1] = t->blk[1];
  p.mats = t->mats;
  p.pitch = t->pitch;
  p.nblk = t->nblk;
  p.kpad = t->kpad;
  p.N = t->N;
  p.pre = t->pre;
  p.post = t->post;
  p.out_stride = t->out_stride;
  p.act = t->act;
  p.need_epi = t->need_epi;
  p.bias = t->bias;
  p.bias_len = t->bias_len;
  return p;
}

template <int DT, bool BLK, int MATS, bool GROUP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_mxg2(
    MxgArgs p0, const MxgArgs* __restrict__ tab, int tiles_m, int tiles_n) {
  constexpr bool FP4 = DT == kFP4;
  constexpr int BM = kBM2;
  constexpr int BNM = MATS == 2 ? 64 : 128;     // weight rows per matrix per tile
  constexpr int WB = FP4 ? 64 : 128;            // code bytes per weight row per K step
  constexpr int SM = 4, SN = BNM / 32;          // 16x16 blocks per wave (waves 2 x 2)
  constexpr int A_BYTES = kTerms * BM * 128;    // one buffer of A terms
  constexpr int B_BYTES = MATS * BNM * WB;
  constexpr int A_SEG = A_BYTES / 1024;         // 1 KiB wave copies per step
  constexpr int B_SEG = B_BYTES / 1024;
  constexpr int B_RPS = 1024 / WB;              // weight rows per 1 KiB copy

  __shared__ __attribute__((aligned(1024))) uint8_t sa[2][A_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t sb[2][B_BYTES];
  __shared__ __attribute__((aligned(256))) uint32_t ssa[2][kTerms * BM];
  __shared__ __attribute__((aligned(256))) uint32_t ssb[2][MATS * BNM];

  const int T = tiles_m * tiles_n;
  // grouped launches: member blockIdx.x / T, whose arguments come from tab
  MxgArgs p;
  if constexpr (GROUP) p = load_args((ConstArgs)tab + blockIdx.x / T);
  else p = p0;
  const int b = GROUP ? blockIdx.x % T : blockIdx.x;
  const int lt = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
  const int m0 = (lt / tiles_n) * BM, n0 = (lt % tiles_n) * BNM;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int i16 = lane & 15, g = lane >> 4;
  const int S = p.kpad / 128;
  const int nblk_a = p.kpad / 32;

  // Per-lane source of each copy this wave issues (K step 0; step s adds
  // s * 128 bytes of A / s * WB bytes of codes / s * 4 bytes of exponents).
  uint32_t aoff[A_SEG / 4], boff[B_SEG / 4 > 0 ? B_SEG / 4 : 1];
#pragma unroll
  for (int k = 0; k < A_SEG / 4; ++k) {
    const int q = wave + 4 * k;                          // segment: 8 rows of one term
    const int t = q / (BM / 8), row = (q % (BM / 8)) * 8 + lane / 8;
    const int j = (lane % 8) ^ ((row >> 1) & 7);
    aoff[k] = (uint32_t)(((size_t)t * p.mpad + m0 + row) * p.kpad + j * 16);
  }
  const uint8_t* bbase[B_SEG / 4 > 0 ? B_SEG / 4 : 1];
#pragma unroll
  for (int k = 0; k < B_SEG / 4; ++k) {
    const int q = wave + 4 * k;
    const int row = q * B_RPS + lane / (WB / 16);       // tile row (both matrices)
    const int jj = lane % (WB / 16);
    const int j = FP4 ? (jj ^ ((row >> 2) & 3)) : (jj ^ ((row >> 1) & 7));
    bbase[k] = row / BNM == 0 ? p.codes[0] : p.codes[MATS - 1];  // no dynamic index into p
    boff[k] = (uint32_t)((size_t)(n0 + row % BNM) * p.pitch + j * 16);
  }
  // exponent copies (one dword per lane): A terms 6 x 64, weights 2 x 64
  const int ea0 = wave * 64 + lane, ea1 = (wave + 4) * 64 + lane;
  const uint32_t asoff0 = (uint32_t)(((size_t)(ea0 / BM) * p.mpad + m0 + ea0 % BM) * nblk_a);
  const bool has_a1 = wave + 4 < kTerms * BM / 64;
  const uint32_t asoff1 =
      has_a1 ? (uint32_t)(((size_t)(ea1 / BM) * p.mpad + m0 + ea1 % BM) * nblk_a) : 0u;
  const bool has_b = BLK && wave < MATS * BNM / 64;
  const uint8_t* bsrc = has_b ? ((wave * 64 + lane) / BNM == 0 ? p.blk[0] : p.blk[MATS - 1]) +
                                    (size_t)(n0 + (wave * 64 + lane) % BNM) * p.nblk
                              : nullptr;
  if constexpr (!BLK) {
    for (int i = tid; i < 2 * MATS * BNM; i += kThreads) (&ssb[0][0])[i] = 0x7F7F7F7Fu;
  }

  auto issue = [&](int s, int buf) {
#pragma unroll
    for (int k = 0; k < A_SEG / 4; ++k)
      lds_dma16(p.a + (aoff[k] + (uint32_t)s * 128u), &sa[buf][(wave + 4 * k) * 1024]);
#pragma unroll
    for (int k = 0; k < B_SEG / 4; ++k)
      lds_dma16(bbase[k] + (boff[k] + (uint32_t)s * WB), &sb[buf][(wave + 4 * k) * 1024]);
    lds_dma4(p.as + (asoff0 + s * 4), &ssa[buf][wave * 64]);
    if (has_a1) lds_dma4(p.as + (asoff1 + s * 4), &ssa[buf][(wave + 4) * 64]);
    if (has_b) lds_dma4(bsrc + s * 4, &ssb[buf][wave * 64]);
  };

  v4f acc[MATS][SM][SN];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int a = 0; a < SM; ++a)
#pragma unroll
      for (int c = 0; c < SN; ++c) acc[m][a][c] = v4f{0.f, 0.f, 0.f, 0.f};

  issue(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = 0; s < S; ++s) {
    const int cur = s & 1;
    v8i bf[MATS][SN];
    int bsc[MATS][SN];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int c = 0; c < SN; ++c) {
        const int row = m * BNM + wn * (BNM / 2) + c * 16 + i16;
        int4 lo, hi = make_int4(0, 0, 0, 0);
        if constexpr (FP4) {
          lo = *reinterpret_cast<const int4*>(&sb[cur][row * 64 + ((g ^ ((row >> 2) & 3)) * 16)]);
        } else {
          const int sw = (row >> 1) & 7;
          lo = *reinterpret_cast<const int4*>(&sb[cur][row * 128 + ((g ^ sw) * 16)]);
          hi = *reinterpret_cast<const int4*>(&sb[cur][row * 128 + (((4 + g) ^ sw) * 16)]);
        }
        bf[m][c] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        bsc[m][c] = (int)((ssb[cur][row] >> (8 * g)) & 0xFFu);
      }
    v8i af[kTerms][SM];
    int asc[kTerms][SM];
#pragma unroll
    for (int t = 0; t < kTerms; ++t)
#pragma unroll
      for (int a = 0; a < SM; ++a) {
        const int row = t * BM + wm * 64 + a * 16 + i16;
        const int sw = (row >> 1) & 7;
        const int4 lo = *reinterpret_cast<const int4*>(&sa[cur][row * 128 + ((g ^ sw) * 16)]);
        const int4 hi = *reinterpret_cast<const int4*>(&sa[cur][row * 128 + (((4 + g) ^ sw) * 16)]);
        af[t][a] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        asc[t][a] = (int)((ssa[cur][row] >> (8 * g)) & 0xFFu);
      }
    // the next step streams into the other buffer while the MFMAs run (that
    // buffer's last readers finished before the previous barrier)
    if (s + 1 < S) issue(s + 1, cur ^ 1);
    // keep the copies ahead of the MFMAs and the wait + barrier behind them
    // (the MFMAs touch only registers, so the scheduler could otherwise move
    // them past the barrier and expose the copy latency every step)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < kTerms; ++t)
#pragma unroll
      for (int a = 0; a < SM; ++a)
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
          for (int c = 0; c < SN; ++c)
            acc[m][a][c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                bf[m][c], af[t][a], acc[m][a][c], wfmt<DT>(), 0, 0, bsc[m][c], 0, asc[t][a]);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // Epilogue. The weights are the MFMA's first operand, so a lane holds
  // output row m = i16 of each block and the 4 consecutive columns 4g..4g+3:
  // one 16-byte store per lane and block when the output allows it. The
  // scale arrays are padded to the row padding, so the float4 scale loads
  // stay in bounds.
  const bool vec_out = (p.out_stride & 3) == 0 && ((reinterpret_cast<uintptr_t>(p.pre) & 15) == 0) &&
                       ((reinterpret_cast<uintptr_t>(p.post) & 15) == 0);
#pragma unroll
  for (int a = 0; a < SM; ++a)
#pragma unroll
    for (int c = 0; c < SN; ++c) {
      const int mrow = m0 + wm * 64 + a * 16 + i16;
      const int nb = n0 + wn * (BNM / 2) + c * 16 + 4 * g;
      if (mrow >= p.M || nb >= p.N) continue;
      float4 sc[MATS];
#pragma unroll
      for (int m = 0; m < MATS; ++m) sc[m] = *reinterpret_cast<const float4*>(p.scale[m] + nb);
      float pre[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float s0 = r == 0 ? sc[0].x : r == 1 ? sc[0].y : r == 2 ? sc[0].z : sc[0].w;
        if constexpr (MATS == 2) {
          const float s1 = r == 0 ? sc[1].x : r == 1 ? sc[1].y : r == 2 ? sc[1].z : sc[1].w;
          const float gv = acc[0][a][c][r] * s0, uv = acc[1][a][c][r] * s1;
          const float gs = (float)act_f64(kSilu, (double)gv);
          pre[r] = (float)((double)gs * (double)uv);
        } else {
          pre[r] = acc[0][a][c][r] * s0;
        }
      }
      // Dense with bias or activation: pre holds y here; the second pass
      // below rewrites it (pre = y + bias, post = act) without accumulators
      // live, so the f64 activation code is not unrolled per element.
      const bool plain = MATS == 2 || !p.need_epi;
      const size_t oi = (size_t)mrow * p.out_stride + nb;
      if (vec_out && nb + 3 < p.N) {
        const float4 v = make_float4(pre[0], pre[1], pre[2], pre[3]);
        *reinterpret_cast<float4*>(p.pre + oi) = v;
        if (plain && MATS == 1 && p.post) *reinterpret_cast<float4*>(p.post + oi) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (nb + r >= p.N) break;
          p.pre[oi + r] = pre[r];
          if (plain && MATS == 1 && p.post) p.post[oi + r] = pre[r];
        }
      }
    }
  if constexpr (MATS == 1) {
    if (p.need_epi) {
#pragma unroll 1
      for (int ac = 0; ac < SM * SN; ++ac) {
        const int a = ac / SN, c = ac % SN;
        const int mrow = m0 + wm * 64 + a * 16 + i16;
        const int nb = n0 + wn * (BNM / 2) + c * 16 + 4 * g;
        if (mrow >= p.M) continue;
#pragma unroll 1
        for (int r = 0; r < 4 && nb + r < p.N; ++r) {
          const int n = nb + r;
          const size_t oi = (size_t)mrow * p.out_stride + n;
          float y = p.pre[oi];
          double v = (double)y;
          if (p.bias && n < p.bias_len) {
            v += p.bias[n];
            y = (float)v;
          }
          p.pre[oi] = y;
          p.post[oi] = (float)act_f64(p.act, v);
        }
      }
    }
  }
}

// Small-M GEMM (M <= 32 activation rows: the weight-streaming regime). A
// workgroup owns RB blocks of 16 weight rows (per matrix) and all K; its 8
// waves take the 128-wide K chunks round-robin. Each wave loads the weight
// fragments of a chunk straight from HBM into registers (non-temporal, no
// LDS) and the activation-term fragments from the split buffer (small,
// L2-resident; RB weight blocks share each of them), and runs kTerms MFMAs
// per weight fragment and 16-row activation block; the next chunk's loads
// are issued before the current chunk's MFMAs. The 8 partial tiles meet in
// LDS for the epilogue.
constexpr int kSmallWaves = 8;

template <int DT, bool BLK, int MATS, int MB, int RB>
__global__ __launch_bounds__(64 * kSmallWaves) void k_mxs(MxgArgs p) {
  constexpr bool FP4 = DT == kFP4;
  constexpr int WB = FP4 ? 64 : 128;  // code bytes per weight row per chunk
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * RB;
  const int S = p.kpad / 128;
  const int nblk_a = p.kpad / 32;

  const uint8_t* wrow[MATS][RB];
  const uint8_t* erow[MATS][RB];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = n0 + rb * 16 + i16;
      wrow[m][rb] = p.codes[m] + (size_t)row * p.pitch + 16 * g;
      erow[m][rb] = BLK ? p.blk[m] + (size_t)row * p.nblk + g : nullptr;
    }
  const uint8_t* xrow[kTerms][MB];
  const uint8_t* srow[kTerms][MB];
#pragma unroll
  for (int t = 0; t < kTerms; ++t)
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const size_t r = (size_t)t * p.mpad + b * 16 + i16;
      xrow[t][b] = p.a + r * p.kpad + 16 * g;
      srow[t][b] = p.as + r * nblk_a + g;
    }

  struct Frag {
    v8i w[MATS][RB];
    int ws[MATS][RB];
    v8i x[kTerms][MB];
    int xs[kTerms][MB];
  };
  auto load = [&](int c, Frag& f) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const uint8_t* src = wrow[m][rb] + (size_t)c * WB;
        const u4 lo = __builtin_nontemporal_load(reinterpret_cast<const u4*>(src));
        u4 hi = u4{0u, 0u, 0u, 0u};
        if constexpr (!FP4) hi = __builtin_nontemporal_load(reinterpret_cast<const u4*>(src + 64));
        f.w[m][rb] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                         (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        f.ws[m][rb] = BLK ? (int)erow[m][rb][c * 4] : 127;
      }
#pragma unroll
    for (int t = 0; t < kTerms; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        const uint8_t* src = xrow[t][b] + (size_t)c * 128;
        const int4 lo = *reinterpret_cast<const int4*>(src);
        const int4 hi = *reinterpret_cast<const int4*>(src + 64);
        f.x[t][b] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        f.xs[t][b] = srow[t][b][c * 4];
      }
  };

  v4f acc[MATS][RB][MB];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int b = 0; b < MB; ++b) acc[m][rb][b] = v4f{0.f, 0.f, 0.f, 0.f};

  // ring of NB fragment sets: NB - 1 chunks in flight while one is computed
  // (the body is unrolled NB times so every ring index is a constant); two
  // sets where three would not fit the register budget
  constexpr int NB = RB * MATS + kTerms * MB <= 7 ? 3 : 2;
  Frag f[NB];
#pragma unroll
  for (int i = 0; i < NB - 1; ++i) {
    const int cc = wave + i * kSmallWaves;
    if (cc < S) load(cc, f[i]);
  }
  for (int base = wave; base < S; base += NB * kSmallWaves) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int cc = base + i * kSmallWaves;
      if (cc < S) {
        const int pf = cc + (NB - 1) * kSmallWaves;
        if (pf < S) load(pf, f[(i + NB - 1) % NB]);
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int t = 0; t < kTerms; ++t)
#pragma unroll
              for (int b = 0; b < MB; ++b)
                acc[m][rb][b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    f[i].w[m][rb], f[i].x[t][b], acc[m][rb][b], wfmt<DT>(), 0, 0, f[i].ws[m][rb],
                    0, f[i].xs[t][b]);
      }
    }
  }

  // acc[m][rb][b]: lane holds weight rows n0 + rb*16 + 4g + r (r = 0..3) and
  // activation row b*16 + i16
  __shared__ float part[kSmallWaves][MATS][RB * MB][64][4];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[wave][m][rb * MB + b][lane][r] = acc[m][rb][b][r];
  __syncthreads();
  // RB*MB tiles x 256 outputs; thread -> (tile, lane, r) positions
  for (int o = threadIdx.x; o < RB * MB * 256; o += 64 * kSmallWaves) {
    const int tile = o / 256, l = (o / 4) % 64, r = o % 4;
    const int rb = tile / MB, b = tile % MB;
    const int mrow = b * 16 + (l & 15), n = n0 + rb * 16 + 4 * (l >> 4) + r;
    if (mrow >= p.M || n >= p.N) continue;
    float tot[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
      float sum = 0.0f;
#pragma unroll
      for (int w = 0; w < kSmallWaves; ++w) sum += part[w][m][tile][l][r];
      tot[m] = sum * p.scale[m][n];
    }
    const size_t oi = (size_t)mrow * p.out_stride + n;
    if constexpr (MATS == 2) {
      const float gs = (float)act_f64(kSilu, (double)tot[0]);
      p.pre[oi] = (float)((double)gs * (double)tot[1]);
    } else {
      float y = tot[0];
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
        if (p.post) p.post[oi] = y;
      }
    }
  }
}

template <int DT, bool BLK, int MATS, int MB>
void launch_small(const MxgArgs& p, hipStream_t st) {
  // the largest weight-row group that still gives >= 256 workgroups, capped
  // where the register budget of two waves per SIMD would spill
  constexpr int kMaxRB = MATS * MB == 1 ? 4 : MATS * MB == 2 ? 2 : 1;
  const int n16 = (p.N + 15) / 16;
  if (kMaxRB >= 4 && n16 >= 4 * 256)
    k_mxs<DT, BLK, MATS, MB, (kMaxRB >= 4 ? 4 : 1)><<<(n16 + 3) / 4, 64 * kSmallWaves, 0, st>>>(p);
  else if (kMaxRB >= 2 && n16 >= 2 * 256)
    k_mxs<DT, BLK, MATS, MB, (kMaxRB >= 2 ? 2 : 1)><<<(n16 + 1) / 2, 64 * kSmallWaves, 0, st>>>(p);
  else
    k_mxs<DT, BLK, MATS, MB, 1><<<n16, 64 * kSmallWaves, 0, st>>>(p);
}

template <int DT, bool BLK, int MATS>
Status launch_t(const MxgArgs& p, int bm, hipStream_t st) {
  if (bm == kBM2) {
    constexpr int bn = MATS == 2 ? 64 : 128;
    if ((size_t)kTerms * p.mpad * p.kpad >= (1ull << 31) ||
        (size_t)round_up(p.N, 128) * p.pitch >= (1ull << 31))
      return Status::err(kUnsupported, "mxg: operands above 2 GiB");
    const int tiles_m = p.mpad / kBM2, tiles_n = (p.N + bn - 1) / bn;
    k_mxg2<DT, BLK, MATS, false><<<(unsigned)(tiles_m * tiles_n), kThreads, 0, st>>>(
        p, nullptr, tiles_m, tiles_n);
  } else {
    if (p.mpad <= 16) launch_small<DT, BLK, MATS, 1>(p, st);
    else launch_small<DT, BLK, MATS, 2>(p, st);
  }
  return hip_status(hipGetLastError(), "mxg launch");
}

template <int MATS>
Status launch_m(const MxgArgs& p, int dtype, bool blk, int bm, hipStream_t st) {
  switch (dtype) {
  case kE4M3: return blk ? launch_t<kE4M3, true, MATS>(p, bm, st) : launch_t<kE4M3, false, MATS>(p, bm, st);
  case kE5M2: return blk ? launch_t<kE5M2, true, MATS>(p, bm, st) : launch_t<kE5M2, false, MATS>(p, bm, st);
  case kFP4: return blk ? launch_t<kFP4, true, MATS>(p, bm, st) : launch_t<kFP4, false, MATS>(p, bm, st);
  }
  return Status::err(kUnsupported, "mxg: dtype");
}

}  // namespace

int mxg_block_m(int M) { return M <= 32 ? 16 : kBM2; }

size_t split_bytes(int M, int kpad) {
  const size_t mpad = (size_t)round_up(M, mxg_block_m(M));
  return (size_t)kTerms * mpad * kpad + (size_t)kTerms * mpad * (kpad / 32);
}

Status launch_split(const float* x, int x_stride, int M, int cols, int kpad, uint8_t* buf,
                    hipStream_t st) {
  const int mpad = (int)round_up(M, mxg_block_m(M));
  uint8_t* a = buf;
  uint8_t* as = buf + (size_t)kTerms * mpad * kpad;
  const int64_t items = (int64_t)mpad * (kpad / 4);
  const unsigned grid = (unsigned)((items + kThreads - 1) / kThreads);
  const bool vec = (x_stride % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15u) == 0);
  if (vec) k_split<true><<<grid, kThreads, 0, st>>>(x, x_stride, M, cols, mpad, kpad, a, as, nullptr);
  else k_split<false><<<grid, kThreads, 0, st>>>(x, x_stride, M, cols, mpad, kpad, a, as, nullptr);
  return hip_status(hipGetLastError(), "split launch");
}

Status launch_split_group(const SplitJob* jobs, int n, bool vec, int x_stride, int M, int cols,
                          int kpad, hipStream_t st) {
  if (n <= 0 || !jobs) return Status::err(kInvalid, "split group: no members");
  const int mpad = (int)round_up(M, mxg_block_m(M));
  const int64_t items = (int64_t)mpad * (kpad / 4);
  const dim3 grid((unsigned)((items + kThreads - 1) / kThreads), (unsigned)n);
  if (vec) k_split<true><<<grid, kThreads, 0, st>>>(nullptr, x_stride, M, cols, mpad, kpad, nullptr, nullptr, jobs);
  else k_split<false><<<grid, kThreads, 0, st>>>(nullptr, x_stride, M, cols, mpad, kpad, nullptr, nullptr, jobs);
  return hip_status(hipGetLastError(), "split group launch");
}

template <int DT, bool BLK, int MATS>
Status launch_group_t(const MxgArgs* tab, const MxgArgs& p, int n, hipStream_t st) {
  constexpr int bn = MATS == 2 ? 64 : 128;
  const int tiles_m = p.mpad / kBM2, tiles_n = (p.N + bn - 1) / bn;
  k_mxg2<DT, BLK, MATS, true><<<(unsigned)(n * tiles_m * tiles_n), kThreads, 0, st>>>(
      p, tab, tiles_m, tiles_n);
  return hip_status(hipGetLastError(), "mxg group launch");
}

Status launch_mxg_group(const MxgArgs* tab, const MxgArgs& p, int n, int dtype, bool blk,
                        hipStream_t st) {
  if (n <= 0 || !tab) return Status::err(kInvalid, "mxg group: no members");
  if (mxg_block_m(p.M) != kBM2 || p.mpad % kBM2 != 0 || p.kpad % 256 != 0)
    return Status::err(kInvalid, "mxg group: needs the large-tile layout");
  if ((size_t)kTerms * p.mpad * p.kpad >= (1ull << 31) ||
      (size_t)round_up(p.N, 128) * p.pitch >= (1ull << 31))
    return Status::err(kUnsupported, "mxg: operands above 2 GiB");
  const bool two = p.mats == 2;
  switch (dtype) {
  case kE4M3:
    if (two) return blk ? launch_group_t<kE4M3, true, 2>(tab, p, n, st) : launch_group_t<kE4M3, false, 2>(tab, p, n, st);
    return blk ? launch_group_t<kE4M3, true, 1>(tab, p, n, st) : launch_group_t<kE4M3, false, 1>(tab, p, n, st);
  case kE5M2:
    if (two) return blk ? launch_group_t<kE5M2, true, 2>(tab, p, n, st) : launch_group_t<kE5M2, false, 2>(tab, p, n, st);
    return blk ? launch_group_t<kE5M2, true, 1>(tab, p, n, st) : launch_group_t<kE5M2, false, 1>(tab, p, n, st);
  case kFP4:
    if (two) return blk ? launch_group_t<kFP4, true, 2>(tab, p, n, st) : launch_group_t<kFP4, false, 2>(tab, p, n, st);
    return blk ? launch_group_t<kFP4, true, 1>(tab, p, n, st) : launch_group_t<kFP4, false, 1>(tab, p, n, st);
  }
  return Status::err(kUnsupported, "mxg group: dtype");
}

Status launch_mxg(const MxgArgs& p, int dtype, bool blk, hipStream_t st) {
  const int bm = mxg_block_m(p.M);
  if (p.mpad % bm != 0 || p.kpad % 256 != 0) return Status::err(kInvalid, "mxg: layout");
  return p.mats == 2 ? launch_m<2>(p, dtype, blk, bm, st) : launch_m<1>(p, dtype, blk, bm, st);
}

}  // namespace wv
