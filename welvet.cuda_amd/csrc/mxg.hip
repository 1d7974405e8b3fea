// Batched quantized GEMM on the CDNA4 scaled matrix cores (batch > 4 rows).
//
//   C[m][n] = rowscale[n] * sum_k x[m][k] * dec(W[n][k]) * blockscale[n][k/32]
//
// x (fp32) is first split into kTerms E4M3 terms with per-32 E8M0 scales
// (k_split: each term quantizes the residual of the previous ones, so
// x ~ sum_t a_t 2^e_t with a relative residual of ~2^-12 for three terms).
// The terms act as extra K: every term is multiplied by the same weight
// fragment and accumulated into the same fp32 accumulator by
// v_mfma_scale_f32_16x16x128_f8f6f4, which takes the stored FP8/FP4 weight
// codes and their E8M0 block scales directly.
//
// Operand layouts of the instruction (lane l, group g = l / 16): FP8 bytes
// 0-15 -> k = 16g + j, bytes 16-31 -> k = 64 + 16g + j; FP4 nibble j ->
// k = 32g + j; scale of lane l: row l % 16, block g; D: col l % 16, rows
// 4g + r. The weights are the first operand, so a lane's accumulator holds 4
// consecutive output columns of one activation row.
//
// The split buffer is stored in that operand order. For each 16-row block rb
// and 128-wide K chunk kc the kTerms fragments are contiguous (2 KiB each:
// half h holds bytes 16h..16h+15 of every lane's operand, lane l at 16 l), so
// a wave fetches an operand with two fully coalesced 1 KiB loads and needs no
// LDS for it; the kTerms E8M0 exponents a lane passes to the instruction sit
// in one dword (byte t), also at 4 l.
#include <type_traits>

#include "codec.h"
#include "act.h"
#include "common.h"
#include "kernels.h"
#include "runtime.h"
#include "split.h"

namespace wv {
namespace {

// Calls f(std::integral_constant<int, i>) for i = I .. N - 1: straight-line
// code with compile-time indices.
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

constexpr int kThreads = 256;

template <int DT>
constexpr int wfmt() {
  return DT == kE4M3 ? 0 : DT == kE5M2 ? 1 : 4;
}

// One scaled MFMA with the weights as first operand and activation term T
// as second: `xs` holds the exponents of all terms (byte t = term t) and the
// instruction's op_sel picks byte T, so no per-term extraction is needed.
// X6: the activation terms are FP6 E2M3 (format 2) instead of E4M3 (0).
template <int DT, int T, bool X6 = false>
__device__ __forceinline__ v4f mfma_term(v8i w, v8i x, v4f c, int wsc, uint32_t xs) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, x, c, wfmt<DT>(), X6 ? 2 : 0, 0, wsc, T,
                                                          (int)xs);
}

// s_waitcnt immediate (gfx9 encoding) waiting for at most `vm` outstanding
// vector-memory operations and `lgkm` LDS/scalar operations.
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8);
}

// The activation split, written in operand order. One wave per (16-row block
// rb, 128-wide K chunk kc): the 16 x 128 fp32 slice is staged in LDS with
// row-contiguous loads; then lane l (row i16 = l % 16, group g = l / 16)
// takes the 32 values of its operand, k = 64h + 16g + j (h = 0, 1; j < 16),
// and split_terms writes them. Rows >= M and columns >= cols give zero codes.
// VEC: x 16-byte aligned, cols and x_stride multiples of 4. stream: the
// split is larger than the L2s hold, so its stores are non-temporal. F6:
// FP6 terms (split_terms6; lane l takes k = 32 g + p of its row instead).
template <bool VEC, int NT, bool F6 = false>
__global__ __launch_bounds__(kThreads) void k_split(const float* __restrict__ x, int x_stride,
                                                    int M, int cols, int mpad, int kpad,
                                                    uint8_t* __restrict__ a,
                                                    uint8_t* __restrict__ as,
                                                    const SplitJob* __restrict__ jobs, int stream) {
  if (jobs) {  // grouped: member blockIdx.y
    const SplitJob j = jobs[blockIdx.y];
    x = j.x;
    a = j.buf;
    as = j.buf + (size_t)kTerms * mpad * kpad;
  }
  constexpr int kWaves = kThreads / 64;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KC = kpad / 128;
  const int w = blockIdx.x * kWaves + wave;
  if (w >= (mpad / 16) * KC) return;  // whole waves; no workgroup barrier below
  const int rb = w / KC, kc = w % KC;

  __shared__ __attribute__((aligned(16))) float stage[kWaves][16][132];
  float(*sl)[132] = stage[wave];  // rows padded by 16 bytes: no bank conflicts below
  // Unconditional loads clamped to the last row and column (16-byte loads
  // when VEC: x aligned, cols and x_stride multiples of 4), then zeroed
  // outside [0, M) x [0, cols).
  const GlobalF xg = (GlobalF)x;
  const int c4 = 4 * (lane & 31), k = kc * 128 + c4;
  float4 xv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = rb * 16 + 2 * i + (lane >> 5);
    const GlobalF row = xg + (size_t)(m < M ? m : M - 1) * x_stride;
    if constexpr (VEC) {
      const f32x4 t = *reinterpret_cast<const __attribute__((address_space(1))) f32x4*>(row + (k < cols ? k : 0));
      xv[i] = make_float4(t.x, t.y, t.z, t.w);
    } else {
      xv[i].x = row[k < cols ? k : cols - 1];
      xv[i].y = row[k + 1 < cols ? k + 1 : cols - 1];
      xv[i].z = row[k + 2 < cols ? k + 2 : cols - 1];
      xv[i].w = row[k + 3 < cols ? k + 3 : cols - 1];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 2 * i + (lane >> 5);
    const bool ok = rb * 16 + r < M;
    float4 t;
    t.x = ok && k < cols ? xv[i].x : 0.0f;
    t.y = ok && k + 1 < cols ? xv[i].y : 0.0f;
    t.z = ok && k + 2 < cols ? xv[i].z : 0.0f;
    t.w = ok && k + 3 < cols ? xv[i].w : 0.0f;
    *reinterpret_cast<float4*>(&sl[r][c4]) = t;
  }
  // The LDS operations of one wave execute in order, so the reads below see
  // this wave's writes.
  const int i16 = lane & 15, g = lane >> 4;
  const GlobalU8 scales = (GlobalU8)(as + (size_t)(rb * KC + kc) * kChunkScaleBytes);
  if constexpr (F6) {
    float v[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = *reinterpret_cast<const float4*>(&sl[i16][32 * g + 4 * q]);
      v[4 * q] = t.x, v[4 * q + 1] = t.y, v[4 * q + 2] = t.z, v[4 * q + 3] = t.w;
    }
    const GlobalU8 chunk = (GlobalU8)(a + (size_t)(rb * KC + kc) * NT * kFrag6Bytes);
    if (stream)
      split_terms6<1, NT, true>(v, chunk, scales, lane);
    else
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
    const GlobalU8 chunk = (GlobalU8)(a + (size_t)(rb * KC + kc) * NT * kFragBytes);
    if (stream)
      split_terms<1, NT, true>(v, chunk, scales, lane);
    else
      split_terms<1, NT, false>(v, chunk, scales, lane);
  }
}

// Large-M tile (M > 32): 128 activation rows x 128 staged weight rows (64 per
// matrix when MATS = 2) per 256-thread workgroup; wave w owns activation rows
// 32w..32w+31 against all 128 weight rows (2 x 8 blocks of 16 x 16, x 3
// terms: 48 MFMAs per 128-wide K step).
//
// Activation operands go straight from the split buffer into registers, each
// wave its own rows, double-buffered: the loads of step s+1 run under the
// MFMAs of step s. The weight tile, which all four waves use, goes through
// LDS, double-buffered the same way: each wave loads its quarter of step
// s+1 (one 16-byte load per lane and KiB) before the MFMAs of step s and
// stores it to the other buffer after them. LDS rows are unpadded (128 bytes
// FP8, 64 bytes FP4) and the 16-byte chunks of row r sit at chunk
// j ^ ((r >> 1) & 7) (FP4: j ^ ((r >> 2) & 3)), so the 16-lane groups of a
// fragment read hit distinct bank groups. A step ends with an LDS wait and a
// plain s_barrier (no fence: the activation loads stay in flight).
//
// Workgroups are dealt round-robin to the 8 XCDs, each with its own L2;
// tiles are renumbered so that every XCD owns one contiguous run of tiles: a
// band of activation rows against all weight tiles, or in grouped launches
// whole members.
constexpr int kBM = 128;
// waves per large-tile workgroup: 8 = two per SIMD, so one wave's MFMAs run
// while the other waits on memory
constexpr int kMxgWaves = 8;

// Wide tiles (256 staged weight rows per step) move half the activation
// bytes per MFMA; taken when they still give every CU a workgroup and N is a
// multiple of their width (the weight rows and scales are padded to 128).
bool mxg_wide(int members, int tiles_m, int N, int mats) {
  const int bn = 256 / mats;
  return N % bn == 0 && (long)members * tiles_m * (N / bn) >= 256;
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
  p.part = t->part;
  p.blkf[0] = t->blkf[0];
  p.blkf[1] = t->blkf[1];
  p.next = t->next;
  p.rope_tab = t->rope_tab;
  p.rope_hd = t->rope_hd;
  p.terms = t->terms;
  p.keep_out = t->keep_out;
  return p;
}

template <int DT, bool BLK, int MATS, bool GROUP, int W, int BR, bool KS = false, int NT = kTerms>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(W / 4, W / 4))) void k_mxg(
    MxgArgs p0, const MxgArgs* __restrict__ tab, int tiles_m, int tiles_n) {
  constexpr bool FP4 = DT == kFP4;
  // BR staged weight rows per step (128, or 256 for wide tiles: twice the
  // MFMAs per byte of activation terms moved), BNM per matrix
  constexpr int BNM = BR / MATS;
  constexpr int WB = FP4 ? 64 : 128;         // code bytes per weight row per K step
  constexpr int SM = kBM / 16 / W;           // 16-row activation blocks per wave
  constexpr int SN = BR / 16;                // 16-row weight blocks
  constexpr int NC = SN / MATS;              // output column blocks
  constexpr int B_BYTES = BR * WB;
  constexpr int B_CPW = B_BYTES / 1024 / W;  // 1 KiB weight copies per wave per step
  constexpr int B_RPS = 1024 / WB;           // weight rows per 1 KiB copy

  __shared__ __attribute__((aligned(1024))) uint8_t sb[2][B_BYTES];
  __shared__ __attribute__((aligned(256))) uint32_t ssb[2][BR];

  const int T = tiles_m * tiles_n;
  const int nb = gridDim.x;
  const int f = (nb % 8 == 0) ? (blockIdx.x % 8) * (nb / 8) + blockIdx.x / 8 : blockIdx.x;
  // grouped launches: member f / T, whose arguments come from tab
  MxgArgs p;
  if constexpr (GROUP) p = load_args((ConstArgs)tab + f / T);
  else p = p0;
  const int lt = GROUP ? f % T : f;
  const int m0 = (lt / tiles_n) * kBM, n0 = (lt % tiles_n) * BNM;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i16 = lane & 15, g = lane >> 4;
  const int KC = p.kpad / 128, S = KC;
  // K steps [kb, ke): all of K, or with KS (split along K, blockIdx.y of
  // gridDim.y) a range of whole step pairs
  int kb = 0, ke = S;
  if constexpr (KS) {
    const int P = S / 2, ks = blockIdx.y, nks = gridDim.y;
    kb = 2 * (int)((long)P * ks / nks);
    ke = 2 * (int)((long)P * (ks + 1) / nks);
  }

  // activation fragments of this wave (step s adds s * CB / s * 256): the
  // NT terms of a (16-row block, K chunk) are contiguous, CB bytes
  // FP6 terms (act_fp6): NT fragments of kFrag6Bytes, dwords 0-3 of lane l at
  // 16 l, dwords 4-5 at 1024 + 8 l
  constexpr bool X6 = act_fp6<NT>();
  constexpr int CB = NT * (X6 ? kFrag6Bytes : kFragBytes);
  const uint8_t* abase[SM];
  const uint32_t* sbase[SM];
#pragma unroll
  for (int a = 0; a < SM; ++a) {
    const size_t rb = (size_t)(m0 / 16 + wave * SM + a);
    abase[a] = p.a + rb * KC * CB + lane * 16;
    sbase[a] = reinterpret_cast<const uint32_t*>(p.as + rb * KC * kChunkScaleBytes) + lane;
  }
  // weight copies: per-lane source of each 1 KiB copy this wave issues at
  // step 0 (step s adds s * WB bytes)
  const uint8_t* bbase[B_CPW];
  uint32_t boff[B_CPW];
#pragma unroll
  for (int k = 0; k < B_CPW; ++k) {
    const int q = wave + W * k;
    const int row = q * B_RPS + lane / (WB / 16);  // staged row (both matrices)
    const int jj = lane % (WB / 16);
    const int j = FP4 ? (jj ^ ((row >> 2) & 3)) : (jj ^ ((row >> 1) & 7));
    bbase[k] = row / BNM == 0 ? p.codes[0] : p.codes[MATS - 1];  // no dynamic index into p
    boff[k] = (uint32_t)((size_t)(n0 + row % BNM) * p.pitch + j * 16);
  }
  // weight block exponents: one dword (4 blocks) per staged row and step;
  // waves w and w + BR / 64 copy the same 64 rows (identical bytes)
  constexpr int EC = BR / 64;
  static_assert(W % EC == 0, "exponent copies");
  const int erow = (wave % EC) * 64 + lane;
  const uint8_t* bsrc =
      BLK ? (erow / BNM == 0 ? p.blk[0] : p.blk[MATS - 1]) + (size_t)(n0 + erow % BNM) * p.nblk
          : nullptr;

  struct AFrag {
    v8i x[NT][SM];
    uint32_t xs[SM];
  };
  auto load_a = [&](int s, AFrag& fr) {
#pragma unroll
    for (int a = 0; a < SM; ++a) {
      const uint8_t* src = abase[a] + (size_t)s * CB;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (X6) {
          const int4 lo = *reinterpret_cast<const int4*>(src + t * kFrag6Bytes);
          const int2 hi = *reinterpret_cast<const int2*>(src + t * kFrag6Bytes + 1024 - lane * 8);
          fr.x[t][a] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, 0, 0};
        } else {
          const int4 lo = *reinterpret_cast<const int4*>(src + t * kFragBytes);
          const int4 hi = *reinterpret_cast<const int4*>(src + t * kFragBytes + 1024);
          fr.x[t][a] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        }
      }
      fr.xs[a] = sbase[a][s * (kChunkScaleBytes / 4)];
    }
  };
  // The weight tile moves global -> registers -> LDS: loads issued before a
  // step's MFMAs, LDS stores after them. (With direct-to-LDS copies in
  // flight beside the activation loads the compiler treats the load counter
  // as out of order and waits for every load before the MFMAs.)
  // (named registers, not an array: an array here ends up in scratch or LDS
  // before the loops that index it are unrolled)
  static_assert(B_CPW == 1 || B_CPW == 2 || B_CPW == 4, "weight copies per wave");
#define WV_BSRC(k, s) reinterpret_cast<const uint4*>(bbase[k] + (boff[k] + (uint32_t)(s) * WB))
#define WV_BDST(k, buf) reinterpret_cast<uint4*>(&sb[buf][(wave + W * (k)) * 1024 + lane * 16])
#define WV_LOAD_B(s)                                           \
  do {                                                         \
    q0 = *WV_BSRC(0, s);                                       \
    if constexpr (B_CPW >= 2) q1 = *WV_BSRC(1, s);             \
    if constexpr (B_CPW == 4) {                                \
      q2 = *WV_BSRC(2, s);                                     \
      q3 = *WV_BSRC(3, s);                                     \
    }                                                          \
    if constexpr (BLK) be = *reinterpret_cast<const uint32_t*>(bsrc + (s) * 4); \
  } while (0)
#define WV_STORE_B(buf)                                        \
  do {                                                         \
    *WV_BDST(0, buf) = q0;                                     \
    if constexpr (B_CPW >= 2) *WV_BDST(1, buf) = q1;           \
    if constexpr (B_CPW == 4) {                                \
      *WV_BDST(2, buf) = q2;                                   \
      *WV_BDST(3, buf) = q3;                                   \
    }                                                          \
    if constexpr (BLK) ssb[buf][(wave % EC) * 64 + lane] = be; \
  } while (0)

  v4f acc[SM][SN];
#pragma unroll
  for (int a = 0; a < SM; ++a)
#pragma unroll
    for (int c = 0; c < SN; ++c) acc[a][c] = v4f{0.f, 0.f, 0.f, 0.f};

  // Two fragment sets and two weight buffers; step s computes from set and
  // buffer s & 1 while step s + 1 streams into the others. kpad is a multiple
  // of 256, so S is even and the loop body is unrolled by two with constant
  // indices and no condition around any load: the compiler then knows
  // exactly which loads are outstanding and waits only for the ones a step
  // uses (a conditional load makes it wait for all of them).
  // 128-row tiles of a single launch with exactly 8 K steps (K = 1024: the
  // MHA projections) take the two-step-ahead form below
  constexpr bool PF2 = BR == 128 && !GROUP && !KS;
  if (!PF2 || ke - kb != 8) {
  AFrag fr[2];
  {
    uint4 q0, q1, q2, q3;
    uint32_t be = 0;
    WV_LOAD_B(kb);
    WV_STORE_B(0);
  }
  load_a(kb, fr[0]);
  if constexpr (!BLK) {
    for (int i = tid; i < 2 * BR; i += 64 * W) (&ssb[0][0])[i] = 0x7F7F7F7Fu;
  }
  __builtin_amdgcn_sched_barrier(0);
  // nothing may be in flight on entry to the loop either (same reason as at
  // its back-edge below)
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  asm volatile("s_barrier" ::: "memory");

  for (int s0 = kb; s0 < ke; s0 += 2) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int s = s0 + i, cur = i;
      {
        // Weight fragments in groups of HB = 4 blocks: the first group
        // before the next step's loads are issued, the others after the
        // previous group's MFMAs, so the MFMAs start after 4 fragment reads
        // rather than after the whole tile (every wave reads the tile right
        // after the barrier). Measured: groups of 8 and of 2 are slower.
        constexpr int HB = SN < 4 ? SN : 4;
        v8i bf[HB];
        int bsc[HB];
        auto read_b = [&](int c0) {
#pragma unroll
          for (int c = 0; c < HB; ++c) {
            const int row = (c0 + c) * 16 + i16;
            int4 lo, hi = make_int4(0, 0, 0, 0);
            if constexpr (FP4) {
              lo = *reinterpret_cast<const int4*>(&sb[cur][row * 64 + ((g ^ ((row >> 2) & 3)) * 16)]);
            } else {
              const int sw = (row >> 1) & 7;
              lo = *reinterpret_cast<const int4*>(&sb[cur][row * 128 + ((g ^ sw) * 16)]);
              hi = *reinterpret_cast<const int4*>(&sb[cur][row * 128 + (((4 + g) ^ sw) * 16)]);
            }
            bf[c] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            bsc[c] = (int)((ssb[cur][row] >> (8 * g)) & 0xFFu);
          }
        };
        auto mfma_half = [&](int c0) {
          static_assert(NT >= 1 && NT <= 3, "one to three activation terms");
#pragma unroll
          for (int a = 0; a < SM; ++a)
#pragma unroll
            for (int c = 0; c < HB; ++c)
              acc[a][c0 + c] = mfma_term<DT, 0, X6>(bf[c], fr[cur].x[0][a], acc[a][c0 + c], bsc[c], fr[cur].xs[a]);
          if constexpr (NT >= 2) {
#pragma unroll
            for (int a = 0; a < SM; ++a)
#pragma unroll
              for (int c = 0; c < HB; ++c)
                acc[a][c0 + c] = mfma_term<DT, 1, X6>(bf[c], fr[cur].x[1][a], acc[a][c0 + c], bsc[c], fr[cur].xs[a]);
          }
          if constexpr (NT == 3) {
#pragma unroll
            for (int a = 0; a < SM; ++a)
#pragma unroll
              for (int c = 0; c < HB; ++c)
                acc[a][c0 + c] = mfma_term<DT, 2, X6>(bf[c], fr[cur].x[NT - 1][a], acc[a][c0 + c], bsc[c], fr[cur].xs[a]);
          }
        };
        read_b(0);
        __builtin_amdgcn_sched_barrier(0);
        // next step into the other buffer and set (their last readers
        // finished before the previous barrier); the last step fetches
        // itself again into them, which nothing reads
        const int nx = s + 1 < ke ? s + 1 : ke - 1;
        uint4 q0, q1, q2, q3;
        uint32_t be = 0;
        WV_LOAD_B(nx);
        load_a(nx, fr[cur ^ 1]);
        // keep the copies ahead of the MFMAs and the wait + barrier behind
        // them (the MFMAs touch only registers)
        __builtin_amdgcn_sched_barrier(0);
        mfma_half(0);
#pragma unroll
        for (int h = 1; h < SN / HB; ++h) {
          __builtin_amdgcn_sched_barrier(0);
          read_b(h * HB);
          __builtin_amdgcn_sched_barrier(0);
          mfma_half(h * HB);
        }
        __builtin_amdgcn_sched_barrier(0);
        // weight tile of step s+1 into the other buffer (the compiler waits
        // for its loads only: the activation loads issued after them stay in
        // flight), visible to all waves after the barrier. After the second
        // step of the pair every load is waited for: one still in flight at
        // the loop back-edge makes the compiler wait for all loads before the
        // first MFMA of the next pass. Unconditional (also after the last
        // step): a branch here would end the basic block, and the compiler
        // sinks the MFMAs past it, behind the next step's loads.
        WV_STORE_B(cur ^ 1);
        if (i == 0) __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
        else __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  } else if constexpr (PF2) {
    // The 8 steps as straight-line code, with loads two steps ahead: step j
    // computes from LDS buffer j & 1 and activation set j % 3, loads step
    // j + 2's weights into register set j & 1 (stored to LDS at the end of
    // step j + 1) and its activations into set (j + 2) % 3. Without a loop
    // back-edge the compiler waits for exactly the loads each step uses.
    // Measured at 4096 x 1024 x 1024: 22.97 -> 22.37 us (three terms), 20.1
    // -> 18.9 us (two terms). Wide tiles do not take it: their weight and
    // activation sets do not fit the register budget (spills).
#define WV_LOAD_BX(s, Q0, Q1, Q2, Q3, BE)                                       \
  do {                                                                          \
    Q0 = *WV_BSRC(0, s);                                                        \
    if constexpr (B_CPW >= 2) Q1 = *WV_BSRC(1, s);                              \
    if constexpr (B_CPW == 4) {                                                 \
      Q2 = *WV_BSRC(2, s);                                                      \
      Q3 = *WV_BSRC(3, s);                                                      \
    }                                                                           \
    if constexpr (BLK) BE = *reinterpret_cast<const uint32_t*>(bsrc + (s) * 4); \
  } while (0)
#define WV_STORE_BX(buf, Q0, Q1, Q2, Q3, BE)                   \
  do {                                                         \
    *WV_BDST(0, buf) = Q0;                                     \
    if constexpr (B_CPW >= 2) *WV_BDST(1, buf) = Q1;           \
    if constexpr (B_CPW == 4) {                                \
      *WV_BDST(2, buf) = Q2;                                   \
      *WV_BDST(3, buf) = Q3;                                   \
    }                                                          \
    if constexpr (BLK) ssb[buf][(wave % EC) * 64 + lane] = BE; \
  } while (0)
    AFrag f3[3];
    uint4 qa0, qa1, qa2, qa3, qb0, qb1, qb2, qb3;
    uint32_t bea = 0, beb = 0;
    WV_LOAD_BX(kb, qa0, qa1, qa2, qa3, bea);
    WV_STORE_BX(0, qa0, qa1, qa2, qa3, bea);
    WV_LOAD_BX(kb + 1, qb0, qb1, qb2, qb3, beb);
    load_a(kb, f3[0]);
    load_a(kb + 1, f3[1]);
    if constexpr (!BLK) {
      for (int i = tid; i < 2 * BR; i += 64 * W) (&ssb[0][0])[i] = 0x7F7F7F7Fu;
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, 8>([&](auto J) {
      constexpr int j = decltype(J)::value;
      constexpr int cur = j & 1;
      const int s = kb + j;
      const AFrag& fa = f3[j % 3];
      constexpr int HB = SN < 4 ? SN : 4;
      v8i bf[HB];
      int bsc[HB];
      auto read_b = [&](int c0) {
#pragma unroll
        for (int c = 0; c < HB; ++c) {
          const int row = (c0 + c) * 16 + i16;
          int4 lo, hi = make_int4(0, 0, 0, 0);
          if constexpr (FP4) {
            lo = *reinterpret_cast<const int4*>(&sb[cur][row * 64 + ((g ^ ((row >> 2) & 3)) * 16)]);
          } else {
            const int sw = (row >> 1) & 7;
            lo = *reinterpret_cast<const int4*>(&sb[cur][row * 128 + ((g ^ sw) * 16)]);
            hi = *reinterpret_cast<const int4*>(&sb[cur][row * 128 + (((4 + g) ^ sw) * 16)]);
          }
          bf[c] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
          bsc[c] = (int)((ssb[cur][row] >> (8 * g)) & 0xFFu);
        }
      };
      auto mfma_half = [&](int c0) {
#pragma unroll
        for (int a = 0; a < SM; ++a)
#pragma unroll
          for (int c = 0; c < HB; ++c)
            acc[a][c0 + c] = mfma_term<DT, 0, X6>(bf[c], fa.x[0][a], acc[a][c0 + c], bsc[c], fa.xs[a]);
        if constexpr (NT >= 2) {
#pragma unroll
          for (int a = 0; a < SM; ++a)
#pragma unroll
            for (int c = 0; c < HB; ++c)
              acc[a][c0 + c] = mfma_term<DT, 1, X6>(bf[c], fa.x[1][a], acc[a][c0 + c], bsc[c], fa.xs[a]);
        }
        if constexpr (NT == 3) {
#pragma unroll
          for (int a = 0; a < SM; ++a)
#pragma unroll
            for (int c = 0; c < HB; ++c)
              acc[a][c0 + c] = mfma_term<DT, 2, X6>(bf[c], fa.x[NT - 1][a], acc[a][c0 + c], bsc[c], fa.xs[a]);
        }
      };
      read_b(0);
      __builtin_amdgcn_sched_barrier(0);
      // register set j & 1 held step j's weights, stored to LDS at the end of
      // step j - 1; activation set (j + 2) % 3 was last read by step j - 1.
      // Past the last step the loads repeat it (nothing reads them).
      const int nx = s + 2 < ke ? s + 2 : ke - 1;
      if constexpr ((j & 1) == 0) WV_LOAD_BX(nx, qa0, qa1, qa2, qa3, bea);
      else WV_LOAD_BX(nx, qb0, qb1, qb2, qb3, beb);
      load_a(nx, f3[(j + 2) % 3]);
      __builtin_amdgcn_sched_barrier(0);
      mfma_half(0);
#pragma unroll
      for (int h = 1; h < SN / HB; ++h) {
        __builtin_amdgcn_sched_barrier(0);
        read_b(h * HB);
        __builtin_amdgcn_sched_barrier(0);
        mfma_half(h * HB);
      }
      __builtin_amdgcn_sched_barrier(0);
      // step j + 1's weights (loaded during step j - 1) into the other buffer
      if constexpr (((j + 1) & 1) == 0) WV_STORE_BX(cur ^ 1, qa0, qa1, qa2, qa3, bea);
      else WV_STORE_BX(cur ^ 1, qb0, qb1, qb2, qb3, beb);
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
      asm volatile("s_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    });
#undef WV_LOAD_BX
#undef WV_STORE_BX
  }

#undef WV_BSRC
#undef WV_BDST
#undef WV_LOAD_B
#undef WV_STORE_B

  // Epilogue. A lane's accumulators hold activation row i16 of each 16-row
  // block and 4 consecutive output columns: stored as they are, every store
  // would write 64-byte pieces of 16 rows. Each wave instead stages its
  // result in LDS, CH columns at a time (its own region: no barrier), and
  // writes whole rows, RPI rows of CH floats per store instruction, with the
  // bias and activation applied in that pass. The scale arrays are padded to
  // the row padding, so the float4 scale loads stay in bounds.
  constexpr int COLS = NC * 16;              // output columns of the tile
  constexpr int CH = COLS < 128 ? COLS : 128;  // columns staged at a time
  constexpr int LPR = CH / 4;                // lanes per output row, a float4 each
  constexpr int RPI = 64 / LPR;              // rows per store instruction
  __shared__ __attribute__((aligned(16))) float stage[W][SM * 16][CH + 4];
  const bool vec_out = (p.out_stride & 3) == 0 && ((reinterpret_cast<uintptr_t>(p.pre) & 15) == 0) &&
                       ((reinterpret_cast<uintptr_t>(p.post) & 15) == 0);
  const int cl = 4 * (lane % LPR);
  const int rbase = m0 + wave * SM * 16;
#pragma unroll
  for (int hc = 0; hc < COLS / CH; ++hc) {
#pragma unroll
    for (int a = 0; a < SM; ++a)
#pragma unroll
      for (int cc = 0; cc < CH / 16; ++cc) {
        const int c = hc * (CH / 16) + cc;
        const int nb = n0 + c * 16 + 4 * g;
        float4 sc[MATS];
#pragma unroll
        for (int m = 0; m < MATS; ++m)
          sc[m] = KS ? make_float4(1.f, 1.f, 1.f, 1.f) : *reinterpret_cast<const float4*>(p.scale[m] + nb);
        float y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float s0 = r == 0 ? sc[0].x : r == 1 ? sc[0].y : r == 2 ? sc[0].z : sc[0].w;
          if constexpr (MATS == 2) {
            const float s1 = r == 0 ? sc[1].x : r == 1 ? sc[1].y : r == 2 ? sc[1].z : sc[1].w;
            const float gv = acc[a][c][r] * s0, uv = acc[a][c + NC][r] * s1;
            const float gs = (float)act_f64(kSilu, (double)gv);
            y[r] = (float)((double)gs * (double)uv);
          } else {
            y[r] = acc[a][c][r] * s0;
          }
        }
        *reinterpret_cast<float4*>(&stage[wave][a * 16 + i16][cc * 16 + 4 * g]) =
            make_float4(y[0], y[1], y[2], y[3]);
      }
    const int n = n0 + hc * CH + cl;
    if constexpr (KS) {
      // raw sums of this K range into split blockIdx.y's plane of the
      // partial buffer (rows of round_up(N, 256) floats; k_mxs_reduce adds
      // the planes in split order and applies the scale and epilogue). The
      // tile's columns stay below round_up(N, 256), so every float4 is in
      // the plane.
      const size_t npad = ((size_t)p.N + 255) / 256 * 256;
      float* dst = p.part + (size_t)blockIdx.y * p.mpad * npad;
#pragma unroll
      for (int rr = 0; rr < SM * 16 / RPI; ++rr) {
        const int r = rr * RPI + lane / LPR;
        if (rbase + r >= p.M) continue;
        *reinterpret_cast<float4*>(dst + (size_t)(rbase + r) * npad + n) =
            *reinterpret_cast<const float4*>(&stage[wave][r][cl]);
      }
    } else if (MATS == 2 || !p.need_epi) {
      // post = pre here; a caller that passes one buffer for both gets it
      // written once. No pre: an inner layer of a chain whose output is not
      // kept (only the next layer's split below is written).
      float* post = MATS == 1 && p.post != p.pre ? p.post : nullptr;
#pragma unroll
      for (int rr = 0; rr < (p.pre ? SM * 16 / RPI : 0); ++rr) {
        const int r = rr * RPI + lane / LPR;
        float4 y = *reinterpret_cast<const float4*>(&stage[wave][r][cl]);
        if constexpr (MATS == 1 && CH == 128) {
          if (p.rope_tab) {
            // the 4 columns sit in one half of one head; the partner columns
            // are in the same staged chunk (128 % rope_hd == 0)
            const int half = p.rope_hd >> 1;
            const int d = (hc * CH + cl) % p.rope_hd;  // n0 is a multiple of 128
            const bool lo = d < half;
            const float4 yp = *reinterpret_cast<const float4*>(&stage[wave][r][lo ? cl + half : cl - half]);
            const int tok = rbase + r < p.M ? rbase + r : p.M - 1;
            const double* tb = p.rope_tab + 2 * ((size_t)tok * half + (lo ? d : d - half));
            const float ya[4] = {y.x, y.y, y.z, y.w}, yb[4] = {yp.x, yp.y, yp.z, yp.w};
            float yo[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const double c = tb[2 * e], sn = tb[2 * e + 1];
              const double a0 = lo ? ya[e] : yb[e], a1 = lo ? yb[e] : ya[e];
              yo[e] = lo ? (float)(a0 * c - a1 * sn) : (float)(a0 * sn + a1 * c);
            }
            y = make_float4(yo[0], yo[1], yo[2], yo[3]);
          }
        }
        if (rbase + r >= p.M || n >= p.N) continue;
        const size_t oi = (size_t)(rbase + r) * p.out_stride + n;
        if (vec_out && n + 3 < p.N && !p.keep_out) {
          // streaming stores: no workgroup of this launch reads the output
          const f32x4 yv = f32x4{y.x, y.y, y.z, y.w};
          __builtin_nontemporal_store(yv, reinterpret_cast<f32x4*>(p.pre + oi));
          if (post) __builtin_nontemporal_store(yv, reinterpret_cast<f32x4*>(post + oi));
        } else if (vec_out && n + 3 < p.N) {
          *reinterpret_cast<float4*>(p.pre + oi) = y;
          if (post) *reinterpret_cast<float4*>(post + oi) = y;
        } else {
          const float yv[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (n + i >= p.N) break;
            p.pre[oi + i] = yv[i];
            if (post) post[oi + i] = yv[i];
          }
        }
      }
    } else {
      // Dense with bias or activation (reference rule: pre = f32(y + bias),
      // post = act evaluated in f64 on y + bias); rolled, so the f64
      // activation code appears once
#pragma unroll 1
      for (int rr = 0; rr < SM * 16 / RPI; ++rr) {
        const int r = rr * RPI + lane / LPR;
        const float4 y4 = *reinterpret_cast<const float4*>(&stage[wave][r][cl]);
        if (rbase + r >= p.M || n >= p.N) continue;
        const size_t oi = (size_t)(rbase + r) * p.out_stride + n;
        float yv[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll 1
        for (int i = 0; i < 4 && n + i < p.N; ++i) {
          float y = yv[i];
          double v = (double)y;
          if (p.bias && n + i < p.bias_len) {
            v += p.bias[n + i];
            y = (float)v;
          }
          yv[i] = (float)act_f64(p.act, v);
          if (p.pre) {
            p.pre[oi + i] = y;
            p.post[oi + i] = yv[i];
          }
        }
        // post stays in the stage for the split below (same lane, same place)
        *reinterpret_cast<float4*>(&stage[wave][r][cl]) = make_float4(yv[0], yv[1], yv[2], yv[3]);
      }
    }
    if constexpr (MATS == 1 && CH == 128 && !KS) {
      // Chained layer: the next layer's split of post, written from the
      // stage (the same terms k_split would make from post in memory). The
      // next layer has the same rows (mpad) and kpad = N. Rows >= M get zero
      // codes; the stage reads follow this wave's own stage writes in program
      // order.
      if (p.next && n0 + hc * CH < p.N) {
        __builtin_amdgcn_wave_barrier();
        const int kcn = p.N / 128, kc = (n0 + hc * CH) / 128;
        uint8_t* nscale = p.next + (size_t)kTerms * p.mpad * p.N;
#pragma unroll
        for (int a = 0; a < SM; ++a) {
          const int rb = rbase / 16 + a;
          const bool live = rb * 16 + i16 < p.M;
          const GlobalU8 nchunk = (GlobalU8)(p.next + (size_t)(rb * kcn + kc) * CB);
          const GlobalU8 nsc = (GlobalU8)(nscale + (size_t)(rb * kcn + kc) * kChunkScaleBytes);
          if constexpr (X6) {
            float v[32];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              const float4 t = *reinterpret_cast<const float4*>(&stage[wave][a * 16 + i16][32 * g + 4 * q]);
              v[4 * q] = live ? t.x : 0.0f, v[4 * q + 1] = live ? t.y : 0.0f;
              v[4 * q + 2] = live ? t.z : 0.0f, v[4 * q + 3] = live ? t.w : 0.0f;
            }
            split_terms6<1, NT, true>(v, nchunk, nsc, lane);
          } else {
            float v[2][16];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const float4 t = *reinterpret_cast<const float4*>(&stage[wave][a * 16 + i16][64 * h + 16 * g + 4 * q]);
                v[h][4 * q] = live ? t.x : 0.0f, v[h][4 * q + 1] = live ? t.y : 0.0f;
                v[h][4 * q + 2] = live ? t.z : 0.0f, v[h][4 * q + 3] = live ? t.w : 0.0f;
              }
            split_terms<1, NT, true>(v, nchunk, nsc, lane);
          }
        }
        __builtin_amdgcn_wave_barrier();
      }
    }
  }
}

// Small-M GEMM (M <= 32 activation rows: the weight-streaming regime), split
// along K. Workgroup (g, ks) has 8 waves; wave w owns RB blocks of 16 weight
// rows (of each matrix), rows 128 RB g + 16 (RB w + j) + .., over the K
// chunks [k0, k1) of split ks (at most KRT chunks). A CU streams HBM at a
// bounded rate (~30-40 GB/s), so the split fills all CUs with one round of
// workgroups, and RB = 2 halves the activation terms each CU stages. The
// activation terms of that K range (all M rows, in operand order) are made
// from the fp32 input in the prologue and kept in LDS; the weights stream
// from HBM straight into registers D - 1 chunks ahead, in the order they are
// consumed, so 8 (D - 1) chunks per CU are in flight. The KRT steps are
// straight-line code (no loop back-edge, which makes the compiler wait for
// every outstanding load) and every load is unconditional: a step past the
// range repeats the last chunk with its weights zeroed. With one split the
// epilogue is applied here; otherwise each split writes its raw sums to the
// partial buffer and k_mxs_reduce adds them and applies the epilogue.
constexpr int kSmallWaves = 8;

// Weight row blocks per wave: two once there are enough rows.
int mxs_rb(int N) { return N >= 2048 ? 2 : 1; }

// Largest K range per workgroup (chunks) for 1 or 2 activation row blocks:
// its staged terms fill at most ~150 KB of LDS.
constexpr int small_krt_max(int mb) { return mb == 1 ? 24 : 12; }

// Splits so that the grid is one round of at most 256 workgroups (one per
// CU), unless the K range of a workgroup would exceed the LDS.
int mxs_ksplit(int N, int kpad, int mpad) {
  const int S = kpad / 128, MB = mpad / 16;
  const int rows = 16 * kSmallWaves * mxs_rb(N);
  const int groups = (N + rows - 1) / rows;
  int ks = 256 / groups > 1 ? 256 / groups : 1;
  const int krt = small_krt_max(MB);
  if (ks < (S + krt - 1) / krt) ks = (S + krt - 1) / krt;
  return ks < S ? ks : S;
}

template <int DT, bool BLK, int MATS, int MB, int RB, int KRT, int D, bool XV, int NT>
__global__ __launch_bounds__(64 * kSmallWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_mxs(
    MxgArgs p, int ksplit) {
  constexpr int ROWS = 16 * kSmallWaves * RB;  // weight rows per workgroup
  constexpr bool FP4 = DT == kFP4;
  constexpr int WB = FP4 ? 64 : 128;  // code bytes per weight row per chunk
  // three terms: FP6 (E2M3) terms (split_terms6), as on the large tiles;
  // fewer terms: E4M3
  constexpr bool X6 = act_fp6<NT>();
  constexpr int CB = NT * (X6 ? kFrag6Bytes : kFragBytes);  // the NT terms of one split unit
  __shared__ __attribute__((aligned(16))) uint8_t sA[MB * KRT * CB];
  __shared__ __attribute__((aligned(16))) uint32_t sS[MB * KRT * 64];

  // the wave index in a scalar register: branches on it are uniform
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i16 = lane & 15, g = lane >> 4;
  const int S = p.kpad / 128, ks = blockIdx.y;
  const int k0 = (int)((long)S * ks / ksplit), k1 = (int)((long)S * (ks + 1) / ksplit);
  const int KR = k1 - k0;  // 1 .. KRT (the launcher's split guarantees it)
  const int n0 = blockIdx.x * ROWS + wave * 16 * RB;

  // weight rows: the codes are padded to a multiple of 128 rows; the grid
  // may cover up to 128 more (RB = 2), whose loads are clamped to the last
  // padded row (their outputs are never stored)
  // Block exponents come from the lane-order copy: the dword of chunk group
  // c / 4 (256 contiguous bytes per wave load), byte c % 4.
  // With the operand-order copy (codesf) a wave's operand is the 1 KiB at
  // lane * 16 of its (row block, chunk, half) slot: chunk stride WB * 16
  // bytes, half stride 1 KiB. Without it, lane (i16, g) reads 16 bytes of
  // row-major row i16 at chunk offset 16 g: chunk stride WB, half stride 64.
  // The choice is made once here (uniform); the K loop has no branch on it.
  const int rmax = (p.N + 127) / 128 * 128 - 1;
  const int egroups = (S + 3) / 4;
  const bool frag = p.codesf[0] != nullptr && (MATS == 1 || p.codesf[MATS - 1] != nullptr);
  const uint32_t cstride = frag ? WB * 16 : WB, hstride = frag ? 1024 : 64;
  const uint8_t* wrow[MATS][RB];
  const uint8_t* erow[MATS][RB];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int row = n0 + 16 * j + i16 < rmax ? n0 + 16 * j + i16 : rmax;
      const int rb16 = (n0 + 16 * j < rmax ? n0 + 16 * j : rmax) / 16;
      wrow[m][j] = frag ? p.codesf[m] + (size_t)rb16 * S * (WB * 16) + lane * 16
                        : p.codes[m] + (size_t)row * p.pitch + 16 * g;
      erow[m][j] = BLK ? p.blkf[m] + (size_t)rb16 * egroups * 256 + lane * 4 : nullptr;
    }
  struct WFrag {
    u32x4 lo[MATS][RB], hi[MATS][RB];
    uint32_t e[MATS][RB];  // exponent dword (4 chunks)
  };
  auto load_w = [&](int r, WFrag& f) {  // chunk k0 + r, clamped to the range
    const int c = k0 + (r < KR ? r : KR - 1);
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const uint8_t* src = wrow[m][j] + (size_t)c * cstride;
        f.lo[m][j] = *reinterpret_cast<const u32x4*>(src);
        if constexpr (!FP4) f.hi[m][j] = *reinterpret_cast<const u32x4*>(src + hstride);
        f.e[m][j] = BLK ? *reinterpret_cast<const uint32_t*>(erow[m][j] + (size_t)(c >> 2) * 256)
                        : 0x7F7F7F7Fu;
      }
  };

  // The activation terms of the K range, made here from the fp32 input with
  // the code k_split uses and kept in LDS: split unit j = (row block b,
  // chunk r), j = b * KR + r, goes to wave j % 8. Each lane loads the 32
  // values of its operand (row b * 16 + i16, k = 64h + 16g + .. for E4M3
  // terms, k = 32g + .. for FP6 terms), with
  // unconditional loads clamped to the last unit, row and column (16-byte
  // loads when XV: x aligned, cols and stride multiples of 4). The first
  // unit's loads are issued before the first D - 1 chunks of weights, so its
  // split waits for them only and the weights stay in flight under it; a
  // wave's further units (K ranges above 8 chunks) load after it.
  constexpr int U = (MB * KRT + kSmallWaves - 1) / kSmallWaves;  // units per wave
  const int units = MB * KR;
  float4 xin[8];
  auto load_unit = [&](int u) {
    const int j = wave + kSmallWaves * u < units ? wave + kSmallWaves * u : units - 1;
    const int row = (j / KR) * 16 + i16;
    const float* src = p.x + (size_t)(row < p.M ? row : p.M - 1) * p.x_stride;
    const int kb = (k0 + j % KR) * 128 + (X6 ? 32 : 16) * g;
    if constexpr (XV) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int k = X6 ? kb + 4 * q : kb + 64 * (q >> 2) + 4 * (q & 3);
        xin[q] = *reinterpret_cast<const float4*>(src + (k < p.cols ? k : 0));
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int k = X6 ? kb + 4 * q : kb + 64 * (q >> 2) + 4 * (q & 3);
        xin[q].x = src[k < p.cols ? k : p.cols - 1];
        xin[q].y = src[k + 1 < p.cols ? k + 1 : p.cols - 1];
        xin[q].z = src[k + 2 < p.cols ? k + 2 : p.cols - 1];
        xin[q].w = src[k + 3 < p.cols ? k + 3 : p.cols - 1];
      }
    }
  };
  load_unit(0);
  __builtin_amdgcn_sched_barrier(0);
  WFrag f[D];
#pragma unroll
  for (int i = 0; i < D - 1; ++i) load_w(i, f[i]);
  constexpr int PREFILL = (D - 1) * MATS * RB * (1 + (FP4 ? 0 : 1) + (BLK ? 1 : 0));
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = wave + kSmallWaves * u;
    if (j < units) {  // uniform
      const bool rowok = (j / KR) * 16 + i16 < p.M;
      const int kb = (k0 + j % KR) * 128 + (X6 ? 32 : 16) * g;
      float v[2][16];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int k = X6 ? kb + 4 * q : kb + 64 * (q >> 2) + 4 * (q & 3);
        const float4 t = xin[q];
        float* d = &v[q >> 2][4 * (q & 3)];  // FP6: v viewed as 32 values in k order
        d[0] = rowok && k < p.cols ? t.x : 0.0f;
        d[1] = rowok && k + 1 < p.cols ? t.y : 0.0f;
        d[2] = rowok && k + 2 < p.cols ? t.z : 0.0f;
        d[3] = rowok && k + 3 < p.cols ? t.w : 0.0f;
      }
      if constexpr (X6)
        split_terms6<3, NT>(reinterpret_cast<float(&)[32]>(v), (LdsU8)(sA + (size_t)j * CB),
                            (LdsU8)(sS + j * 64), lane);
      else
        split_terms<3, NT>(v, (LdsU8)(sA + (size_t)j * CB), (LdsU8)(sS + j * 64), lane);
    }
    if (u + 1 < U) load_unit(u + 1);
  }
  // the terms written by every wave are visible after the barrier; the
  // weight loads stay in flight
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(PREFILL, 0));
  asm volatile("s_barrier" ::: "memory");

  v4f acc[MATS][RB][MB];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int b = 0; b < MB; ++b) acc[m][j][b] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int r = 0; r < KRT; ++r) {
    if (r + D - 1 < KRT) load_w(r + D - 1, f[(r + D - 1) % D]);  // compile-time condition
    __builtin_amdgcn_sched_barrier(0);
    const bool live = r < KR;  // uniform
    const int rr = live ? r : KR - 1;
    v8i x[NT][MB];
    uint32_t xs[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const uint8_t* src = sA + (size_t)(b * KR + rr) * CB + lane * 16;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (X6) {
          const int4 lo = *reinterpret_cast<const int4*>(src + t * kFrag6Bytes);
          const int2 hi = *reinterpret_cast<const int2*>(src + t * kFrag6Bytes + 1024 - lane * 8);
          x[t][b] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, 0, 0};
        } else {
          const int4 lo = *reinterpret_cast<const int4*>(src + t * kFragBytes);
          const int4 hi = *reinterpret_cast<const int4*>(src + t * kFragBytes + 1024);
          x[t][b] = v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        }
      }
      xs[b] = sS[(b * KR + rr) * 64 + lane];
    }
    // a step past the range repeats the last chunk: zero weights add
    // exactly nothing (its activations are those of a live step)
    const WFrag& fr = f[r % D];
    const int eb = 8 * ((k0 + rr) & 3);  // byte of this chunk in the exponent dwords
    int we[MATS][RB];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < RB; ++j) we[m][j] = (int)((fr.e[m][j] >> eb) & 0xFFu);
    v8i w[MATS][RB];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const u32x4 lo = fr.lo[m][j];
        const u32x4 hi = FP4 ? u32x4{0u, 0u, 0u, 0u} : fr.hi[m][j];
        w[m][j] = live ? v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y,
                             (int)hi.z, (int)hi.w}
                       : v8i{0, 0, 0, 0, 0, 0, 0, 0};
      }
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < RB; ++j)
#pragma unroll
        for (int b = 0; b < MB; ++b)
          acc[m][j][b] = mfma_term<DT, 0, X6>(w[m][j], x[0][b], acc[m][j][b], we[m][j], xs[b]);
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < RB; ++j)
#pragma unroll
        for (int b = 0; b < MB; ++b)
          acc[m][j][b] = mfma_term<DT, 1, X6>(w[m][j], x[1][b], acc[m][j][b], we[m][j], xs[b]);
    if constexpr (NT == 3) {
#pragma unroll
      for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int j = 0; j < RB; ++j)
#pragma unroll
          for (int b = 0; b < MB; ++b)
            acc[m][j][b] = mfma_term<DT, 2, X6>(w[m][j], x[NT - 1][b], acc[m][j][b], we[m][j], xs[b]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // acc[m][j][b]: lane holds activation row 16 b + i16 and weight rows
  // n0 + 16 j + 4g + r (r = 0..3)
  if (ksplit > 1) {
    const size_t npad = ((size_t)p.N + ROWS - 1) / ROWS * ROWS;
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int m = 0; m < MATS; ++m)
          *reinterpret_cast<v4f*>(p.part + (((size_t)ks * MATS + m) * p.mpad + b * 16 + i16) * npad +
                                  n0 + 16 * j + 4 * g) = acc[m][j][b];
    return;
  }
#pragma unroll
  for (int j = 0; j < RB; ++j)
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const int mrow = b * 16 + i16;
    const int nb = n0 + 16 * j + 4 * g;
    if (mrow >= p.M) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = nb + r;
      if (n >= p.N) break;
      const size_t oi = (size_t)mrow * p.out_stride + n;
      if constexpr (MATS == 2) {
        const float gs = (float)act_f64(kSilu, (double)(acc[0][j][b][r] * p.scale[0][n]));
        p.pre[oi] = (float)((double)gs * (double)(acc[1][j][b][r] * p.scale[1][n]));
      } else {
        float y = acc[0][j][b][r] * p.scale[0][n];
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
}

// Small-M GEMM (M <= 32 activation rows) over the whole K per workgroup, for
// products with enough weight rows to fill the GPU without a K split: 16
// weight rows (of each matrix) per workgroup; its W waves cut K into ranges
// and add their sums in LDS, so no partial sums leave the workgroup and no
// reduce launch follows. The activation terms come from the split buffer
// (three FP6 terms, written by k_split first), read by every workgroup from
// L2. A wave streams its weight and activation fragments D - 1 chunks ahead
// in a ring, as straight-line code over at most NS chunks with unconditional
// loads: a step past the wave's range repeats its last chunk with the weights
// zeroed, so it adds exactly nothing. With ROT, workgroup g starts its waves'
// ranges at chunk offset g mod range (the workgroups then read different
// activation lines at a time). The waves' sums are added in wave order, and
// the epilogue is k_mxs's.
//
// Measured on the 16-row SwiGLU of d_model 4096 and d_ff 11008 (timing-only
// harness, 64 rotated weight copies): the gate+up pair k_split + k_mxr
// 19.3 us against 20.9 us for k_mxs + its reduce; the down product 14.7
// against 13.7 us (there every workgroup reads 396 KB of activation terms for
// 88 KB of weights), so only the two-matrix product takes it.
constexpr int kRowWaves = 8;

template <int DT, bool BLK, int MATS, int MB, int NS, int D, int W = kRowWaves, bool ROT = false,
          int RB = 1>
__global__ __launch_bounds__(64 * W) void k_mxr(MxgArgs p) {
  constexpr bool FP4 = DT == kFP4;
  constexpr int NT = kTerms;  // FP6 terms (act_fp6)
  constexpr int WB = FP4 ? 64 : 128;          // code bytes per weight row per chunk
  constexpr int CB = NT * kFrag6Bytes;        // the terms of one (row block, chunk)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i16 = lane & 15, g = lane >> 4;
  const int S = p.kpad / 128;
  const int k0 = S * wave / W, KR = S * (wave + 1) / W - k0;  // 0 .. NS
  const int n0 = 16 * RB * (int)blockIdx.x;  // RB blocks of 16 weight rows
  const int ab0 = MB * (int)blockIdx.y;      // first activation row block of this workgroup
  const int egroups = (S + 3) / 4;
  // weights: the operand-order copy (a wave's operand is the 1 KiB at
  // lane * 16 of its (row block, chunk, half) slot) or row-major rows
  // (lane (i16, g) reads 16 bytes of row n0 + i16 at chunk offset 16 g); the
  // grid covers whole 16-row blocks of the rows, which are padded to 128
  const bool frag = p.codesf[0] != nullptr && (MATS == 1 || p.codesf[MATS - 1] != nullptr);
  const uint32_t cstride = frag ? WB * 16 : WB, hstride = frag ? 1024 : 64;
  const uint8_t* wrow[MATS][RB];
  const uint8_t* erow[MATS][RB];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int rb16 = n0 / 16 + j;
      wrow[m][j] = frag ? p.codesf[m] + (size_t)rb16 * S * (WB * 16) + lane * 16
                        : p.codes[m] + (size_t)(16 * rb16 + i16) * p.pitch + 16 * g;
      erow[m][j] = BLK ? p.blkf[m] + (size_t)rb16 * egroups * 256 + lane * 4 : nullptr;
    }
  // activation terms of row block b, chunk c: term t's 16 bytes of lane l at
  // ((b S + c) NT + t) 1536 + 16 l, its 8 more at + 1024 + 8 l; the
  // exponent dword (byte t: term t) at (b S + c) 256 + 4 l
  const uint8_t* abase[MB];
  const uint8_t* sbase[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    abase[b] = p.a + (size_t)(ab0 + b) * S * CB + lane * 16;
    sbase[b] = p.as + (size_t)(ab0 + b) * S * kChunkScaleBytes + lane * 4;
  }
  struct Frag {
    u32x4 lo[MATS][RB], hi[MATS][RB];
    uint32_t e[MATS][RB];
    int4 xl[NT][MB];
    int2 xh[NT][MB];
    uint32_t xs[MB];
  };
  const int rot = ROT && KR > 0 ? (int)(blockIdx.x % (unsigned)KR) : 0;
  auto chunk = [&](int r) {  // step r's chunk: the range from a per-workgroup offset
    const int rr = r < KR ? r : (KR > 0 ? KR - 1 : 0);
    return k0 + (ROT ? (rr + rot < KR ? rr + rot : rr + rot - KR) : rr);
  };
  auto load = [&](int r, Frag& f) {  // chunk k0 + r, clamped to the range
    const int c = chunk(r);
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const uint8_t* src = wrow[m][j] + (size_t)c * cstride;
        f.lo[m][j] = *reinterpret_cast<const u32x4*>(src);
        if constexpr (!FP4) f.hi[m][j] = *reinterpret_cast<const u32x4*>(src + hstride);
        f.e[m][j] = BLK ? *reinterpret_cast<const uint32_t*>(erow[m][j] + (size_t)(c >> 2) * 256)
                        : 0x7F7F7F7Fu;
      }
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const uint8_t* src = abase[b] + (size_t)c * CB;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f.xl[t][b] = *reinterpret_cast<const int4*>(src + t * kFrag6Bytes);
        f.xh[t][b] = *reinterpret_cast<const int2*>(src + t * kFrag6Bytes + 1024 - lane * 8);
      }
      f.xs[b] = *reinterpret_cast<const uint32_t*>(sbase[b] + (size_t)c * kChunkScaleBytes);
    }
  };

  v4f acc[MATS][RB][MB];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int b = 0; b < MB; ++b) acc[m][j][b] = v4f{0.f, 0.f, 0.f, 0.f};
  Frag f[D];
#pragma unroll
  for (int i = 0; i < D - 1; ++i) load(i, f[i]);
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    if (r + D - 1 < NS) load(r + D - 1, f[(r + D - 1) % D]);  // compile-time condition
    __builtin_amdgcn_sched_barrier(0);
    const Frag& fr = f[r % D];
    const bool live = r < KR;  // uniform
    const int c = chunk(r);
    const int eb = 8 * (c & 3);  // byte of this chunk in the exponent dwords
    v8i w[MATS][RB];
    int we[MATS][RB];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const u32x4 lo = fr.lo[m][j];
        const u32x4 hi = FP4 ? u32x4{0u, 0u, 0u, 0u} : fr.hi[m][j];
        w[m][j] = live ? v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y,
                             (int)hi.z, (int)hi.w}
                       : v8i{0, 0, 0, 0, 0, 0, 0, 0};
        we[m][j] = (int)((fr.e[m][j] >> eb) & 0xFFu);
      }
    static_for<0, NT>([&](auto T) {
      constexpr int t = decltype(T)::value;
#pragma unroll
      for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int j = 0; j < RB; ++j)
#pragma unroll
          for (int b = 0; b < MB; ++b) {
            const int4 xl = fr.xl[t][b];
            const int2 xh = fr.xh[t][b];
            const v8i x = v8i{xl.x, xl.y, xl.z, xl.w, xh.x, xh.y, 0, 0};
            acc[m][j][b] = mfma_term<DT, t, true>(w[m][j], x, acc[m][j][b], we[m][j], fr.xs[b]);
          }
    });
    __builtin_amdgcn_sched_barrier(0);
  }

  // acc[m][j][b]: lane holds activation row 16 b + i16 and weight rows
  // n0 + 16 j + 4g + r (r = 0..3); the waves' sums meet in LDS
  __shared__ float red[W][MATS][RB][MB][4][64];
#pragma unroll
  for (int m = 0; m < MATS; ++m)
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][m][j][b][r][lane] = acc[m][j][b][r];
  // chained products (RB = 2, one matrix): post of the 16 rows x 32 columns
  // of each row block, for the next layer's split
  constexpr bool CAN_NEXT = MATS == 1 && RB == 2;
  __shared__ float nstage[CAN_NEXT ? MB : 1][16][33];
  __syncthreads();
  // output e: row block e / (256 RB), activation row (e / 16 RB) % 16,
  // column n0 + e % 16 RB (16 RB consecutive outputs per 16 RB threads)
  constexpr int NOUT = RB * MB * 256;
  for (int e = tid; e < NOUT; e += 64 * W) {
    const int b = e / (256 * RB), m16 = (e / (16 * RB)) % 16, nc = e % (16 * RB);
    const int j = nc >> 4, n16 = nc & 15;
    const int src = m16 + 16 * (n16 >> 2), r = n16 & 3;
    const int mrow = 16 * (ab0 + b) + m16, n = n0 + nc;
    const bool live = mrow < p.M && n < p.N;
    float tot[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
      float v = red[0][m][j][b][r][src];
#pragma unroll
      for (int w = 1; w < W; ++w) v += red[w][m][j][b][r][src];
      tot[m] = v;
    }
    const size_t oi = (size_t)mrow * p.out_stride + n;
    if constexpr (MATS == 2) {
      if (live) {
        const float gs = (float)act_f64(kSilu, (double)(tot[0] * p.scale[0][n]));
        p.pre[oi] = (float)((double)gs * (double)(tot[1] * p.scale[1][n]));
      }
    } else {
      float y = 0.0f, out = 0.0f;
      if (live) {
        y = tot[0] * p.scale[0][n];
        out = y;
        if (p.need_epi) {
          double v = (double)y;
          if (p.bias && n < p.bias_len) {
            v += p.bias[n];
            y = (float)v;
          }
          out = (float)act_f64(p.act, v);
          if (p.pre) p.pre[oi] = y;
          if (p.post) p.post[oi] = out;
        } else {
          if (p.pre) p.pre[oi] = y;
          if (p.post && p.post != p.pre) p.post[oi] = y;
        }
      }
      if constexpr (CAN_NEXT) nstage[b][m16][nc] = out;  // zero outside [0, M) x [0, N)
    }
  }
  if constexpr (CAN_NEXT) {
    // The next layer's split of post (the terms k_split makes from post in
    // memory; same rows mpad, kpad = N): this workgroup's 32 columns are one
    // block of a 128-wide chunk, held in operand order by lanes i + 16 g of
    // each (row block, chunk) slot, one lane per activation row.
    if (p.next) {
      __syncthreads();
      if (tid < 16 * MB) {
        const int b = tid >> 4, i = tid & 15, rb = ab0 + b;
        const int kcn = p.N / 128, kc = n0 / 128, gb = (n0 % 128) / 32;
        float v[32];
#pragma unroll
        for (int q = 0; q < 32; ++q) v[q] = nstage[b][i][q];
        const GlobalU8 nchunk = (GlobalU8)(p.next + (size_t)(rb * kcn + kc) * CB);
        const GlobalU8 nsc = (GlobalU8)(p.next + (size_t)kTerms * p.mpad * p.N +
                                        (size_t)(rb * kcn + kc) * kChunkScaleBytes);
        split_terms6<1, NT, true>(v, nchunk, nsc, i + 16 * gb);
      }
    }
  }
}

// The SwiGLU gate+up pair at 5..16 activation rows with FP4 weights and at
// most 4 K chunks per wave: k_mxr's product with persistent workgroups. One
// workgroup per CU walks the 16-row blocks blockIdx.x, + gridDim.x, ...; each
// wave loads the activation terms of its K range once into registers (three
// FP6 terms of 16 rows: 72 bytes per lane and chunk) and reuses them for every
// block, where k_mxr's workgroups (one per block) each read them again from
// L2, 2.25 times the bytes of the weights they stream. The next block's
// weights are loaded before the current block's MFMAs. Sums, their order and
// the epilogue are k_mxr's (bit-identical outputs). Measured on the 16-row
// SwiGLU of d_model 4096 and d_ff 11008 (timing-only harness, 64 rotated
// weight copies): 13.6 us against 16.1-16.6 us for k_mxr; without any
// activation loads k_mxr would take 10.2-11.0 us.
template <int DT, bool BLK, int NS, int W = kRowWaves>
__global__ __launch_bounds__(64 * W) void k_mxp(MxgArgs p) {
  constexpr int MATS = 2, NT = kTerms;
  constexpr bool FP4 = DT == kFP4;
  static_assert(FP4, "k_mxp holds the FP4 weights of two blocks in registers");
  constexpr int WB = 64, CB = NT * kFrag6Bytes;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int S = p.kpad / 128;
  const int k0 = S * wave / W, KR = S * (wave + 1) / W - k0;  // 1 .. NS
  const int egroups = (S + 3) / 4;
  const int blocks = (p.N + 15) / 16;
  auto chunk = [&](int r) { return k0 + (r < KR ? r : KR - 1); };
  // this wave's activation terms (row block 0), once
  int4 xl[NS][NT];
  int2 xh[NS][NT];
  uint32_t xs[NS];
#pragma unroll
  for (int r = 0; r < NS; ++r) {
    const int c = chunk(r);
    const uint8_t* src = p.a + (size_t)c * CB + lane * 16;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      xl[r][t] = *reinterpret_cast<const int4*>(src + t * kFrag6Bytes);
      xh[r][t] = *reinterpret_cast<const int2*>(src + t * kFrag6Bytes + 1024 - lane * 8);
    }
    xs[r] = *reinterpret_cast<const uint32_t*>(p.as + (size_t)c * kChunkScaleBytes + lane * 4);
  }
  struct Wt {
    u32x4 lo[MATS][NS];
    uint32_t e[MATS][NS];
  };
  auto load = [&](int blk, Wt& f) {  // the operand-order codes of row block blk
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
      const uint8_t* base = p.codesf[m] + (size_t)blk * S * (WB * 16) + lane * 16;
      const uint8_t* eb = BLK ? p.blkf[m] + (size_t)blk * egroups * 256 + lane * 4 : nullptr;
#pragma unroll
      for (int r = 0; r < NS; ++r) {
        const int c = chunk(r);
        f.lo[m][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + (size_t)c * (WB * 16)));
        f.e[m][r] = BLK ? *reinterpret_cast<const uint32_t*>(eb + (size_t)(c >> 2) * 256) : 0x7F7F7F7Fu;
      }
    }
  };
  auto product = [&](const Wt& f, v4f (&acc)[MATS]) {
#pragma unroll
    for (int r = 0; r < NS; ++r) {
      const bool live = r < KR;  // uniform; a repeated chunk adds nothing
      const int eb = 8 * (chunk(r) & 3);
      v8i w[MATS];
      int we[MATS];
#pragma unroll
      for (int m = 0; m < MATS; ++m) {
        const u32x4 lo = f.lo[m][r];
        w[m] = live ? v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, 0, 0, 0, 0}
                    : v8i{0, 0, 0, 0, 0, 0, 0, 0};
        we[m] = (int)((f.e[m][r] >> eb) & 0xFFu);
      }
      static_for<0, NT>([&](auto T) {
        constexpr int t = decltype(T)::value;
        const v8i x = v8i{xl[r][t].x, xl[r][t].y, xl[r][t].z, xl[r][t].w, xh[r][t].x, xh[r][t].y, 0, 0};
#pragma unroll
        for (int m = 0; m < MATS; ++m) acc[m] = mfma_term<DT, t, true>(w[m], x, acc[m], we[m], xs[r]);
      });
    }
  };
  __shared__ float red[W][MATS][4][64];
  Wt wt[2];
  load((int)blockIdx.x, wt[0]);
  int cur = 0;
  for (int blk = (int)blockIdx.x; blk < blocks; blk += (int)gridDim.x) {
    v4f acc[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m) acc[m] = v4f{0.f, 0.f, 0.f, 0.f};
    const int nxt = blk + (int)gridDim.x;  // uniform
    if (cur == 0) {
      if (nxt < blocks) load(nxt, wt[1]);
      product(wt[0], acc);
    } else {
      if (nxt < blocks) load(nxt, wt[0]);
      product(wt[1], acc);
    }
    cur ^= 1;
    // acc[m]: activation row i16, weight rows 16 blk + 4g + r; the waves'
    // sums meet in LDS and are added in wave order
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][m][r][lane] = acc[m][r];
    __syncthreads();
    for (int e = tid; e < 256; e += 64 * W) {
      const int m16 = e / 16, n16 = e % 16;
      const int src = m16 + 16 * (n16 >> 2), r = n16 & 3;
      const int n = 16 * blk + n16;
      float tot[MATS];
#pragma unroll
      for (int m = 0; m < MATS; ++m) {
        float v = red[0][m][r][src];
#pragma unroll
        for (int w = 1; w < W; ++w) v += red[w][m][r][src];
        tot[m] = v;
      }
      if (m16 < p.M && n < p.N) {
        const float gs = (float)act_f64(kSilu, (double)(tot[0] * p.scale[0][n]));
        p.pre[(size_t)m16 * p.out_stride + n] = (float)((double)gs * (double)(tot[1] * p.scale[1][n]));
      }
    }
    __syncthreads();  // red is rewritten by the next block
  }
}

// Whether a small-M product takes k_mxr: the SwiGLU gate+up pair with three
// activation terms, enough 16-row blocks for every CU and at least one
// chunk per wave, at most 16 chunks per wave.
bool mxr_fits(const MxgArgs& p) {
  const int S = p.kpad / 128;
  return p.mats == 2 && p.terms == kTerms && p.a != nullptr && (p.N + 15) / 16 >= 256 &&
         S >= kRowWaves && (S + kRowWaves - 1) / kRowWaves <= 16;
}

template <int DT, bool BLK, int MATS, int MB, int NS, int W, bool ROT, int RB = 1>
void launch_mxr_grid(const MxgArgs& p, dim3 grid, hipStream_t st) {
  constexpr int D = NS < 3 ? NS : 3;
  k_mxr<DT, BLK, MATS, MB, NS, D, W, ROT, RB><<<grid, 64 * W, 0, st>>>(p);
}

// The large-tile products split along K (mxg_ksplit > 1: fewer than 128
// tiles of 128 x 128, such as the 256 x 1024 x 1024 layers of a serial volume
// chain) take k_mxr instead when they have one matrix, three activation
// terms and 2..128 K chunks: 16 (chained: 32) weight rows x 32 activation
// rows per workgroup (grid.y over the pairs of row blocks), 8 waves over K,
// no partial sums and no reduce launch. (A fused RoPE takes no K split.)
int mxg_ksplit(int M, int kpad, int N, int mats);
bool replaces_ksplit(int M, int kpad, int N, int mats, int terms) {
  const int S = kpad / 128;
  return mats == 1 && terms == kTerms && M > 32 && mxg_ksplit(M, kpad, N, mats) > 1 &&
         S >= 2 && S <= 16 * kRowWaves;
}

template <int DT, bool BLK, int RB>
void launch_mxr_large_rb(const MxgArgs& p, hipStream_t st) {
  const int ns = (p.kpad / 128 + kRowWaves - 1) / kRowWaves;
  const dim3 grid((unsigned)((p.N + 16 * RB - 1) / (16 * RB)), (unsigned)(p.mpad / 32));
  if (ns <= 1) launch_mxr_grid<DT, BLK, 1, 2, 1, kRowWaves, false, RB>(p, grid, st);
  else if (ns <= 2) launch_mxr_grid<DT, BLK, 1, 2, 2, kRowWaves, false, RB>(p, grid, st);
  else if (ns <= 4) launch_mxr_grid<DT, BLK, 1, 2, 4, kRowWaves, false, RB>(p, grid, st);
  else if (ns <= 8) launch_mxr_grid<DT, BLK, 1, 2, 8, kRowWaves, false, RB>(p, grid, st);
  else launch_mxr_grid<DT, BLK, 1, 2, 16, kRowWaves, false, RB>(p, grid, st);
}

// 16 weight rows per workgroup; 32 for a chained product, whose epilogue
// then holds whole 32-column blocks of post and writes the next layer's split
// (the K ranges of the waves, and so every sum, are the same for both).
template <int DT, bool BLK>
Status launch_mxr_large(const MxgArgs& p, hipStream_t st) {
  if (p.next) {
    if (p.N % 128 != 0) return Status::err(kInvalid, "mxr: a chained split needs N % 128 == 0");
    launch_mxr_large_rb<DT, BLK, 2>(p, st);
  } else {
    launch_mxr_large_rb<DT, BLK, 1>(p, st);
  }
  return hip_status(hipGetLastError(), "mxr launch");
}

template <int DT, bool BLK, int MATS, int MB>
Status launch_rows(const MxgArgs& p, hipStream_t st) {
  // x -> the three-term split in the product's split buffer
  WV_TRY(launch_split(p.x, p.x_stride, p.M, p.cols, p.kpad, const_cast<uint8_t*>(p.a), st, kTerms));
  const int ns = (p.kpad / 128 + kRowWaves - 1) / kRowWaves;
  const unsigned grid = (unsigned)((p.N + 15) / 16);
  if constexpr (DT == kFP4 && MATS == 2 && MB == 1) {
    if (ns <= 4 && p.codesf[0] && p.codesf[1]) {
      const int cus = cu_count();
      const unsigned pgrid = (unsigned)(cus > 0 && (unsigned)cus < grid ? cus : grid);
      k_mxp<DT, BLK, 4><<<pgrid, 64 * kRowWaves, 0, st>>>(p);
      return hip_status(hipGetLastError(), "mxp launch");
    }
  }
  constexpr int D = MB == 1 ? 3 : 2;
  constexpr int W = kRowWaves;
  if (ns <= 4) k_mxr<DT, BLK, MATS, MB, 4, D, W, true><<<grid, 64 * W, 0, st>>>(p);
  else if (ns <= 8) k_mxr<DT, BLK, MATS, MB, 8, D, W, true><<<grid, 64 * W, 0, st>>>(p);
  else if (ns <= 12) k_mxr<DT, BLK, MATS, MB, 12, D, W, true><<<grid, 64 * W, 0, st>>>(p);
  else k_mxr<DT, BLK, MATS, MB, 16, D, W, true><<<grid, 64 * W, 0, st>>>(p);
  return hip_status(hipGetLastError(), "mxr launch");
}

template <int DT, bool BLK, int MATS, int MB, int RB, int KRT, bool XV = true>
void launch_small_krt(const MxgArgs& p, int ksplit, hipStream_t st) {
  constexpr int NT3 = kTerms;
  // ring depth: 6-14 KiB of weights in flight per wave within the register
  // budget of two waves per SIMD
  constexpr int D0 = (DT == kFP4 ? 8 : 6) / MATS + (DT == kFP4 && MATS == 2 ? 2 : 0);
  constexpr int D1 = RB == 2 ? (D0 + 1) / 2 + 1 : D0;
  constexpr int D = D1 < KRT ? D1 : KRT;
  const int rows = 16 * kSmallWaves * RB;
  const dim3 grid((unsigned)((p.N + rows - 1) / rows), (unsigned)ksplit);
  // two activation terms: Dense only (one matrix)
  if constexpr (MATS == 1) {
    if (p.terms == 2) {
      k_mxs<DT, BLK, MATS, MB, RB, KRT, D, XV, 2><<<grid, 64 * kSmallWaves, 0, st>>>(p, ksplit);
      return;
    }
  }
  k_mxs<DT, BLK, MATS, MB, RB, KRT, D, XV, NT3><<<grid, 64 * kSmallWaves, 0, st>>>(p, ksplit);
}

template <int DT, bool BLK, int MATS, int MB, int RB>
void launch_small_rb(const MxgArgs& p, int ksplit, hipStream_t st) {
  const int S = p.kpad / 128, kr = (S + ksplit - 1) / ksplit;  // largest range
  constexpr int K1 = MB == 1 ? 4 : 4, K2 = MB == 1 ? 8 : 8, K3 = MB == 1 ? 12 : 12;
  // element loads of an unaligned input: one variant (the largest range)
  if (!p.x_vec) launch_small_krt<DT, BLK, MATS, MB, RB, small_krt_max(MB), false>(p, ksplit, st);
  else if (kr <= K1) launch_small_krt<DT, BLK, MATS, MB, RB, K1>(p, ksplit, st);
  else if (kr <= K2) launch_small_krt<DT, BLK, MATS, MB, RB, K2>(p, ksplit, st);
  else if (kr <= K3 || MB == 2) launch_small_krt<DT, BLK, MATS, MB, RB, K3>(p, ksplit, st);
  else if (kr <= 16) launch_small_krt<DT, BLK, MATS, MB, RB, (MB == 1 ? 16 : 12)>(p, ksplit, st);
  else launch_small_krt<DT, BLK, MATS, MB, RB, small_krt_max(MB)>(p, ksplit, st);
}

template <int DT, bool BLK, int MATS, int MB>
Status launch_small(const MxgArgs& p, hipStream_t st) {
  if (!p.x || p.cols <= 0 || p.cols > p.kpad || p.x_stride < p.cols || p.M <= 0 || p.M > p.mpad)
    return Status::err(kInvalid, "mxg: small-M input");
  if constexpr (MATS == 2) {
    if (mxr_fits(p)) return launch_rows<DT, BLK, MATS, MB>(p, st);
  }
  const int ksplit = mxs_ksplit(p.N, p.kpad, p.mpad);
  if (ksplit > 1 && !p.part) return Status::err(kInvalid, "mxg: K-split partial buffer missing");
  const int rb = mxs_rb(p.N);
  if (rb == 2) launch_small_rb<DT, BLK, MATS, MB, 2>(p, ksplit, st);
  else launch_small_rb<DT, BLK, MATS, MB, 1>(p, ksplit, st);
  if (ksplit > 1) {
    // the kernel boundary makes every split's partial sums visible (the
    // XCDs' L2 caches are not coherent with each other)
    launch_mxs_reduce(p, ksplit, 16 * kSmallWaves * rb, MATS, st);
  }
  return hip_status(hipGetLastError(), "mxs launch");
}

// Split along K for a large-tile product of one matrix with few tiles (fewer
// than 128 of 128 columns): whole step pairs per split, about 256 workgroups
// in all. Used when no RoPE is fused into the epilogue: the reduce kernel
// applies the scale and epilogue (and writes a chained split).
int mxg_ksplit(int M, int kpad, int N, int mats) {
  if (M <= 32 || mats != 1) return 1;
  const int64_t tiles = round_up(M, kBM) / kBM * ((N + 127) / 128);
  const int pairs = kpad / 256;
  if (tiles >= 128 || pairs < 2) return 1;
  const int ks = (int)(256 / tiles);
  return ks < pairs ? ks : pairs;
}

template <int DT, bool BLK, int MATS>
Status launch_t(const MxgArgs& p, int bm, hipStream_t st) {
  if (p.rope_tab && (bm != kBM || MATS != 1 || p.need_epi || p.next || p.rope_hd <= 0 ||
                     p.rope_hd % 8 != 0 || 128 % p.rope_hd != 0))
    return Status::err(kInvalid, "mxg: RoPE epilogue needs the large tiles, one matrix, no epilogue");
  if (bm == kBM) {
    if ((size_t)kTerms * p.mpad * p.kpad >= (1ull << 31) ||
        (size_t)round_up(p.N, 256) * p.pitch >= (1ull << 31))
      return Status::err(kUnsupported, "mxg: operands above 2 GiB");
    const int tiles_m = p.mpad / kBM;
    // with p.next set, a K split ends in the reduce that also writes the
    // next layer's split (launch_reduce_split); unsplit, the epilogue does
    const int ks = p.rope_tab ? 1 : mxg_ksplit(p.M, p.kpad, p.N, MATS);
    if (p.next && (MATS != 1 || p.N % 256 != 0 || (ks == 1 && p.need_epi)))
      return Status::err(kInvalid, "mxg: a chained split needs one matrix, N % 256 == 0 and, "
                                   "unsplit, no epilogue");
    // the split reduce stores 16-byte vectors of pre and post
    if (p.next && ks > 1 &&
        (p.out_stride % 4 != 0 || ((reinterpret_cast<uintptr_t>(p.pre) | reinterpret_cast<uintptr_t>(p.post)) & 15)))
      return Status::err(kInvalid, "mxg: a chained split reduce needs 16-byte aligned outputs");
    if constexpr (MATS == 1) {
      if (ks > 1 && replaces_ksplit(p.M, p.kpad, p.N, MATS, p.terms))
        return launch_mxr_large<DT, BLK>(p, st);
      if (ks > 1) {
        if (!p.part) return Status::err(kInvalid, "mxg: K-split partial buffer missing");
        const int tiles_n = (p.N + 127) / 128;
        const dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)ks);
        if (p.terms == 1)
          k_mxg<DT, BLK, 1, false, kMxgWaves, 128, true, 1><<<grid, 64 * kMxgWaves, 0, st>>>(
              p, nullptr, tiles_m, tiles_n);
        else if (p.terms == 2)
          k_mxg<DT, BLK, 1, false, kMxgWaves, 128, true, 2><<<grid, 64 * kMxgWaves, 0, st>>>(
              p, nullptr, tiles_m, tiles_n);
        else
          k_mxg<DT, BLK, 1, false, kMxgWaves, 128, true><<<grid, 64 * kMxgWaves, 0, st>>>(
              p, nullptr, tiles_m, tiles_n);
        // the kernel boundary makes every split's partial sums visible
        if (p.next) {
          launch_reduce_split(p, ks, st);
        } else {
          launch_mxs_reduce(p, ks, 256, 1, st);
        }
        return hip_status(hipGetLastError(), "mxg K-split launch");
      }
    }
    const bool wide = mxg_wide(1, tiles_m, p.N, MATS);
    const int tiles_n = wide ? (p.N + 256 / MATS - 1) / (256 / MATS) : (p.N + 128 / MATS - 1) / (128 / MATS);
    const unsigned grid = (unsigned)(tiles_m * tiles_n);
    if constexpr (MATS == 1) {
      if (p.terms == 1) {
        if (wide)
          k_mxg<DT, BLK, 1, false, kMxgWaves, 256, false, 1><<<grid, 64 * kMxgWaves, 0, st>>>(
              p, nullptr, tiles_m, tiles_n);
        else
          k_mxg<DT, BLK, 1, false, kMxgWaves, 128, false, 1><<<grid, 64 * kMxgWaves, 0, st>>>(
              p, nullptr, tiles_m, tiles_n);
        return hip_status(hipGetLastError(), "mxg launch");
      }
      if (p.terms == 2) {
        if (wide)
          k_mxg<DT, BLK, 1, false, kMxgWaves, 256, false, 2><<<grid, 64 * kMxgWaves, 0, st>>>(
              p, nullptr, tiles_m, tiles_n);
        else
          k_mxg<DT, BLK, 1, false, kMxgWaves, 128, false, 2><<<grid, 64 * kMxgWaves, 0, st>>>(
              p, nullptr, tiles_m, tiles_n);
        return hip_status(hipGetLastError(), "mxg launch");
      }
    }
    if (wide)
      k_mxg<DT, BLK, MATS, false, kMxgWaves, 256><<<grid, 64 * kMxgWaves, 0, st>>>(p, nullptr,
                                                                                  tiles_m, tiles_n);
    else
      k_mxg<DT, BLK, MATS, false, kMxgWaves, 128><<<grid, 64 * kMxgWaves, 0, st>>>(p, nullptr,
                                                                                  tiles_m, tiles_n);
  } else {
    return p.mpad <= 16 ? launch_small<DT, BLK, MATS, 1>(p, st) : launch_small<DT, BLK, MATS, 2>(p, st);
  }
  return hip_status(hipGetLastError(), "mxg launch");
}

template <int MATS>
Status launch_m(const MxgArgs& p, int dtype, bool blk, int bm, hipStream_t st) {
  if (p.terms < 1 || p.terms > kTerms) return Status::err(kInvalid, "mxg: terms must be 1, 2 or 3");
  if (MATS == 2 && p.terms != kTerms)
    return Status::err(kUnsupported, "mxg: fewer activation terms are for one-matrix products");
  if (p.terms == 1 && bm != kBM)
    return Status::err(kUnsupported, "mxg: one activation term needs more than 32 rows");
  switch (dtype) {
  case kE4M3: return blk ? launch_t<kE4M3, true, MATS>(p, bm, st) : launch_t<kE4M3, false, MATS>(p, bm, st);
  case kE5M2: return blk ? launch_t<kE5M2, true, MATS>(p, bm, st) : launch_t<kE5M2, false, MATS>(p, bm, st);
  case kFP4: return blk ? launch_t<kFP4, true, MATS>(p, bm, st) : launch_t<kFP4, false, MATS>(p, bm, st);
  }
  return Status::err(kUnsupported, "mxg: dtype");
}

}  // namespace

int mxg_block_m(int M) { return M <= 32 ? 16 : kBM; }

size_t mxg_part_bytes(int M, int kpad, int N, int mats) {
  if (mxg_block_m(M) != 16) {
    const int ks = mxg_ksplit(M, kpad, N, mats);
    return ks > 1 ? (size_t)ks * round_up(M, kBM) * round_up(N, 256) * sizeof(float) : 0;
  }
  const int mpad = (int)round_up(M, 16);
  const int ks = mxs_ksplit(N, kpad, mpad);
  const int rows = 16 * kSmallWaves * mxs_rb(N);
  return ks > 1 ? (size_t)ks * mats * mpad * round_up(N, rows) * sizeof(float) : 0;
}

size_t split_bytes(int M, int kpad) {
  const size_t mpad = (size_t)round_up(M, mxg_block_m(M));
  // term codes, then one exponent dword per (16-row block, K chunk, lane)
  return (size_t)kTerms * mpad * kpad + mpad * (size_t)kpad / 8;
}

// Splits of at least this many code bytes per launch are written with
// streaming stores (the eight XCD L2s hold 32 MB together). Smaller ones,
// such as the 4096 x 1024 input of a projection (12.6 MB counted, 9.4 MB of
// FP6 terms), keep plain stores, which leave the split in the L2s for the
// product that reads it next: 4096 x 1024 x 1024 Dense 20.70-20.73 us
// against 20.82-21.00 us with streaming stores.
constexpr size_t kStreamSplitBytes = 16u << 20;

Status launch_split(const float* x, int x_stride, int M, int cols, int kpad, uint8_t* buf,
                    hipStream_t st, int terms) {
  if (terms < 1 || terms > kTerms) return Status::err(kInvalid, "split: terms must be 1, 2 or 3");
  if (kpad % 128 != 0) return Status::err(kInvalid, "split: kpad must be a multiple of 128");
  const int mpad = (int)round_up(M, mxg_block_m(M));
  uint8_t* a = buf;
  uint8_t* as = buf + (size_t)kTerms * mpad * kpad;
  const int64_t waves = (int64_t)(mpad / 16) * (kpad / 128);
  const unsigned grid = (unsigned)((waves + kThreads / 64 - 1) / (kThreads / 64));
  const bool vec = x_stride % 4 == 0 && cols % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  const int stream = (size_t)terms * mpad * kpad >= kStreamSplitBytes;
  if (terms == 1) {
    if (vec) k_split<true, 1><<<grid, kThreads, 0, st>>>(x, x_stride, M, cols, mpad, kpad, a, as, nullptr, stream);
    else k_split<false, 1><<<grid, kThreads, 0, st>>>(x, x_stride, M, cols, mpad, kpad, a, as, nullptr, stream);
  } else if (terms == 2) {
    if (vec) k_split<true, 2><<<grid, kThreads, 0, st>>>(x, x_stride, M, cols, mpad, kpad, a, as, nullptr, stream);
    else k_split<false, 2><<<grid, kThreads, 0, st>>>(x, x_stride, M, cols, mpad, kpad, a, as, nullptr, stream);
  } else {
    // three terms: FP6 (act_fp6)
    if (vec) k_split<true, kTerms, true><<<grid, kThreads, 0, st>>>(x, x_stride, M, cols, mpad, kpad, a, as, nullptr, stream);
    else k_split<false, kTerms, true><<<grid, kThreads, 0, st>>>(x, x_stride, M, cols, mpad, kpad, a, as, nullptr, stream);
  }
  return hip_status(hipGetLastError(), "split launch");
}

Status launch_split_group(const SplitJob* jobs, int n, bool vec, int x_stride, int M, int cols,
                          int kpad, hipStream_t st, int terms) {
  if (terms < 1 || terms > kTerms) return Status::err(kInvalid, "split: terms must be 1, 2 or 3");
  if (n <= 0 || !jobs) return Status::err(kInvalid, "split group: no members");
  if (kpad % 128 != 0) return Status::err(kInvalid, "split: kpad must be a multiple of 128");
  const int mpad = (int)round_up(M, mxg_block_m(M));
  const int64_t waves = (int64_t)(mpad / 16) * (kpad / 128);
  const dim3 grid((unsigned)((waves + kThreads / 64 - 1) / (kThreads / 64)), (unsigned)n);
  const int stream = (size_t)terms * mpad * kpad * n >= kStreamSplitBytes;
  if (terms == 1) {
    if (vec) k_split<true, 1><<<grid, kThreads, 0, st>>>(nullptr, x_stride, M, cols, mpad, kpad, nullptr, nullptr, jobs, stream);
    else k_split<false, 1><<<grid, kThreads, 0, st>>>(nullptr, x_stride, M, cols, mpad, kpad, nullptr, nullptr, jobs, stream);
  } else if (terms == 2) {
    if (vec) k_split<true, 2><<<grid, kThreads, 0, st>>>(nullptr, x_stride, M, cols, mpad, kpad, nullptr, nullptr, jobs, stream);
    else k_split<false, 2><<<grid, kThreads, 0, st>>>(nullptr, x_stride, M, cols, mpad, kpad, nullptr, nullptr, jobs, stream);
  } else {
    // three terms: FP6 (act_fp6)
    if (vec) k_split<true, kTerms, true><<<grid, kThreads, 0, st>>>(nullptr, x_stride, M, cols, mpad, kpad, nullptr, nullptr, jobs, stream);
    else k_split<false, kTerms, true><<<grid, kThreads, 0, st>>>(nullptr, x_stride, M, cols, mpad, kpad, nullptr, nullptr, jobs, stream);
  }
  return hip_status(hipGetLastError(), "split group launch");
}

template <int DT, bool BLK, int MATS>
Status launch_group_t(const MxgArgs* tab, const MxgArgs& p, int n, hipStream_t st) {
  const int tiles_m = p.mpad / kBM;
  const bool wide = mxg_wide(n, tiles_m, p.N, MATS);
  const int tiles_n = wide ? (p.N + 256 / MATS - 1) / (256 / MATS) : (p.N + 128 / MATS - 1) / (128 / MATS);
  const unsigned grid = (unsigned)(n * tiles_m * tiles_n);
  if constexpr (MATS == 1) {
    if (p.terms == 1) {
      if (wide)
        k_mxg<DT, BLK, 1, true, kMxgWaves, 256, false, 1><<<grid, 64 * kMxgWaves, 0, st>>>(
            p, tab, tiles_m, tiles_n);
      else
        k_mxg<DT, BLK, 1, true, kMxgWaves, 128, false, 1><<<grid, 64 * kMxgWaves, 0, st>>>(
            p, tab, tiles_m, tiles_n);
      return hip_status(hipGetLastError(), "mxg group launch");
    }
    if (p.terms == 2) {
      if (wide)
        k_mxg<DT, BLK, 1, true, kMxgWaves, 256, false, 2><<<grid, 64 * kMxgWaves, 0, st>>>(
            p, tab, tiles_m, tiles_n);
      else
        k_mxg<DT, BLK, 1, true, kMxgWaves, 128, false, 2><<<grid, 64 * kMxgWaves, 0, st>>>(
            p, tab, tiles_m, tiles_n);
      return hip_status(hipGetLastError(), "mxg group launch");
    }
  }
  if (wide)
    k_mxg<DT, BLK, MATS, true, kMxgWaves, 256><<<grid, 64 * kMxgWaves, 0, st>>>(p, tab, tiles_m,
                                                                               tiles_n);
  else
    k_mxg<DT, BLK, MATS, true, kMxgWaves, 128><<<grid, 64 * kMxgWaves, 0, st>>>(p, tab, tiles_m,
                                                                               tiles_n);
  return hip_status(hipGetLastError(), "mxg group launch");
}

Status launch_mxg_group(const MxgArgs* tab, const MxgArgs& p, int n, int dtype, bool blk,
                        hipStream_t st) {
  if (n <= 0 || !tab) return Status::err(kInvalid, "mxg group: no members");
  if (p.terms < 1 || p.terms > kTerms) return Status::err(kInvalid, "mxg: terms must be 1, 2 or 3");
  if (p.mats == 2 && p.terms != kTerms)
    return Status::err(kUnsupported, "mxg: fewer activation terms are for one-matrix products");
  if (mxg_block_m(p.M) != kBM || p.mpad % kBM != 0 || p.kpad % 256 != 0)
    return Status::err(kInvalid, "mxg group: needs the large-tile layout");
  if ((size_t)kTerms * p.mpad * p.kpad >= (1ull << 31) ||
      (size_t)round_up(p.N, 256) * p.pitch >= (1ull << 31))
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
