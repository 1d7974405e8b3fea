// MHA ModeSelf attention core with the reference's indexing
// (src/cuda/kernels.cu:470-631):
//   token t = b*seq + s sits at global position pos = t;
//   queries of batch b see key positions k_pos in [0, b*seq + seq) allowed by
//   the mask (:470-485), scored against the KV ring row k_pos % msl, which by
//   then holds the latest position p <= last = b*seq + seq - 1 with
//   p == k_pos (mod msl): p = last - ((last - k_pos) mod msl);
//   RoPE rotates Q and K at their global position (:487-504), ALiBi uses
//   k_pos (:526-533); softmax or sigmoid over the allowed keys (:603-619).
// The reference loop is serial f64 on one thread. Here the causal and
// bidirectional masks without ALiBi run on the matrix cores (k_attn_mfma,
// below); the other masks take k_attention, where one wave handles one
// (token, head), keys are scored 64 at a time (one per lane), and the
// softmax is accumulated online in fp32. RoPE is applied by the Q and K
// projections' GEMM epilogue when they run on the large tiles, else by
// k_rope before either kernel.
#include "common.h"
#include "kernels.h"
#include "split.h"

namespace wv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// x as three bf16 terms hi + mid + lo, each rounding the remainder of the
// previous ones (to nearest even): x - hi - mid - lo is below 2^-24 |x|
// (three 8-bit significands)
__device__ __forceinline__ void split3(float x, __bf16 (&t)[3]) {
  const __bf16 hi = (__bf16)x;
  const float r1 = x - (float)hi;
  const __bf16 mid = (__bf16)r1;
  t[0] = hi;
  t[1] = mid;
  t[2] = (__bf16)(r1 - (float)mid);
}

__device__ __forceinline__ bool allow(int qp, int kp, const AttnArgs& a) {
  if (a.mask == 2) return true;
  if (a.mask == 3) {
    const int w = a.window > 0 ? a.window : a.msl;
    if (a.window_causal) return kp <= qp && kp >= qp - w + 1;
    const int d = qp > kp ? qp - kp : kp - qp;
    return d < w;
  }
  if (a.mask == 4) {
    if (qp < a.prefix_len && kp < a.prefix_len) return true;
    return kp <= qp;
  }
  return kp <= qp;
}

__device__ __forceinline__ double rope_angle(int t, int d, int hd, double theta) {
  return (double)t / pow(theta, (double)(2 * d) / (double)hd);
}

__global__ void k_rope_table(double* __restrict__ tab, int tokens, int hd, double theta) {
  const int half = hd / 2;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tokens * half) return;
  const double ang = rope_angle(i / half, i % half, hd, theta);
  tab[2 * i] = cos(ang);
  tab[2 * i + 1] = sin(ang);
}

// Rotates the pair (d, d + hd/2) of every head of Q (num_heads) and K
// (num_kv) rows of token t by angle t / theta^(2d/hd), in f64 (cos and sin
// from the table when one is given).
__global__ void k_rope(float* __restrict__ q, float* __restrict__ k, int tokens, int heads,
                       int kv_heads, int hd, double theta, const double* __restrict__ tab) {
  const int t = blockIdx.x;
  const int half = hd / 2;
  const int per_tok = (heads + kv_heads) * half;
  for (int i = threadIdx.x; i < per_tok; i += blockDim.x) {
    const int h = i / half, d = i % half;
    float* row = h < heads ? q + ((size_t)t * heads + h) * hd
                           : k + ((size_t)t * kv_heads + (h - heads)) * hd;
    double c, s;
    if (tab) {
      c = tab[2 * (t * half + d)];
      s = tab[2 * (t * half + d) + 1];
    } else {
      const double ang = rope_angle(t, d, hd, theta);
      c = cos(ang), s = sin(ang);
    }
    const double a0 = row[d], a1 = row[d + half];
    row[d] = (float)(a0 * c - a1 * s);
    row[d + half] = (float)(a0 * s + a1 * c);
  }
}

constexpr int kMaxHdPerLane = 4;  // head_dim <= 256

__global__ __launch_bounds__(64) void k_attention(AttnArgs a) {
  const int t = blockIdx.x;  // query token
  const int h = blockIdx.y;  // query head
  const int lane = threadIdx.x;
  const int b = t / a.seq;
  const int qp = t;
  const int kv_len = b * a.seq + a.seq;
  const int last = kv_len - 1;
  const int kvh = h / (a.heads / a.kv_heads);
  const int qd = a.heads * a.hd, kvd = a.kv_heads * a.hd;
  const float* qv = a.q + (size_t)t * qd + (size_t)h * a.hd;

  __shared__ float qs[256];
  for (int d = lane; d < a.hd; d += 64) qs[d] = qv[d];
  __syncthreads();

  float m = -INFINITY, l = 0.0f;
  float acc[kMaxHdPerLane];
#pragma unroll
  for (int i = 0; i < kMaxHdPerLane; ++i) acc[i] = 0.0f;
  int n_allowed = 0;

  double slope = 0.0;
  if (a.alibi) slope = pow(2.0, -(double)(h + 1) * 8.0 / (double)(a.heads > 0 ? a.heads : 1));

  for (int base = 0; base < kv_len; base += 64) {
    const int kp = base + lane;
    bool ok = kp < kv_len && allow(qp, kp, a);
    int p = 0;
    float s = -INFINITY;
    if (ok) {
      p = last - ((last - kp) % a.msl);
      const float* kr = a.k + (size_t)p * kvd + (size_t)kvh * a.hd;
      float dot = 0.0f;
      for (int d = 0; d < a.hd; d += 4) {
        const float4 kk = *reinterpret_cast<const float4*>(kr + d);
        dot = fmaf(qs[d], kk.x, dot);
        dot = fmaf(qs[d + 1], kk.y, dot);
        dot = fmaf(qs[d + 2], kk.z, dot);
        dot = fmaf(qs[d + 3], kk.w, dot);
      }
      double sc = (double)dot * a.scale;
      if (a.alibi) {
        const int dd = qp > kp ? qp - kp : kp - qp;
        sc += -slope * (double)dd;
      }
      s = (float)sc;
    }
    const unsigned long long mask_bits = __ballot(ok);
    n_allowed += __popcll(mask_bits);
    if (mask_bits == 0ull) continue;
    float w;
    if (a.sigmoid) {
      w = ok ? 1.0f / (1.0f + expf(-s)) : 0.0f;
    } else {
      float bm = s;
      for (int off = 32; off > 0; off >>= 1) bm = fmaxf(bm, __shfl_xor(bm, off, 64));
      const float nm = fmaxf(m, bm);
      const float corr = (m == -INFINITY) ? 0.0f : expf(m - nm);
      w = ok ? expf(s - nm) : 0.0f;
      float ws = w;
      for (int off = 32; off > 0; off >>= 1) ws += __shfl_xor(ws, off, 64);
      l = l * corr + ws;
#pragma unroll
      for (int i = 0; i < kMaxHdPerLane; ++i) acc[i] *= corr;
      m = nm;
    }
    // acc[d] += sum_j w_j V[p_j][d]; lane owns dims lane, lane+64, ...
    for (int j = 0; j < 64; ++j) {
      const float wj = __shfl(w, j, 64);
      if (((mask_bits >> j) & 1ull) == 0ull) continue;
      const int pj = __shfl(p, j, 64);
      const float* vr = a.v + (size_t)pj * kvd + (size_t)kvh * a.hd;
#pragma unroll
      for (int i = 0; i < kMaxHdPerLane; ++i) {
        const int d = lane + 64 * i;
        if (d < a.hd) acc[i] = fmaf(wj, vr[d], acc[i]);
      }
    }
  }
  float* out = a.out + (size_t)t * qd + (size_t)h * a.hd;
  const float inv = (a.sigmoid || n_allowed == 0) ? 1.0f : 1.0f / l;
#pragma unroll
  for (int i = 0; i < kMaxHdPerLane; ++i) {
    const int d = lane + 64 * i;
    if (d < a.hd) out[d] = n_allowed == 0 ? 0.0f : acc[i] * inv;
  }
}


// ---------------------------------------------------------------------------
// Matrix-core path for the causal and bidirectional masks without ALiBi.
//
// Under the reference indexing a query of batch b scans key positions
// kp in [0, b*seq + seq), and kp reads ring row p = last - ((last - kp) mod
// msl), so only the rows p in [max(0, last - msl + 1), last] occur, row p
// once for every allowed kp == p (mod msl). The score of a key depends on
// its row only (no ALiBi), so the softmax over key positions equals a
// softmax over distinct rows with multiplicity weights:
//   bidirectional: c(p) = floor(p / msl) + 1 (every kp = p - i*msl >= 0),
//   causal:        c(p) - 1 when p > qp (only kp = p itself is masked out:
//                  p - msl <= last - msl < b*seq <= qp since msl >= seq).
// Scores and sums are the same function of the same values; only the fp32
// summation order differs from the per-position loop.
//
// A workgroup of 16 waves (8 at hd 128) takes 16 queries per wave of one
// (batch, head) and walks the distinct rows in tiles of 64 keys staged in LDS in
// matrix-core operand order, double-buffered through registers, one barrier
// per tile. Per 16-key block a wave runs
//   S^T = K Q^T  on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16, hd/32
//                steps), Q and K each split into two bf16 terms hi + lo
//                (x - hi - lo ~ 2^-17 |x|), and the three products down to
//                2^-16 relative kept (hh, hl, lh): the scores carry ~2^-16
//                relative accuracy. Lane l holds the scores of query l%16 for keys
//                4*(l/16) + i, i = 0..3;
//   O^T += V^T P^T: the same 4 values per lane are the B operand (MFMA k
//                index l/16 <-> key 4*(l/16) + j at step j), V^T the A
//                operand, so no transpose is needed.
// The scores of a whole tile (4 blocks) are formed first, so the online
// softmax (fp32, per query: max and sum over the 4 lanes that share a
// query, xor 16 / xor 32) and the rescaling of O happen once per 64 keys.
// The softmax runs in base 2 (scores scaled by log2 e, weights from the
// hardware exp2, within a few ulp of e^x).
// Waves per workgroup, 16 queries each: 16 up to head_dim 64 (one
// 1024-thread workgroup per CU, four waves per SIMD, each K/V tile staged
// once for 256 queries: the B=8, S=512, 16x64 layer measured 0.1367 ms with
// 8-wave workgroups, two per CU, and 0.1301 ms with 16), 8 for head_dim 128
// (whose waves need more than 128 registers).
constexpr int attn_waves(int hd) { return hd <= 64 ? 16 : 8; }
constexpr int kKT = 64;  // keys per LDS tile

template <int HD, bool SIG>
__global__ __launch_bounds__(64 * attn_waves(HD)) __attribute__((amdgpu_waves_per_eu(HD <= 64 ? 4 : 2, 8)))
void k_attn_mfma(AttnArgs a, int qblocks) {
  constexpr int KS = HD / 32;                           // QK MFMA steps (32 head dims)
  constexpr int DT = HD / 16;                           // 16-wide head-dim tiles of O
  constexpr int kAttnWaves = attn_waves(HD);
  constexpr int kQB = 16 * kAttnWaves;                  // queries per workgroup
  constexpr int NT = 64 * kAttnWaves;                   // threads
  // K in bf16 operand order: [16-key block kb][step ks][hi, lo][lane][8]:
  // lane 16 g + c16 holds key 16 kb + c16, head dims 32 ks + 8 g + j
  constexpr int KBYTES = 4 * KS * 2 * 1024;
  __shared__ __attribute__((aligned(16))) uint8_t ksb[2][KBYTES];
  // V in bf16 operand order: [32-key group q][head-dim tile dt][hi, lo][lane][8]
  constexpr int VBYTES = 2 * DT * 2 * 1024;
  __shared__ __attribute__((aligned(16))) uint8_t vsb[2][VBYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, g = lane >> 4;
  const int b = blockIdx.x / qblocks, qb = blockIdx.x % qblocks;
  const int h = blockIdx.y;
  const int kvh = h / (a.heads / a.kv_heads);
  const int qd = a.heads * HD, kvd = a.kv_heads * HD;
  const int last = b * a.seq + a.seq - 1;
  const int p_lo = last - a.msl + 1 > 0 ? last - a.msl + 1 : 0;
  const int s_q = qb * kQB + wave * 16 + c16;      // query within the sequence
  const bool q_ok = s_q < a.seq;
  const int qp = b * a.seq + (q_ok ? s_q : a.seq - 1);
  const bool causal = a.mask == 1;
  // score scales: softmax weights are 2^(s log2 e - max), in log2 units;
  // the sigmoid variant works in natural units
  const float scale_log2 = (float)(a.scale * 1.4426950408889634);
  const float scale_nat = (float)a.scale;

  // Q operand: lane (query c16, group g), head dims 32 ks + 8 g + j, as
  // two bf16 terms (hi and the rounded remainder: 16 significand bits, as K)
  bf16x8 qop[KS][2];
  {
    const float* qrow = a.q + (size_t)qp * qd + (size_t)h * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const v4f q0 = *reinterpret_cast<const v4f*>(qrow + 32 * ks + 8 * g);
      const v4f q1 = *reinterpret_cast<const v4f*>(qrow + 32 * ks + 8 * g + 4);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        __bf16 t3[3];
        split3(j < 4 ? q0[j] : q1[j - 4], t3);
        qop[ks][0][j] = t3[0], qop[ks][1][j] = t3[1];
      }
    }
  }
  v4f o[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = v4f{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  // K and V rows of a tile in pair units: unit i = tid + NT u covers row
  // i / (HD/8) and the column quads c4 and c4 + HD/2, c4 = 4 (i % (HD/8)).
  // Rows past `last` are exact zeros (a tile wholly past it is a zero tile:
  // the loads stay unconditional).
  constexpr int UNITS = kKT * HD / 8, PU = (UNITS + NT - 1) / NT;
  v4f kreg[2 * PU], vreg[2 * PU];
  auto load_k = [&](int t0) {
#pragma unroll
    for (int u = 0; u < PU; ++u) {
      const int i = tid + NT * u;
      if (UNITS % NT != 0 && i >= UNITS) break;  // whole waves (HD = 32)
      const int r = i / (HD / 8), c4 = (i % (HD / 8)) * 4;
      const int p = t0 + r, pc = p <= last ? p : last;
      const size_t off = (size_t)pc * kvd + (size_t)kvh * HD + c4;
      const v4f k0 = *reinterpret_cast<const v4f*>(a.k + off);
      const v4f k1 = *reinterpret_cast<const v4f*>(a.k + off + HD / 2);
      const v4f z = v4f{0.f, 0.f, 0.f, 0.f};
      kreg[2 * u] = p <= last ? k0 : z;
      kreg[2 * u + 1] = p <= last ? k1 : z;
    }
  };
  auto load_v = [&](int t0) {
#pragma unroll
    for (int u = 0; u < PU; ++u) {
      const int i = tid + NT * u;
      if (UNITS % NT != 0 && i >= UNITS) break;
      const int r = i / (HD / 8), c4 = (i % (HD / 8)) * 4;
      const int p = t0 + r, pc = p <= last ? p : last;
      const size_t off = (size_t)pc * kvd + (size_t)kvh * HD + c4;
      const v4f v0 = *reinterpret_cast<const v4f*>(a.v + off);
      const v4f v1 = *reinterpret_cast<const v4f*>(a.v + off + HD / 2);
      const v4f z = v4f{0.f, 0.f, 0.f, 0.f};
      vreg[2 * u] = p <= last ? v0 : z;
      vreg[2 * u + 1] = p <= last ? v1 : z;
    }
  };
  // K row r, head dims d..d+3 (d = c4 or c4 + HD/2, a multiple of 4) go to
  // block r / 16, step d / 32, lane 16 ((d / 8) % 4) + r % 16, elements
  // d % 8 .. + 3: one 8-byte store per term. K takes two bf16 terms, hi and
  // lo = bf16(k - hi) (k - hi is exact): k to ~2^-17 relative.
  auto store_k = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PU; ++u) {
      const int i = tid + NT * u;
      if (UNITS % NT != 0 && i >= UNITS) break;
      const int r = i / (HD / 8), c4 = (i % (HD / 8)) * 4;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int d = c4 + half * (HD / 2);
        __bf16 t[2][4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float k = kreg[2 * u + half][e];
          const __bf16 hi = (__bf16)k;
          t[0][e] = hi;
          t[1][e] = (__bf16)(k - (float)hi);
        }
        uint8_t* dst = ksb[buf] + (size_t)(((r >> 4) * KS + (d >> 5)) * 2) * 1024 +
                       (((d >> 3) & 3) * 16 + (r & 15)) * 16 + (d & 7) * 2;
#pragma unroll
        for (int term = 0; term < 2; ++term) {
          bf16x4 v = {t[term][0], t[term][1], t[term][2], t[term][3]};
          *reinterpret_cast<bf16x4*>(dst + term * 1024) = v;
        }
      }
    }
  };
  // V row r (key) and head dim d go to the bf16 A operand of the P V
  // products: 32-key group q = r / 32, and within it the lane group g and
  // element j that also hold that key's weight in the score layout (key
  // 16 kb + 4 g + i of the group <-> g, j = 4 kb + i); lane 16 g + d % 16 of
  // head-dim tile d / 16. Each value is stored as bf16 hi and lo = v - hi.
  auto store_v = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PU; ++u) {
      const int i = tid + NT * u;
      if (UNITS % NT != 0 && i >= UNITS) break;
      const int r = i / (HD / 8), c4 = (i % (HD / 8)) * 4;
      const int q = r >> 5, rr = r & 31;
      const int gk = (rr >> 2) & 3, j = 4 * (rr >> 4) + (rr & 3);
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = c4 + e + half * (HD / 2);
          const float v = vreg[2 * u + half][e];
          const __bf16 hi = (__bf16)v, lo = (__bf16)(v - (float)hi);
          uint8_t* dst = vsb[buf] + (size_t)((q * DT + (d >> 4)) * 2) * 1024 + (gk * 16 + (d & 15)) * 16 + j * 2;
          *reinterpret_cast<__bf16*>(dst) = hi;
          *reinterpret_cast<__bf16*>(dst + 1024) = lo;
        }
    }
  };
  // S^T of a tile: 4 blocks of 16 keys; K (hi, lo) times Q (hi, lo): the
  // three products down to 2^-16 relative, the small ones first
  auto scores = [&](const uint8_t* kt, v4f (&sc)[4]) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      sc[kb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint8_t* kp = kt + (size_t)((kb * KS + ks) * 2) * 1024 + lane * 16;
        const bf16x8 kh = *reinterpret_cast<const bf16x8*>(kp);
        const bf16x8 kl = *reinterpret_cast<const bf16x8*>(kp + 1024);
        sc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qop[ks][0], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qop[ks][1], sc[kb], 0, 0, 0);
        sc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qop[ks][0], sc[kb], 0, 0, 0);
      }
    }
  };

  load_k(p_lo);
  load_v(p_lo);
  store_k(0);
  store_v(0);
  __syncthreads();

  // tile i in buffer i & 1; the loads of tile i+1 are issued into registers
  // before tile i's products and stored to the other buffer after them (it
  // was last read before the previous barrier). All loads are unconditional
  // (a tile past the range is a zero tile, stored but never read).
#pragma unroll 1
  for (int t0 = p_lo, cur = 0; t0 <= last; t0 += kKT, cur ^= 1) {
    load_k(t0 + kKT);
    load_v(t0 + kKT);
    const uint8_t* vt = vsb[cur];
    // multiplicity base of the tile start: floor(t0 / msl) + 1 (msl >= 64, so
    // the tile crosses at most one multiple of msl)
    const int base0 = t0 / a.msl + 1;
    const int next_mult = base0 * a.msl;  // first p with a larger base
    // multiplicity of the row of key k (block kb, lane key i) for this query
    const float base0f = (float)base0;
    auto mult = [&](int kb, int i) {
      const int p = t0 + 16 * kb + 4 * g + i;
      const float c = p <= last ? base0f + (p >= next_mult ? 1.0f : 0.0f) : 0.0f;
      return c - (causal && p > qp ? 1.0f : 0.0f);
    };
    // Most tiles give every key of the wave the same multiplicity: wholly
    // inside [p_lo, last], not crossing a multiple of msl, and wholly at or
    // below (c = base) or wholly above (c = base - 1, causal) the wave's 16
    // queries. cu is that value (wave-uniform), or -1 for per-key values; a
    // tile with cu == 0 adds nothing to this wave's queries.
    const int kmax = t0 + kKT - 1;
    const int qw0 = b * a.seq + qb * kQB + __builtin_amdgcn_readfirstlane(wave) * 16;
    int cu = -1;
    if (kmax <= last && next_mult > kmax) {
      if (!causal || kmax <= qw0) cu = base0;
      else if (t0 > qw0 + 15) cu = base0 - 1;
    }
    if (cu != 0) {  // wave-uniform
    v4f sc[4];
    scores(ksb[cur], sc);
    float w[16];
    if constexpr (SIG) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float c = cu > 0 ? (float)cu : mult(kb, i);
          w[4 * kb + i] = c > 0.0f ? c / (1.0f + expf(-sc[kb][i] * scale_nat)) : 0.0f;
        }
    } else {
      // base-2 scores with the multiplicity folded into the exponent
      // (c 2^x = 2^(x + log2 c)); masked keys at -inf
      float smax = -INFINITY;
      if (cu > 0) {
        const float lc = __builtin_amdgcn_logf((float)cu);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            w[4 * kb + i] = sc[kb][i] * scale_log2 + lc;
            smax = fmaxf(smax, w[4 * kb + i]);
          }
      } else {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float c = mult(kb, i);
            w[4 * kb + i] = c > 0.0f ? sc[kb][i] * scale_log2 + __builtin_amdgcn_logf(c) : -INFINITY;
            smax = fmaxf(smax, w[4 * kb + i]);
          }
      }
      smax = fmaxf(smax, __shfl_xor(smax, 16, 64));
      smax = fmaxf(smax, __shfl_xor(smax, 32, 64));
      const float nm = fmaxf(m, smax);
      const float nz = nm == -INFINITY ? 0.0f : nm;  // all masked so far: weights 0
      const float corr = __builtin_amdgcn_exp2f(m - nz);  // m = -inf: 0
      float ws = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        w[i] = __builtin_amdgcn_exp2f(w[i] - nz);
        ws += w[i];
      }
      ws += __shfl_xor(ws, 16, 64);
      ws += __shfl_xor(ws, 32, 64);
      l = l * corr + ws;
#pragma unroll
      for (int d = 0; d < DT; ++d) o[d] *= corr;
      m = nm;
    }
    // O^T += V^T P^T on the bf16 matrix cores, 32 keys per product, each
    // operand split into bf16 hi + lo: hi*hi + hi*lo + lo*hi (the dropped
    // lo*lo term and the split leave ~2^-16 relative error per product).
    // Lane (query c16, group g) passes the weights it already holds: element
    // j of group g is key 16 (2q + j / 4) + 4g + j % 4 of the tile.
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      bf16x8 ph, pl;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float wv = w[4 * (2 * q + (j >> 2)) + (j & 3)];
        const __bf16 h = (__bf16)wv;
        ph[j] = h;
        pl[j] = (__bf16)(wv - (float)h);
      }
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const uint8_t* vb = vt + (size_t)((q * DT + d) * 2) * 1024 + lane * 16;
        const bf16x8 vh = *reinterpret_cast<const bf16x8*>(vb);
        const bf16x8 vl = *reinterpret_cast<const bf16x8*>(vb + 1024);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph, o[d], 0, 0, 0);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl, o[d], 0, 0, 0);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph, o[d], 0, 0, 0);
      }
    }
    }
    store_k(cur ^ 1);
    store_v(cur ^ 1);
    __syncthreads();
  }
  if (!q_ok) return;
  // o[d]: lane holds query c16, head dims d*16 + 4g + i
  const float inv = SIG ? 1.0f : (l > 0.0f ? 1.0f / l : 0.0f);
  float* out = a.out + (size_t)qp * qd + (size_t)h * HD;
  // with a.split (seq % 16 == 0: the wave's 16 queries are rows 16 rb ..
  // 16 rb + 15, all valid), the outputs are also staged in LDS, which the
  // K/V tiles no longer use after the loop's last barrier: 64 HD bytes per
  // wave, waves 0-7 in ksb and 8-15 in vsb
  float* stg = reinterpret_cast<float*>(wave < 8 ? &ksb[0][0] + wave * 64 * HD
                                                 : &vsb[0][0] + (wave - 8) * 64 * HD);
#pragma unroll
  for (int d = 0; d < DT; ++d) {
    const float4 v = make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
    *reinterpret_cast<float4*>(out + d * 16 + 4 * g) = v;
    if (a.split) *reinterpret_cast<float4*>(stg + c16 * HD + d * 16 + 4 * g) = v;
  }
  if (a.split && lane < 16 * (HD / 32)) {  // (the LDS operations of a wave run in order)
    // the head's 32-element blocks of row i16: operand lane i16 + 16 gq of
    // the O projection's 16 x 128 slice (rb, kc), gq = (h HD % 128) / 32 + gg,
    // split exactly as k_split splits the stored outputs
    const int i16 = lane & 15, gg = lane >> 4;
    float v[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = *reinterpret_cast<const float4*>(stg + i16 * HD + 32 * gg + 4 * q);
      v[4 * q] = t.x, v[4 * q + 1] = t.y, v[4 * q + 2] = t.z, v[4 * q + 3] = t.w;
    }
    const int col0 = h * HD, kc = col0 / 128, KC = qd / 128;
    const int rb = (qp - c16) / 16;
    const int vlane = i16 + 16 * ((col0 % 128) / 32 + gg);
    const GlobalU8 chunk = (GlobalU8)(a.split + (size_t)(rb * KC + kc) * kTerms * kFrag6Bytes);
    const GlobalU8 scales = (GlobalU8)(a.split + (size_t)kTerms * a.split_mpad * qd +
                                       (size_t)(rb * KC + kc) * kChunkScaleBytes);
    split_terms6<1, kTerms, false>(v, chunk, scales, vlane);
  }
}

}  // namespace

Status build_rope_table(double* tab, int tokens, int hd, double theta, hipStream_t st) {
  const int n = tokens * (hd / 2);
  if (n <= 0) return Status::ok();
  k_rope_table<<<(n + 255) / 256, 256, 0, st>>>(tab, tokens, hd, theta);
  return hip_status(hipGetLastError(), "rope table launch");
}

// the matrix-core kernel's conditions (launch_attention)
static bool attention_fast(const AttnArgs& a) {
  return (a.mask == 1 || a.mask == 2) && !a.alibi && a.msl >= kKT && a.msl >= a.seq &&
         (a.hd == 32 || a.hd == 64 || a.hd == 128) && a.seq > 0 && a.tokens % a.seq == 0;
}

bool attention_writes_split(const AttnArgs& a) {
  return attention_fast(a) && (a.heads * a.hd) % 256 == 0 && a.seq % 16 == 0;
}

Status launch_attention(const AttnArgs& a, hipStream_t st) {
  if (a.hd > 64 * kMaxHdPerLane || a.hd % 4 != 0)
    return Status::err(kUnsupported, "attention: head_dim must be a multiple of 4 and <= 256");
  // the tile multiplicity update assumes at most one multiple of msl per
  // 64-key tile, hence msl >= 64
  const bool fast = attention_fast(a);
  if (a.split && (!attention_writes_split(a) || a.split_mpad < a.tokens || a.split_mpad % 16 != 0))
    return Status::err(kInvalid, "attention: the output split needs the matrix-core path, "
                                 "heads * hd % 256 == 0 and seq % 16 == 0");
  if (a.rope) {
    k_rope<<<a.tokens, 256, 0, st>>>(const_cast<float*>(a.q), const_cast<float*>(a.k), a.tokens,
                                     a.heads, a.kv_heads, a.hd, a.rope_theta, a.rope_tab);
    WV_HIP(hipGetLastError());
  }
  if (fast) {
    const int waves = attn_waves(a.hd <= 64 ? a.hd : 128), qb_rows = 16 * waves;
    const int qblocks = (a.seq + qb_rows - 1) / qb_rows;
    dim3 grid((unsigned)(a.tokens / a.seq * qblocks), (unsigned)a.heads);
    const dim3 blk(64 * waves);
    switch (a.hd) {
    case 32:
      if (a.sigmoid) k_attn_mfma<32, true><<<grid, blk, 0, st>>>(a, qblocks);
      else k_attn_mfma<32, false><<<grid, blk, 0, st>>>(a, qblocks);
      break;
    case 64:
      if (a.sigmoid) k_attn_mfma<64, true><<<grid, blk, 0, st>>>(a, qblocks);
      else k_attn_mfma<64, false><<<grid, blk, 0, st>>>(a, qblocks);
      break;
    default:
      if (a.sigmoid) k_attn_mfma<128, true><<<grid, blk, 0, st>>>(a, qblocks);
      else k_attn_mfma<128, false><<<grid, blk, 0, st>>>(a, qblocks);
      break;
    }
    return hip_status(hipGetLastError(), "attention launch");
  }
  dim3 grid(a.tokens, a.heads);
  k_attention<<<grid, 64, 0, st>>>(a);
  return hip_status(hipGetLastError(), "attention launch");
}

}  // namespace wv
