// MHA ModeSelf attention core with the reference's indexing
// (src/cuda/kernels.cu:470-631):
//   token t = b*seq + s sits at global position pos = t;
//   queries of batch b see key positions k_pos in [0, b*seq + seq) allowed by
//   the mask (:470-485), scored against the KV ring row k_pos % msl, which by
//   then holds the latest position p <= last = b*seq + seq - 1 with
//   p == k_pos (mod msl): p = last - ((last - k_pos) mod msl);
//   RoPE rotates Q and K at their global position (:487-504), ALiBi uses
//   k_pos (:526-533); softmax or sigmoid over the allowed keys (:603-619).
// The reference loop is serial f64 on one thread; here one wave handles one
// (token, head), keys are scored 64 at a time (one per lane), and the
// softmax is accumulated online in fp32.
#include "common.h"
#include "kernels.h"

namespace wv {
namespace {

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

// Rotates the pair (d, d + hd/2) of every head of Q (num_heads) and K
// (num_kv) rows of token t by angle t / theta^(2d/hd), in f64.
__global__ void k_rope(float* __restrict__ q, float* __restrict__ k, int tokens, int heads,
                       int kv_heads, int hd, double theta) {
  const int t = blockIdx.x;
  const int half = hd / 2;
  const int per_tok = (heads + kv_heads) * half;
  for (int i = threadIdx.x; i < per_tok; i += blockDim.x) {
    const int h = i / half, d = i % half;
    float* row = h < heads ? q + ((size_t)t * heads + h) * hd
                           : k + ((size_t)t * kv_heads + (h - heads)) * hd;
    const double ang = (double)t / pow(theta, (double)(2 * d) / (double)hd);
    const double c = cos(ang), s = sin(ang);
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

}  // namespace

Status launch_attention(const AttnArgs& a, hipStream_t st) {
  if (a.hd > 64 * kMaxHdPerLane || a.hd % 4 != 0)
    return Status::err(kUnsupported, "attention: head_dim must be a multiple of 4 and <= 256");
  if (a.rope) {
    k_rope<<<a.tokens, 256, 0, st>>>(const_cast<float*>(a.q), const_cast<float*>(a.k), a.tokens,
                                     a.heads, a.kv_heads, a.hd, a.rope_theta);
    WV_HIP(hipGetLastError());
  }
  dim3 grid(a.tokens, a.heads);
  k_attention<<<grid, 64, 0, st>>>(a);
  return hip_status(hipGetLastError(), "attention launch");
}

}  // namespace wv
