// Measurement kernels (no reference counterpart):
// - a plain streaming read of a device buffer: the lower bound on the time of
//   any kernel that reads the same bytes once (it does nothing else), the
//   read floor the batch-1 GEMV is compared with. Each workgroup of 256 lanes
//   reads one contiguous run of 256 x 16 x kUnroll bytes with 16-byte
//   non-temporal loads (all kUnroll loads of a lane in flight before any is
//   used, as the GEMV issues its weight rows), XOR-folds them and writes one
//   word, so the loads cannot be removed;
// - a fetch-rate read: every workgroup reads 64 KiB regions of a buffer of
//   chosen size over and over (a region of a few MiB stays in L2, one of GiB
//   streams from HBM), which gives the bytes per cycle one CU can take;
// - the issue rate of the scaled matrix-core instruction for a pair of
//   operand formats and shapes: back-to-back independent MFMAs, 4 waves of a
//   workgroup, no memory traffic in the loop.
#include "common.h"
#include "kernels.h"

namespace wv {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr size_t kRun = (size_t)kThreads * 16 * kUnroll;  // bytes per workgroup

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void k_read(const uint8_t* __restrict__ buf, size_t bytes,
                                                   uint32_t* __restrict__ out) {
  const size_t base = (size_t)blockIdx.x * kRun + (size_t)threadIdx.x * 16;
  u32x4 v[kUnroll];
#pragma unroll
  for (int i = 0; i < kUnroll; ++i) {
    const size_t off = base + (size_t)i * kThreads * 16;
    v[i] = off + 16 <= bytes ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(buf + off))
                             : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < kUnroll; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off, 64);
  __shared__ uint32_t part[kThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// Reads `iters` regions of 64 KiB: region (blockIdx * 7 + it) % nreg, four
// 16-byte loads per lane in flight.
__global__ __launch_bounds__(kThreads) void k_fetch(const uint8_t* __restrict__ buf, int nreg,
                                                    int iters, uint32_t* __restrict__ out) {
  constexpr int kBatch = kThreads * 16 * kUnroll;  // bytes per batch of loads
  uint32_t x = 0;
  for (int it = 0; it < iters; ++it) {
    const size_t reg = (size_t)((blockIdx.x * 7u + (unsigned)it) % (unsigned)nreg) * 65536u;
    for (int b = 0; b < 65536 / kBatch; ++b) {
      u32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        v[u] = *reinterpret_cast<const u32x4*>(buf + reg + (size_t)b * kBatch + (size_t)u * kThreads * 16 +
                                               threadIdx.x * 16);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
  }
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off, 64);
  __shared__ uint32_t part[kThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// kAcc independent accumulators per wave, `iters` rounds of one MFMA on each.
// Operand bytes avoid the E4M3 / E5M2 NaN and infinity encodings (exponent
// field below its maximum); every format decodes them to finite values.
constexpr int kAcc = 8;
template <int FA, int FB, int SHAPE>
__global__ __launch_bounds__(kThreads) void k_mfma_rate(float* __restrict__ out, int iters) {
  const uint32_t l = threadIdx.x & 63;
  v8i a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t p = (l * 0x01010101u + (uint32_t)i * 0x03050709u) & 0x37373737u;
    a[i] = (int)p;
    b[i] = (int)(p ^ 0x11111111u);
  }
  float s = 0.0f;
  if constexpr (SHAPE == 16) {
    v4f acc[kAcc];
#pragma unroll
    for (int j = 0; j < kAcc; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < kAcc; ++j)
        acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[j], FA, FB, 0, 127, 0, 127);
    }
#pragma unroll
    for (int j = 0; j < kAcc; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  } else {
    v16f acc[kAcc / 2];
#pragma unroll
    for (int j = 0; j < kAcc / 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[j][i] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < kAcc / 2; ++j)
        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[j], FA, FB, 0, 127, 0, 127);
    }
#pragma unroll
    for (int j = 0; j < kAcc / 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) s += acc[j][i];
  }
  out[(size_t)blockIdx.x * kThreads + threadIdx.x] = s;
}

// One lane writes the device's constant-rate wall clock (wall_clock64) to
// *out: placed before and after a run of kernels in one stream or graph, two
// stamps time that run on the device.
__global__ __launch_bounds__(64) void k_clock_stamp(unsigned long long* __restrict__ out) {
  if (threadIdx.x == 0) *out = wall_clock64();
}

}  // namespace

Status launch_clock_stamp(uint64_t* out, hipStream_t st) {
  if (!out) return Status::err(kInvalid, "clock stamp: null output");
  k_clock_stamp<<<1, 64, 0, st>>>(reinterpret_cast<unsigned long long*>(out));
  return hip_status(hipGetLastError(), "clock stamp");
}

size_t read_probe_words(size_t bytes) { return (bytes + kRun - 1) / kRun; }

Status launch_fetch_probe(const uint8_t* buf, size_t region_bytes, int iters, int workgroups,
                          uint32_t* out, hipStream_t st) {
  if (!buf || !out || region_bytes == 0 || region_bytes % 65536 != 0 ||
      region_bytes / 65536 > 0x7FFFFFFFu || iters <= 0 || workgroups <= 0)
    return Status::err(kInvalid, "fetch probe: region a positive multiple of 64 KiB, iters and "
                                 "workgroups positive");
  k_fetch<<<(unsigned)workgroups, kThreads, 0, st>>>(buf, (int)(region_bytes / 65536), iters, out);
  return hip_status(hipGetLastError(), "fetch probe");
}

// Operand format pairs the issue-rate probe is built for (A, B): E4M3 x E4M3,
// FP6 x E4M3 (the three-term products on FP8 weights), FP6 x E5M2, FP6 x FP4
// (on FP4 weights), FP4 x FP4; 16x16x128 and 32x32x64.
template <int FA, int FB>
static Status mfma_rate_t(int shape, int iters, int workgroups, float* out, hipStream_t st) {
  if (shape == 16) k_mfma_rate<FA, FB, 16><<<(unsigned)workgroups, kThreads, 0, st>>>(out, iters);
  else k_mfma_rate<FA, FB, 32><<<(unsigned)workgroups, kThreads, 0, st>>>(out, iters);
  return hip_status(hipGetLastError(), "mfma probe");
}

Status launch_mfma_probe(int fmt_a, int fmt_b, int shape, int iters, int workgroups, float* out,
                         hipStream_t st) {
  if (!out || iters <= 0 || workgroups <= 0 || (shape != 16 && shape != 32))
    return Status::err(kInvalid, "mfma probe: shape 16 or 32, iters and workgroups positive");
  const int pair = fmt_a * 8 + fmt_b;
  switch (pair) {
  case 0 * 8 + 0: return mfma_rate_t<0, 0>(shape, iters, workgroups, out, st);
  case 2 * 8 + 0: return mfma_rate_t<2, 0>(shape, iters, workgroups, out, st);
  case 2 * 8 + 1: return mfma_rate_t<2, 1>(shape, iters, workgroups, out, st);
  case 2 * 8 + 4: return mfma_rate_t<2, 4>(shape, iters, workgroups, out, st);
  case 4 * 8 + 4: return mfma_rate_t<4, 4>(shape, iters, workgroups, out, st);
  }
  return Status::err(kUnsupported, "mfma probe: format pair not built (E4M3xE4M3, FP6xE4M3, "
                                   "FP6xE5M2, FP6xFP4, FP4xFP4)");
}

Status launch_read_probe(const uint8_t* buf, size_t bytes, uint32_t* out, hipStream_t st) {
  if (!buf || !out || bytes == 0 || bytes % 16 != 0)
    return Status::err(kInvalid, "read probe: bytes must be a positive multiple of 16");
  k_read<<<(unsigned)read_probe_words(bytes), kThreads, 0, st>>>(buf, bytes, out);
  return hip_status(hipGetLastError(), "read probe");
}

}  // namespace wv
