// A plain streaming read of a device buffer: the lower bound on the time of
// any kernel that reads the same bytes once (it does nothing else). Used to
// measure the read floor the batch-1 GEMV is compared with.
//
// Each workgroup of 256 lanes reads one contiguous run of 256 x 16 x kUnroll
// bytes with 16-byte non-temporal loads (all kUnroll loads of a lane in
// flight before any is used, as the GEMV issues its weight rows), XOR-folds
// them and writes one word, so the loads cannot be removed.
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

Status launch_read_probe(const uint8_t* buf, size_t bytes, uint32_t* out, hipStream_t st) {
  if (!buf || !out || bytes == 0 || bytes % 16 != 0)
    return Status::err(kInvalid, "read probe: bytes must be a positive multiple of 16");
  k_read<<<(unsigned)read_probe_words(bytes), kThreads, 0, st>>>(buf, bytes, out);
  return hip_status(hipGetLastError(), "read probe");
}

}  // namespace wv
