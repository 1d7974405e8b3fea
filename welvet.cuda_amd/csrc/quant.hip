// Mount-time quantization on the device: scale selection, bit-exact encode
// into the derived device layout and into the reference FormatNone payload
// (src/weights/native_codec.cpp:193-211), and the exhaustive codec sweep.
#include "codec.h"
#include "common.h"
#include "kernels.h"
#include "runtime.h"

namespace wv {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(v, off, 64);
    v = (o > v) ? o : v;
  }
  return v;
}

// amax of every row, with the reference's NaN-skipping '>' scan
// (native_codec.cpp:20-27): a NaN never replaces the running maximum.
__global__ __launch_bounds__(kThreads) void k_amax_rows(const float* __restrict__ W, int cols,
                                                        float* __restrict__ amax) {
  __shared__ float part[kThreads / 64];
  const int r = blockIdx.x;
  const float* wr = W + (size_t)r * cols;
  float m = 0.0f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float a = fabsf(wr[c]);
    m = (a > m) ? a : m;
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = part[0];
    for (int i = 1; i < kThreads / 64; ++i) t = (part[i] > t) ? part[i] : t;
    amax[r] = t;
  }
}

// Row scales for every padded row. TENSOR reduces the row maxima first.
__global__ __launch_bounds__(kThreads) void k_row_scales(const float* __restrict__ amax_row,
                                                         int rows, int rpad, int scheme,
                                                         float maxrep, float* __restrict__ scale) {
  __shared__ float part[kThreads / 64];
  __shared__ float tensor_s;
  if (scheme == kSchemeTensor) {
    float m = 0.0f;
    for (int r = threadIdx.x; r < rows; r += kThreads) m = (amax_row[r] > m) ? amax_row[r] : m;
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = part[0];
      for (int i = 1; i < kThreads / 64; ++i) t = (part[i] > t) ? part[i] : t;
      tensor_s = scale_for(t, maxrep);
    }
    __syncthreads();
  }
  for (int r = threadIdx.x; r < rpad; r += kThreads) {
    float s = 1.0f;
    if (scheme == kSchemeTensor) s = tensor_s;
    else if (scheme == kSchemeRow && r < rows) s = scale_for(amax_row[r], maxrep);
    scale[r] = s;
  }
}

// E8M0 byte per (row, 32-column block) of the padded layout. Lane per 4
// consecutive columns (16-byte loads when cols % 4 == 0, so a wave reads
// 1 KiB contiguous), the block's 8 lanes combine their maxima with xor
// shuffles. The max keeps the larger value and never takes a NaN
// ((a > m) ? a : m from m = 0), so the combining order does not change it.
__global__ __launch_bounds__(kThreads) void k_block_exp(const float* __restrict__ W, int rows,
                                                        int cols, int rpad, int nblk, float maxrep,
                                                        uint8_t* __restrict__ blk) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t nq = (int64_t)rpad * nblk * 8;  // a multiple of 8: groups stay whole
  const bool live = t < nq;
  const int64_t tq = live ? t : nq - 1;
  const int r = (int)(tq / ((int64_t)nblk * 8)), q = (int)(tq % ((int64_t)nblk * 8));
  const int c0 = q * 4;
  float m = 0.0f;
  if (live && r < rows && c0 < cols) {
    const float* w = W + (size_t)r * cols + c0;
    if ((cols & 3) == 0) {
      const float4 v = *reinterpret_cast<const float4*>(w);
      const float a[4] = {fabsf(v.x), fabsf(v.y), fabsf(v.z), fabsf(v.w)};
#pragma unroll
      for (int i = 0; i < 4; ++i) m = (a[i] > m) ? a[i] : m;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c0 + i < cols) {
          const float a = fabsf(w[i]);
          m = (a > m) ? a : m;
        }
    }
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    const float v = __shfl_xor(m, o, 64);
    m = (v > m) ? v : m;
  }
  if (live && (q & 7) == 0) {
    const int e = r < rows && c0 < cols ? e8m0_exponent(m, maxrep) : 0;
    blk[(size_t)r * nblk + q / 8] = (uint8_t)(e + 127);
  }
}

// Value handed to the element encoder for W[r][c] under the scheme.
__device__ __forceinline__ float scaled_input(const float* W, int cols, int r, int c, int scheme,
                                              const float* scale, const uint8_t* blk, int nblk) {
  const float w = W[(size_t)r * cols + c];
  if (scheme == kSchemeTensor || scheme == kSchemeRow) return w / scale[r];
  if (scheme == kSchemeBlock32) return w * pow2f(127 - (int)blk[(size_t)r * nblk + c / 32]);
  return w;
}

// Padded canonical layout, FP8: one thread per 4 consecutive columns.
__global__ __launch_bounds__(kThreads) void k_encode_fp8(const float* __restrict__ W, int rows,
                                                         int cols, int dtype, int scheme,
                                                         const float* __restrict__ scale,
                                                         const uint8_t* __restrict__ blk, int nblk,
                                                         int rpad, int pitch,
                                                         uint8_t* __restrict__ codes) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int quads = pitch / 4;
  if (t >= (int64_t)rpad * quads) return;
  const int r = (int)(t / quads), c0 = (int)(t % quads) * 4;
  uint32_t word = 0;
  if (r < rows) {
    for (int i = 0; i < 4; ++i) {
      const int c = c0 + i;
      if (c < cols) {
        const uint8_t q = encode(dtype, scaled_input(W, cols, r, c, scheme, scale, blk, nblk));
        word |= (uint32_t)canonical(dtype, q) << (8 * i);
      }
    }
  }
  reinterpret_cast<uint32_t*>(codes)[t] = word;
}

// Padded layout, FP4: one thread per byte (columns 2j, 2j+1).
__global__ __launch_bounds__(kThreads) void k_encode_fp4(const float* __restrict__ W, int rows,
                                                         int cols, int scheme,
                                                         const float* __restrict__ scale,
                                                         const uint8_t* __restrict__ blk, int nblk,
                                                         int rpad, int pitch,
                                                         uint8_t* __restrict__ codes) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= (int64_t)rpad * pitch) return;
  const int r = (int)(t / pitch), c0 = (int)(t % pitch) * 2;
  uint8_t byte = 0;
  if (r < rows) {
    if (c0 < cols) byte = encode_fp4(scaled_input(W, cols, r, c0, scheme, scale, blk, nblk)) & 15u;
    if (c0 + 1 < cols)
      byte |= (uint8_t)((encode_fp4(scaled_input(W, cols, r, c0 + 1, scheme, scale, blk, nblk)) & 15u) << 4);
  }
  codes[t] = byte;
}

// Reference FormatNone payload: FP8 one byte per flattened element; FP4 byte i
// holds flattened elements 2i (low nibble) and 2i+1 (high nibble).
__global__ __launch_bounds__(kThreads) void k_encode_raw(const float* __restrict__ W, int rows,
                                                         int cols, int dtype, int scheme,
                                                         const float* __restrict__ scale,
                                                         const uint8_t* __restrict__ blk, int nblk,
                                                         uint8_t* __restrict__ raw) {
  const int64_t n = (int64_t)rows * cols;
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (dtype != kFP4) {
    if (t >= n) return;
    const int r = (int)(t / cols), c = (int)(t % cols);
    raw[t] = encode(dtype, scaled_input(W, cols, r, c, scheme, scale, blk, nblk));
    return;
  }
  if (t >= (n + 1) / 2) return;
  uint8_t byte = 0;
  for (int h = 0; h < 2; ++h) {
    const int64_t e = 2 * t + h;
    if (e < n) {
      const int r = (int)(e / cols), c = (int)(e % cols);
      byte |= (uint8_t)((encode_fp4(scaled_input(W, cols, r, c, scheme, scale, blk, nblk)) & 15u) << (4 * h));
    }
  }
  raw[t] = byte;
}

// Reference payload -> padded canonical layout (mount from stored codes).
__global__ __launch_bounds__(kThreads) void k_relayout(const uint8_t* __restrict__ raw, int rows,
                                                       int cols, int dtype, int rpad, int pitch,
                                                       uint8_t* __restrict__ codes) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= (int64_t)rpad * pitch) return;
  const int r = (int)(t / pitch), j = (int)(t % pitch);
  uint8_t out = 0;
  if (r < rows) {
    if (dtype != kFP4) {
      if (j < cols) out = canonical(dtype, raw[(size_t)r * cols + j]);
    } else {
      for (int h = 0; h < 2; ++h) {
        const int c = 2 * j + h;
        if (c < cols) {
          const int64_t e = (int64_t)r * cols + c;
          const uint8_t b = raw[e >> 1];
          const uint8_t q = (e & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15u);
          out |= (uint8_t)(q << (4 * h));
        }
      }
    }
  }
  codes[t] = out;
}

__global__ void k_fill_u8(uint8_t* p, int64_t n, uint8_t v) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t < n) p[t] = v;
}

__global__ void k_fill_f32(float* p, int64_t n, float v) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t < n) p[t] = v;
}

__global__ void k_zero_i64(unsigned long long* p, int64_t n) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t < n) p[t] = 0ull;
}

// Encoder over every f32 bit pattern of chunks [first, first + n): each
// 256-thread block covers 4096 patterns of one 2^20-pattern chunk and adds
// (sum code, sum code * low20) into out[2 * chunk_local].
__global__ __launch_bounds__(kThreads) void k_sweep(int dtype, uint32_t first_chunk,
                                                    unsigned long long* __restrict__ out) {
  const uint32_t local_chunk = blockIdx.x >> 8;
  const uint32_t chunk = first_chunk + local_chunk;
  const uint32_t base = (chunk << 20) | ((blockIdx.x & 255u) << 12);
  unsigned long long s1 = 0, s2 = 0;
  for (int i = 0; i < 16; ++i) {
    const uint32_t low = ((blockIdx.x & 255u) << 12) | (uint32_t)(i * kThreads + threadIdx.x);
    const uint32_t u = (base & 0xFFF00000u) | low;
    const unsigned long long code = encode(dtype, float_of(u));
    s1 += code;
    s2 += code * low;
  }
  for (int off = 32; off > 0; off >>= 1) {
    s1 += __shfl_xor(s1, off, 64);
    s2 += __shfl_xor(s2, off, 64);
  }
  __shared__ unsigned long long p1[4], p2[4];
  if ((threadIdx.x & 63) == 0) p1[threadIdx.x >> 6] = s1, p2[threadIdx.x >> 6] = s2;
  __syncthreads();
  if (threadIdx.x == 0) {
    atomicAdd(&out[2 * local_chunk], p1[0] + p1[1] + p1[2] + p1[3]);
    atomicAdd(&out[2 * local_chunk + 1], p2[0] + p2[1] + p2[2] + p2[3]);
  }
}

inline unsigned grid_for(int64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

// Lane-order copy of the E8M0 block exponents (DeviceWeights::blk_frag): one
// thread per output byte; chunks past the K padding get 127 (2^0).
__global__ __launch_bounds__(kThreads) void k_blk_frag(const uint8_t* __restrict__ blk, int rpad,
                                                       int nblk, int chunks, int groups,
                                                       uint8_t* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= (int64_t)(rpad / 16) * groups * 256) return;
  const int j = (int)(t & 3), l = (int)((t >> 2) & 63);
  const int64_t rest = t >> 8;
  const int q = (int)(rest % groups), rb = (int)(rest / groups);
  const int c = 4 * q + j;
  out[t] = c < chunks ? blk[(size_t)(rb * 16 + (l & 15)) * nblk + c * 4 + (l >> 4)] : (uint8_t)127;
}

Status build_blk_frag(DeviceWeights* dw, hipStream_t st) {
  const int chunks = dw->kpad / 128, groups = (chunks + 3) / 4;
  const int64_t n = (int64_t)(dw->rpad / 16) * groups * 256;
  WV_TRY(dw->blk_frag.alloc((size_t)n));
  k_blk_frag<<<grid_for(n), kThreads, 0, st>>>(dw->blk.as<const uint8_t>(), dw->rpad, dw->nblk,
                                               chunks, groups, dw->blk_frag.as<uint8_t>());
  return hip_status(hipGetLastError(), "blk_frag");
}

// Operand-order copy of the codes (DeviceWeights::codes_frag): one thread
// per 16-byte lane slot t = ((rb * chunks + c) * halves + h) * 64 + l.
__global__ __launch_bounds__(kThreads) void k_codes_frag(const uint8_t* __restrict__ codes,
                                                         int pitch, int chunks, int halves,
                                                         int64_t n, uint8_t* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= n) return;
  const int l = (int)(t & 63);
  int64_t rest = t >> 6;
  const int h = (int)(rest % halves);
  rest /= halves;
  const int c = (int)(rest % chunks);
  const int64_t rb = rest / chunks;
  const int wb = 64 * halves;  // code bytes per row per chunk
  const uint4 v = *reinterpret_cast<const uint4*>(
      codes + (size_t)(rb * 16 + (l & 15)) * pitch + (size_t)c * wb + 64 * h + 16 * (l >> 4));
  *reinterpret_cast<uint4*>(out + (size_t)t * 16) = v;
}

}  // namespace

Status build_codes_frag(DeviceWeights* dw, hipStream_t st) {
  if (!dw->codes.p) return Status::err(kInvalid, "codes_frag: no codes");
  const int chunks = dw->kpad / 128, halves = dw->dtype == kFP4 ? 1 : 2;
  const int64_t n = (int64_t)(dw->rpad / 16) * chunks * halves * 64;
  WV_TRY(dw->codes_frag.alloc((size_t)n * 16));
  k_codes_frag<<<grid_for(n), kThreads, 0, st>>>(dw->codes.as<const uint8_t>(), dw->pitch, chunks,
                                                 halves, n, dw->codes_frag.as<uint8_t>());
  return hip_status(hipGetLastError(), "codes_frag");
}

Status quantize_to_device(const float* dW, int dtype, int scheme, int rows, int cols,
                          DeviceWeights* dw, uint8_t* d_raw, hipStream_t st) {
  dw->dtype = dtype;
  dw->scheme = scheme;
  dw->rows = rows;
  dw->cols = cols;
  dw->rpad = (int)round_up(rows, kRowPad);
  dw->kpad = (int)round_up(cols, kColPad);
  dw->pitch = dtype == kFP4 ? dw->kpad / 2 : dw->kpad;
  dw->nblk = dw->kpad / 32;
  WV_TRY(dw->codes.alloc((size_t)dw->rpad * dw->pitch));
  WV_TRY(dw->row_scale.alloc((size_t)dw->rpad * sizeof(float)));
  const float maxrep = max_representable(dtype);
  DevBuf amax;
  WV_TRY(amax.alloc((size_t)rows * sizeof(float)));
  if (scheme == kSchemeTensor || scheme == kSchemeRow) {
    k_amax_rows<<<rows, kThreads, 0, st>>>(dW, cols, amax.as<float>());
    WV_HIP(hipGetLastError());
  }
  k_row_scales<<<1, kThreads, 0, st>>>(amax.as<float>(), rows, dw->rpad, scheme, maxrep,
                                       dw->row_scale.as<float>());
  WV_HIP(hipGetLastError());
  uint8_t* blk = nullptr;
  if (scheme == kSchemeBlock32) {
    WV_TRY(dw->blk.alloc((size_t)dw->rpad * dw->nblk));
    blk = dw->blk.as<uint8_t>();
    k_block_exp<<<grid_for((int64_t)dw->rpad * dw->nblk * 8), kThreads, 0, st>>>(
        dW, rows, cols, dw->rpad, dw->nblk, maxrep, blk);
    WV_HIP(hipGetLastError());
    WV_TRY(build_blk_frag(dw, st));
  }
  const float* sc = dw->row_scale.as<float>();
  if (dtype == kFP4) {
    k_encode_fp4<<<grid_for((int64_t)dw->rpad * dw->pitch), kThreads, 0, st>>>(
        dW, rows, cols, scheme, sc, blk, dw->nblk, dw->rpad, dw->pitch, dw->codes.as<uint8_t>());
  } else {
    k_encode_fp8<<<grid_for((int64_t)dw->rpad * (dw->pitch / 4)), kThreads, 0, st>>>(
        dW, rows, cols, dtype, scheme, sc, blk, dw->nblk, dw->rpad, dw->pitch,
        dw->codes.as<uint8_t>());
  }
  WV_HIP(hipGetLastError());
  if (d_raw) {
    const int64_t n = (int64_t)rows * cols;
    const int64_t nbytes = dtype == kFP4 ? (n + 1) / 2 : n;
    k_encode_raw<<<grid_for(nbytes), kThreads, 0, st>>>(dW, rows, cols, dtype, scheme, sc, blk,
                                                       dw->nblk, d_raw);
    WV_HIP(hipGetLastError());
  }
  WV_TRY(find_nonfinite_rows(dw, st));
  // amax is freed when this function returns; the kernels reading it must be done.
  WV_HIP(hipStreamSynchronize(st));
  return Status::ok();
}

Status relayout_to_device(const uint8_t* d_raw, int dtype, int scheme, int rows, int cols,
                          const float* d_row_scale, const uint8_t* d_blk_rows,
                          DeviceWeights* dw, hipStream_t st) {
  dw->dtype = dtype;
  dw->scheme = scheme;
  dw->rows = rows;
  dw->cols = cols;
  dw->rpad = (int)round_up(rows, kRowPad);
  dw->kpad = (int)round_up(cols, kColPad);
  dw->pitch = dtype == kFP4 ? dw->kpad / 2 : dw->kpad;
  dw->nblk = dw->kpad / 32;
  WV_TRY(dw->codes.alloc((size_t)dw->rpad * dw->pitch));
  WV_TRY(dw->row_scale.alloc((size_t)dw->rpad * sizeof(float)));
  k_relayout<<<grid_for((int64_t)dw->rpad * dw->pitch), kThreads, 0, st>>>(
      d_raw, rows, cols, dtype, dw->rpad, dw->pitch, dw->codes.as<uint8_t>());
  WV_HIP(hipGetLastError());
  k_fill_f32<<<grid_for(dw->rpad), kThreads, 0, st>>>(dw->row_scale.as<float>(), dw->rpad, 1.0f);
  WV_HIP(hipGetLastError());
  if (d_row_scale) {
    WV_HIP(hipMemcpyAsync(dw->row_scale.as<float>(), d_row_scale, (size_t)rows * sizeof(float),
                          hipMemcpyDeviceToDevice, st));
  }
  if (scheme == kSchemeBlock32) {
    WV_TRY(dw->blk.alloc((size_t)dw->rpad * dw->nblk));
    k_fill_u8<<<grid_for((int64_t)dw->rpad * dw->nblk), kThreads, 0, st>>>(
        dw->blk.as<uint8_t>(), (int64_t)dw->rpad * dw->nblk, 127);
    WV_HIP(hipGetLastError());
    const int src_nblk = (cols + 31) / 32;
    if (d_blk_rows) {
      WV_HIP(hipMemcpy2DAsync(dw->blk.as<uint8_t>(), dw->nblk, d_blk_rows, src_nblk, src_nblk, rows,
                              hipMemcpyDeviceToDevice, st));
    }
    WV_TRY(build_blk_frag(dw, st));
  }
  WV_TRY(find_nonfinite_rows(dw, st));
  WV_HIP(hipStreamSynchronize(st));
  return Status::ok();
}

namespace {
__global__ __launch_bounds__(kThreads) void k_decode_store(const uint8_t* __restrict__ bytes,
                                                           int dtype, int64_t e0, int64_t n,
                                                           int cols,
                                                           const float* __restrict__ row_scale,
                                                           const uint8_t* __restrict__ blk, int nb,
                                                           float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t e = e0 + i;
  uint8_t q;
  if (dtype == kFP4) {
    const uint8_t b = bytes[e / 2 - e0 / 2];
    q = (e & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15u);
  } else {
    q = bytes[i];
  }
  const int64_t r = e / cols - e0 / cols;
  const int c = (int)(e % cols);
  const float v = decode(dtype, q);
  if (blk) out[i] = v * pow2f((int)blk[r * nb + c / 32] - 127);
  else out[i] = row_scale ? v * row_scale[r] : v;
}
}  // namespace

Status launch_decode_store(const uint8_t* bytes, int dtype, int64_t e0, int64_t n, int cols,
                           const float* row_scale, const uint8_t* blk, int nb, float* out,
                           hipStream_t st) {
  if (n <= 0) return Status::ok();
  if (!bytes || !out || cols <= 0 || e0 < 0 || (blk && nb != (cols + 31) / 32))
    return Status::err(kInvalid, "decode store: bad args");
  k_decode_store<<<grid_for(n), kThreads, 0, st>>>(bytes, dtype, e0, n, cols, row_scale, blk, nb,
                                                   out);
  return hip_status(hipGetLastError(), "decode store launch");
}

Status codec_sweep(int dtype, uint32_t first_chunk, uint32_t n_chunks, int64_t* host_out,
                   hipStream_t st) {
  DevBuf out;
  WV_TRY(out.alloc((size_t)n_chunks * 2 * sizeof(int64_t)));
  k_zero_i64<<<grid_for((int64_t)n_chunks * 2), kThreads, 0, st>>>(out.as<unsigned long long>(),
                                                                     (int64_t)n_chunks * 2);
  WV_HIP(hipGetLastError());
  // 256 blocks per chunk; launch at most 1024 chunks per grid.
  for (uint32_t c = 0; c < n_chunks; c += 1024) {
    const uint32_t cnt = (n_chunks - c) < 1024 ? (n_chunks - c) : 1024;
    k_sweep<<<cnt * 256, kThreads, 0, st>>>(dtype, first_chunk + c,
                                            out.as<unsigned long long>() + 2 * (size_t)c);
    WV_HIP(hipGetLastError());
  }
  WV_TRY(copy_d2h(host_out, out.p, (size_t)n_chunks * 2 * sizeof(int64_t), st));
  WV_HIP(hipStreamSynchronize(st));
  return Status::ok();
}

}  // namespace wv
