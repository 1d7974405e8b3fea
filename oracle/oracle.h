/*
 * CPU oracle for the quantized-weight Dense path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * numerical contract (openfluke/welvet.cuda 0.79). It is test infrastructure: only the
 * tests, the smoke check and the CPU-baseline leg of the benchmark load it.
 * The product library (welvet.cuda_amd) never links or calls it.
 *
 * Every function cites the reference file:line it restates. Parity status of
 * each function (how it is pinned) is listed beside it.
 */
#ifndef WELVET_ORACLE_H
#define WELVET_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DType ids (include/welvet/dtype.hpp:14-26). */
enum { OR_FP8E4M3 = 4, OR_FP8E5M2 = 5, OR_FP4 = 16 };

/* Quant schemes carried in the ABI's `backend` argument (build-defined
 * extension; the reference only has scheme 0 = FormatNone, scale 1). */
enum { OR_SCHEME_REF = 0, OR_SCHEME_TENSOR = 1, OR_SCHEME_ROW = 2, OR_SCHEME_BLOCK32 = 3 };

/* --- element codecs: src/core/float_codecs.cpp ---------------------------
 * Pinned by: full decode tables and 2^32-input encode digests produced by the
 * compiled reference codecs (tests/golden), plus hand-derived special cases. */
uint8_t or_enc_e4m3(float f);   /* float_codecs.cpp:57-97  */
float or_dec_e4m3(uint8_t b);   /* float_codecs.cpp:99-117 */
uint8_t or_enc_e5m2(float f);   /* float_codecs.cpp:119-158 */
float or_dec_e5m2(uint8_t b);   /* float_codecs.cpp:160-182 */
uint8_t or_enc_fp4(float f);    /* float_codecs.cpp:184-198 */
float or_dec_fp4(uint8_t c);    /* float_codecs.cpp:200 */

uint8_t or_encode(int dtype, float f);
float or_decode(int dtype, uint8_t code);

/* Digest of the encoder over all f32 bit patterns of 2^20-pattern chunks
 * [first, first+count): out[2*c] = sum(code), out[2*c+1] = sum(code * (u & 0xFFFFF)).
 * For FP4 the per-element 4-bit code is used. Threads: nthreads (>=1). */
void or_sweep_digest(int dtype, uint32_t first_chunk, uint32_t n_chunks, int64_t* out, int nthreads);

/* --- FormatNone packing: src/weights/native_codec.cpp:193-211 (pack),
 * :534-549 (weight_at), :726-733 (nibble order) -------------------------
 * Pinned by: WeightStore::make/export_f32 of the compiled reference. */
size_t or_native_bytes(int dtype, int64_t n);
void or_pack(int dtype, const float* w, int64_t n, uint8_t* out);
float or_weight_at(int dtype, const uint8_t* raw, int64_t i);

/* --- scale extension (build-defined, not in the reference) ----------------
 * Scheme rules: maxrep = 240 (E4M3), 57344 (E5M2), 6 (FP4).
 *   TENSOR / ROW: s = amax / maxrep (f32), s == 0 -> 1; q = enc(w / s);
 *                 dequant = f32(dec(q) * s).
 *   BLOCK32:      per row, per 32 consecutive columns: e = least integer in
 *                 [-127, 127] with amax <= maxrep * 2^e (amax == 0 -> e = 0);
 *                 byte = e + 127; q = enc(w * 2^-e); dequant = dec(q) * 2^e.
 *   REF:          s = 1, q = enc(w) (reference FormatNone behaviour).
 * Codes are packed as the reference packs them (flattened row-major).
 * row_scale: rows floats (TENSOR fills every row with the tensor scale; REF
 * and BLOCK32 fill 1). blk_exp: rows * ceil(cols/32) bytes (BLOCK32 only, else
 * may be NULL). Pinned by: closed form (power-of-two exactness, amax
 * boundary cases) in the tests. */
int or_maxrep_ok(int dtype);
float or_maxrep(int dtype);
int or_e8m0_exponent(float amax, float maxrep);
void or_quantize(int dtype, int scheme, int rows, int cols, const float* W, uint8_t* native,
                 float* row_scale, uint8_t* blk_exp);
/* Dequantized weights W_dq[rows*cols] (f32), as the layer parity reference. */
void or_dequant(int dtype, int scheme, int rows, int cols, const uint8_t* native,
                const float* row_scale, const uint8_t* blk_exp, float* W_dq);

/* --- activations: src/core/activate.cpp:7-29 (host f64) --------------------
 * Pinned by: closed forms (Linear/ReLU exact; SiLU/GELU/Tanh/Sigmoid from
 * libm). Device math of the reference is CUDA's: parity unpinned beyond the
 * layer tolerance. */
double or_activate(int act, double x);

/* --- Dense forward: src/cuda/kernels.cu:130-161, :895-906 -------------------
 * y[b,o] = f32(sum_k f64(W[o,k]) * f64(x[b,k])) in serial k order; then, if
 * act != Linear or a bias exists: v = f64(y) (+ bias[o] if o < bias_len, and
 * then pre = f32(v)); post = f32(act(v)); else post = pre.
 * Pinned by: brute force on tiny shapes, fp32-exact cases, the 2x2 identity
 * known answer of scripts/release_smoke.py:55-70. nthreads splits rows. */
void or_dense_forward(int batch, int in, int out, int act, const float* W, const double* bias,
                      int bias_len, const float* x, float* pre, float* post, int nthreads);

/* --- SwiGLU product: src/cuda/kernels.cu:296-304 ----------------------------
 * h = f32(f64(f32(SiLU(f64 g))) * f64(u)). */
void or_swiglu_product(const float* g, const float* u, float* h, int64_t n);

/* --- MHA ModeSelf attention core: src/cuda/kernels.cu:470-631 ---------------
 * Restates the reference's serial f64 loop including its global positions
 * (pos = b*seq + s), kv_len = b*seq + seq and the KV ring row = k_pos % msl.
 * mask: 1 causal, 2 bidirectional, 3 sliding window, 4 prefix LM; pos_kind:
 * 0 RoPE, 1 none, 2 ALiBi, 3 RoPE+ALiBi; softmax_kind 0 standard, 1 sigmoid.
 * Parity: brute force at small sizes; transcendental math unpinned (tolerance). */
void or_mha_attention(const float* q, const float* k, const float* v, float* attn, int batch,
                      int seq, int num_heads, int num_kv, int head_dim, int msl, int mask,
                      int pos_kind, int softmax_kind, int window, int prefix_len, int window_causal,
                      double rope_theta, double scale_override);
/* The same on nthreads threads, heads spread over them (bit-identical: each
 * head's arithmetic is unchanged). */
void or_mha_attention_mt(const float* q, const float* k, const float* v, float* attn, int batch,
                         int seq, int num_heads, int num_kv, int head_dim, int msl, int mask,
                         int pos_kind, int softmax_kind, int window, int prefix_len,
                         int window_causal, double rope_theta, double scale_override,
                         int nthreads);

/* --- Dense backward (NormalBP) and SGD --------------------------------------
 * act'(x) in f64: src/cuda/kernels.cu:48-81 (host twin src/core/activate.cpp:31-63).
 * Pinned by: the compiled reference activate_deriv_f64 (oracle/_ref), and
 * central differences of or_activate. */
double or_act_deriv(int act, double x);
/* kernels.cu:83-127 with W the dequantized f32 matrix [out][in]:
 *   dpre[b][o] = f32(f64(gy[b][o]) * act'(f64 pre[b][o]));
 *   dX[b][i]   = f32(sum over o in order of f64(W[o][i]) * f64(dpre[b][o]));
 *   dW[o][i]   = acc over b in order, acc = f32(f64(acc) + f64(dpre) * f64(x)).
 * Pinned by: W^T dpre and the outer product in numpy f64, exact-integer cases,
 * and central differences of the forward. nthreads splits the columns of dX. */
void or_dense_backward(int batch, int in, int out, int act, const float* W, const float* gy,
                       const float* pre, const float* x, float* dpre, float* dX, float* dW,
                       int nthreads);
/* src/runtime/training.cpp:44-69: loss = sum (p - t)^2 / n in f64 (serial);
 * grad = f32(2/n * (f64 p - f64 t)). Pinned by numpy closed forms. */
double or_mse(int64_t n, const float* pred, const float* target);
void or_mse_grad(int64_t n, const float* pred, const float* target, float* grad);
/* src/weights/native_codec.cpp:1112-1128 (WeightStore::apply_sgd per element):
 * next = f32(f64(w) - lr * f64(dW)); the caller re-encodes next. Pinned by the
 * compiled reference WeightStore::apply_sgd (oracle/_ref). */
void or_sgd(int64_t n, const float* w, const float* dW, double lr, float* next);
/* SwiGLU backward product, src/cuda/kernels.cu:307-320: s = f32(SiLU(f64 g)),
 * ds = f32(SiLU'(f64 g)); d_up = f32(f64(gh) * f64(s)); d_gate =
 * f32(f64(gh) * f64(u) * f64(ds)). Pinned by central differences of the
 * forward product h = SiLU(g) * u and by the compiled reference act'. */
void or_swiglu_bwd_product(const float* g, const float* u, const float* gh, float* d_up,
                           float* d_gate, int64_t n);

/* --- packed block formats (QuantFormat): oracle/formats.c -----------------
 * The reference reserves the enum (include/welvet/weights.hpp:12-15) and lists
 * the formats (README.md:361-383) without implementing them; restated from
 * ggml's published block layouts and rules (ggml-common.h, ggml-quants.c).
 * Pinned by: IEEE half conversions against numpy's float16; closed-form blocks
 * (grid values reproduced exactly, known scales, the nibble and high-bit
 * positions of single set codes); the quantizers' error bounds and
 * idempotence on their own grids. Parity against ggml itself: unpinned (no
 * ggml output is in the image). */
enum { OR_FMT_Q8_0 = 1, OR_FMT_Q4_0 = 2, OR_FMT_Q4_1 = 3, OR_FMT_Q5_0 = 4, OR_FMT_Q5_1 = 5,
       OR_FMT_Q2_K = 6, OR_FMT_Q3_K = 7, OR_FMT_Q4_K = 8, OR_FMT_Q5_K = 9, OR_FMT_Q6_K = 10,
       OR_FMT_IQ4_NL = 16, OR_FMT_IQ4_XS = 17 };
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
/* elements per block (32 or 256) and packed bytes per block; 0 unsupported */
int or_fmt_block_elems(int fmt);
int or_fmt_block_bytes(int fmt);
/* n elements (a multiple of 32) of row-major x -> n / 32 packed blocks.
 * Q8_0, Q4_0, Q4_1, Q5_0, Q5_1 only (the reference quantizers); -1 otherwise. */
int or_fmt_quantize(int fmt, int64_t n, const float* x, uint8_t* out);
/* n elements (a multiple of the block) of packed blocks -> f32; -1 on error. */
int or_fmt_dequant(int fmt, int64_t n, const uint8_t* in, float* out);

/* --- CPU baseline timing (reported beside the GPU) ---------------------------
 * Mount: decode codes to an f64 row-major W (src/layers/dense/dense.cpp:28-39).
 * Execute: or_dense semantics with f64 W, rows split over nthreads.
 * Returns seconds per execute averaged over iters (after warmup). mount_s gets
 * the mount time. */
double or_cpu_dense_bench(int dtype, int scheme, int batch, int in, int out, const uint8_t* native,
                          const float* row_scale, const uint8_t* blk_exp, const float* x,
                          float* y, int nthreads, int warmup, int iters, double* mount_s);

#ifdef __cplusplus
}
#endif
#endif
