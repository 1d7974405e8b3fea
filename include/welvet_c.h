/*
 * welvet C ABI — MI355X (gfx950) implementation of the quantized-weight Dense
 * path of openfluke/welvet.cuda 0.79.
 *
 * Every reference entry point keeps its name, signature, argument meaning and
 * error convention (reference include/welvet_c.h). Entry points of the
 * quantized Dense path compute on the GPU; the reference's other entry points
 * are exported with identical signatures and return code 3 ("gap?").
 *
 * Scale schemes. Reference FP8/FP4 weights carry no scale (FormatNone,
 * native_codec.cpp:176). The reference ignores the int32 `backend` argument;
 * here it selects the weight scale scheme:
 *   0  reference behaviour: codes of W, scale 1
 *   1  one fp32 scale per tensor  (s = amax / maxrep)
 *   2  one fp32 scale per output row
 *   3  one E8M0 scale per 32 consecutive inputs of each row
 * with maxrep = 240 (E4M3), 57344 (E5M2), 6 (FP4). Supported dtypes:
 * FP8E4M3 = 4, FP8E5M2 = 5, FP4 = 16 (reference dtype ids); any other dtype
 * returns code 2.
 */
#ifndef WELVET_C_H
#define WELVET_C_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WELVET_API __attribute__((visibility("default")))

/* Reference include/welvet_c.h:26-29. code: 0 ok, 1 invalid, 2 unsupported,
 * 3 gap, 4 internal. */
typedef struct welvet_status {
  int32_t code;
  char message[256];
} welvet_status;

typedef struct welvet_dense_session welvet_dense_session;
typedef struct welvet_model_session welvet_model_session;
/* Reference include/welvet_c.h:46. Freed with welvet_cuda_blob_free. */
typedef struct welvet_cuda_blob {
  uint8_t* data;
  size_t size;
} welvet_cuda_blob;

/* ---- runtime (reference include/welvet_c.h:33-39) ---- */
/* Replaces welvet_c.h:33 (src/interop/c_abi.cpp:53-56): ABI version "0.79". */
WELVET_API const char* welvet_version(void);
/* Replaces welvet_c.h:34 (src/cuda/device.cpp:88-92). Returns
 * "hip:<name>:idx=0:arch=<gfx>:cu=<n>:mem=<MiB>MiB" (thread-local). */
WELVET_API const char* welvet_runtime_identity(void);
/* Replaces welvet_c.h:36 (src/cuda/device.cpp:40-61): device 0; code 2 when
 * no GPU is visible. */
WELVET_API welvet_status welvet_cuda_init(void);
/* Replaces welvet_c.h:37. */
WELVET_API int32_t welvet_cuda_available(void);
/* Replaces welvet_c.h:38-39 (gaps census): counts of this library's ledger. */
WELVET_API int32_t welvet_gaps_count(void);
WELVET_API int32_t welvet_gaps_done(void);

/* ---- Dense (the hot path) ---- */
/* Replaces welvet_c.h:64-67 (c_abi.cpp:95-117): quantize W_init [out*in]
 * (row-major [out][in]) per dtype/backend, y = W x, bias (f64, first bias_len
 * outputs) and activation; pre/post [batch*out]. */
WELVET_API welvet_status welvet_dense_forward_f32(
    int32_t batch, int32_t in, int32_t out, int32_t act, int32_t dtype, int32_t backend,
    const float* W_init, const double* bias, size_t bias_len, const float* x, float* pre,
    float* post);
/* Replaces welvet_c.h:81-86 (c_abi.cpp:72-93, src/layers/dense/session.cpp):
 * mount once (batch fixed), execute many with host buffers. Scheme 0. */
WELVET_API welvet_status welvet_dense_mount(int32_t batch, int32_t in, int32_t out, int32_t act,
                                            int32_t dtype, const float* W_init, const double* bias,
                                            size_t bias_len, welvet_dense_session** sess_out);
WELVET_API welvet_status welvet_dense_execute(welvet_dense_session* sess, const float* x,
                                              float* pre, float* post);
WELVET_API void welvet_dense_release(welvet_dense_session* sess);

/* ---- SwiGLU (welvet_c.h:132-135, c_abi.cpp:543-583, swiglu.cpp:87-136) ----
 * Gate/Up [inter*in], Down [in*inter]; x [batch*seq*in];
 * pre = h [batch*seq*inter]; post [batch*seq*in]. */
WELVET_API welvet_status welvet_swiglu_forward_f32(
    int32_t batch, int32_t seq, int32_t input_dim, int32_t intermediate_dim, int32_t dtype,
    int32_t backend, const float* Gate, const float* Up, const float* Down, const float* x,
    float* pre, float* post);

/* ---- MHA ModeSelf (welvet_c.h:165-169, c_abi.cpp:785-827, mha.cpp:123-183) ----
 * Q [q_dim*d], K/V [kv_dim*d], O [d*q_dim]; x [batch*seq*d];
 * pre = attention [batch*seq*q_dim]; post [batch*seq*d]. */
WELVET_API welvet_status welvet_mha_forward_f32(
    int32_t batch, int32_t seq, int32_t d_model, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t max_seq_len, int32_t mask, int32_t pos, int32_t dtype,
    int32_t backend, const float* Q, const float* K, const float* V, const float* O, const float* x,
    float* pre, float* post);

/* ---- model sessions (welvet_c.h:47-61, src/interop/model_session.cpp) ----
 * WMN1 descriptors with Dense / NestedStack / SwiGLU / MHA children, roots
 * Stack (0) and Grid (2); forward returns the output tensor blob. */
WELVET_API int32_t welvet_model_abi_version(void);
WELVET_API welvet_status welvet_model_mount(const uint8_t* descriptor, size_t size,
                                            welvet_model_session** out);
WELVET_API welvet_status welvet_model_forward(welvet_model_session* s, const uint8_t* input,
                                              size_t size, welvet_cuda_blob* out);
WELVET_API welvet_status welvet_model_export_weights(welvet_model_session* s,
                                                     welvet_cuda_blob* out);
WELVET_API void welvet_model_release(welvet_model_session* s);
WELVET_API void welvet_cuda_blob_free(welvet_cuda_blob* b);

/* ==== extensions (no counterpart in the reference) ==== */

/* Dense session with a scale scheme (the reference's welvet_dense_mount has no
 * backend argument). Same contract as welvet_dense_mount otherwise. */
WELVET_API welvet_status welvet_dense_mount_q(int32_t batch, int32_t in, int32_t out, int32_t act,
                                              int32_t dtype, int32_t backend, const float* W_init,
                                              const double* bias, size_t bias_len,
                                              welvet_dense_session** sess_out);
/* Device-resident execute: x [batch*in], pre/post [batch*out] are device
 * pointers; the work is queued on `stream` (a hipStream_t; NULL = the
 * session's stream) and the call returns without waiting. post may equal pre
 * only for Linear without bias. */
WELVET_API welvet_status welvet_dense_execute_device(welvet_dense_session* sess, const float* x,
                                                     float* pre, float* post, void* stream);
/* Extension: backward of a mounted session on device buffers, queued on
 * `stream` (the session's own when null), returning without waiting. x
 * [batch*in], pre and post [batch*out] from the forward; g is the output
 * gradient (use_target 0) or an MSE target (use_target 1: post is read and
 * loss_part[ceil(batch*out/256)] receives partial sums of (post - g)^2).
 * Writes d_pre [batch*out], dX [batch*in], dW [out*in]: the arithmetic of
 * welvet_dense_normalbp_f32. The first call allocates the session's dX
 * partial buffer; later calls allocate nothing (graph-capturable). */
WELVET_API welvet_status welvet_dense_backward_device(welvet_dense_session* sess, const float* x,
                                                      const float* pre, const float* post,
                                                      const float* g, int32_t use_target,
                                                      float* dpre, float* dX, float* dW,
                                                      double* loss_part, void* stream);
/* Copies the session's quantized store to host memory: the reference
 * FormatNone payload (native_cap bytes available; *native_len set), the
 * per-row scales [out] and, for scheme 3, the E8M0 bytes [out*ceil(in/32)]. */
WELVET_API welvet_status welvet_dense_export_store(welvet_dense_session* sess, uint8_t* native,
                                                   size_t native_cap, size_t* native_len,
                                                   float* row_scale, uint8_t* blk_exp,
                                                   float* tensor_scale);

/* Dense session over a packed block format (QuantFormat). The reference
 * reserves the enum (include/welvet/weights.hpp:12-15) and lists the formats
 * (README.md:361-383) without implementing any; this is the mount that a
 * binding of those values would call. format: 1 Q8_0, 2 Q4_0, 3 Q4_1,
 * 4 Q5_0, 5 Q5_1, 6 Q2_K, 7 Q3_K, 8 Q4_K, 9 Q5_K, 10 Q6_K, 16 IQ4_NL,
 * 17 IQ4_XS (ggml's block layouts); the other values of the table (11-15,
 * 18-20) return code 3. Exactly one of W_init (fp32 [out*in], quantized on
 * the device: Q8_0 .. Q5_1 with ggml's reference quantizers, the K formats
 * and IQ4_NL / IQ4_XS with the library's one-pass quantizers) and blocks
 * (the packed row-major blocks, blocks_len bytes) is given; in must be a
 * multiple of
 * the block (32, or 256 for the K formats and IQ4_XS). Execute,
 * execute_device, execute_noalloc and release are those of
 * welvet_dense_session (device x must be 16-byte aligned); backward and the
 * grouped calls return an error. */
WELVET_API welvet_status welvet_dense_mount_format(int32_t batch, int32_t in, int32_t out,
                                                   int32_t act, int32_t format,
                                                   const float* W_init, const uint8_t* blocks,
                                                   size_t blocks_len, const double* bias,
                                                   size_t bias_len,
                                                   welvet_dense_session** sess_out);
/* The packed blocks of a format session (cap bytes available; *len set). */
WELVET_API welvet_status welvet_dense_export_blocks(welvet_dense_session* sess, uint8_t* blocks,
                                                    size_t cap, size_t* len);
/* A Dense session's weights dequantized to fp32 [out*in] host memory (the
 * role of WeightStore::export_f32, reference src/weights/store.cpp:42-71):
 * codes times row scales and E8M0 factors, or the format's dequantization. */
WELVET_API welvet_status welvet_dense_export_f32(welvet_dense_session* sess, float* W);

/* Grouped execution of Dense sessions of one shape (no counterpart in the
 * reference; for the independent cells of a volume): every session must have
 * the same batch, in, out, activation, dtype and scheme. x[i], pre[i],
 * post[i] are device buffers of member i, fixed at mount; execute queues all
 * members on `stream` (NULL = the group's stream) as one split launch and one
 * matrix-core launch when the batch exceeds 32 rows, else member by member.
 * The sessions must outlive the group; calls on a group must not overlap. */
typedef struct welvet_dense_group welvet_dense_group;
WELVET_API welvet_status welvet_dense_group_mount(welvet_dense_session* const* sessions, int32_t n,
                                                  const float* const* x, float* const* pre,
                                                  float* const* post, welvet_dense_group** out);
WELVET_API welvet_status welvet_dense_group_execute(welvet_dense_group* g, void* stream);
WELVET_API void welvet_dense_group_release(welvet_dense_group* g);

/* Chained groups (no counterpart in the reference; for the layers of a
 * volume's cells, the serial Stack of each cell run for all cells at once):
 * groups[k + 1] reads what groups[k] writes, i.e. for every member i,
 * x[i] of group k + 1 is post[i] of group k (or its pre when that group's
 * activation is Linear without bias). execute runs the groups in order on
 * `stream` (NULL = the chain's stream) with the same outputs as executing
 * them one by one. Above 32 rows, where a group's out is a multiple of 256
 * its matrix-core epilogue also writes the next group's activation split, so
 * that group skips its split launch. The groups must outlive the chain. */
typedef struct welvet_dense_chain welvet_dense_chain;
WELVET_API welvet_status welvet_dense_chain_mount(welvet_dense_group* const* groups, int32_t n,
                                                  welvet_dense_chain** out);
/* As welvet_dense_chain_mount, with flags (no counterpart in the reference).
 * WELVET_CHAIN_INNER_NOT_KEPT: a group whose epilogue writes the next
 * group's split (above 32 rows, out a multiple of 256) writes only that
 * split, not its own pre and post, whose contents after execute are then
 * unspecified; the last group's outputs, and those of every group that the
 * next one reads from memory, are written as before. For callers that need
 * only the last layer's output, as a volume's cells return it. Other bits:
 * code 1. */
#define WELVET_CHAIN_INNER_NOT_KEPT 1
WELVET_API welvet_status welvet_dense_chain_mount_ex(welvet_dense_group* const* groups, int32_t n,
                                                     int32_t flags, welvet_dense_chain** out);
WELVET_API welvet_status welvet_dense_chain_execute(welvet_dense_chain* c, void* stream);
WELVET_API void welvet_dense_chain_release(welvet_dense_chain* c);

/* SwiGLU / MHA sessions: mount once, execute many (host or device buffers). */
typedef struct welvet_swiglu_session welvet_swiglu_session;
WELVET_API welvet_status welvet_swiglu_mount(int32_t batch, int32_t seq, int32_t input_dim,
                                             int32_t intermediate_dim, int32_t dtype,
                                             int32_t backend, const float* Gate, const float* Up,
                                             const float* Down, welvet_swiglu_session** out);
WELVET_API welvet_status welvet_swiglu_execute(welvet_swiglu_session* s, const float* x,
                                               float* pre, float* post);
WELVET_API welvet_status welvet_swiglu_execute_device(welvet_swiglu_session* s, const float* x,
                                                      float* pre, float* post, void* stream);
WELVET_API void welvet_swiglu_release(welvet_swiglu_session* s);

typedef struct welvet_mha_session welvet_mha_session;
WELVET_API welvet_status welvet_mha_mount(int32_t batch, int32_t seq, int32_t d_model,
                                          int32_t num_heads, int32_t num_kv_heads,
                                          int32_t head_dim, int32_t max_seq_len, int32_t mask,
                                          int32_t pos, int32_t dtype, int32_t backend,
                                          const float* Q, const float* K, const float* V,
                                          const float* O, welvet_mha_session** out);
WELVET_API welvet_status welvet_mha_execute(welvet_mha_session* s, const float* x, float* pre,
                                            float* post);
WELVET_API welvet_status welvet_mha_execute_device(welvet_mha_session* s, const float* x,
                                                   float* pre, float* post, void* stream);
WELVET_API void welvet_mha_release(welvet_mha_session* s);

/* Model mount with a scale scheme: schemes 1-3 re-quantize each child's fp32
 * weights (the descriptor's Dense/SwiGLU/MHA W) with that scheme; 0 is
 * welvet_model_mount. */
WELVET_API welvet_status welvet_model_mount_q(const uint8_t* descriptor, size_t size,
                                              int32_t backend, welvet_model_session** out);
/* Device-resident model forward: x and y are device pointers with the shapes
 * of welvet_model_forward; y must hold the output (batch * last width). */
WELVET_API welvet_status welvet_model_forward_device(welvet_model_session* s, const float* x,
                                                     int32_t batch, int32_t width, float* y,
                                                     int32_t y_cap, void* stream);

/* Codec self-check: encodes every f32 bit pattern of the 2^20-pattern chunks
 * [first_chunk, first_chunk + n_chunks) with the device encoder used at mount
 * and returns per chunk (sum code, sum code * (pattern & 0xFFFFF)) in
 * out[2 * n_chunks]. dtype 4, 5 or 16 (FP4: the 4-bit code). */
WELVET_API welvet_status welvet_codec_sweep(int32_t dtype, uint32_t first_chunk,
                                            uint32_t n_chunks, int64_t* out);

/* No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). welvet_dense_execute_device on `rows` rows (any count, not
 * only the mounted batch) whose scratch memory (the activation split and
 * K-split partial sums of the matrix-core paths above 4 rows) is a fixed
 * 64 MiB device array of the library instead of an allocation: the call
 * allocates nothing. Code 1 when rows * in needs more than 64 MiB (about
 * 5.3 M activations on the split path). Calls on one device share the array:
 * calls that overlap in time on one device race; the previous call's
 * contents are never read. x [rows*in], pre/post [rows*out] device pointers;
 * queued on `stream` (null: the session's) without waiting. */
WELVET_API welvet_status welvet_dense_execute_noalloc(welvet_dense_session* sess, int32_t rows,
                                                      const float* x, float* pre, float* post,
                                                      void* stream);

/* Measurement extension, no reference counterpart: one streaming read of the
 * device buffer buf (bytes a positive multiple of 16) with 16-byte loads,
 * queued on `stream` (null: the default stream); out_words (device,
 * welvet_read_probe_words(bytes) entries, out_cap of them available)
 * receives one XOR digest per workgroup. Its duration is the floor for any
 * kernel that reads the same bytes once. */
WELVET_API welvet_status welvet_read_probe(const void* buf, size_t bytes, uint32_t* out_words,
                                           size_t out_cap, void* stream);
WELVET_API size_t welvet_read_probe_words(size_t bytes);

/* Measurement extension, no reference counterpart: `workgroups` workgroups
 * of 256 lanes each read `iters` 64 KiB regions of buf[0, region_bytes)
 * (region_bytes a positive multiple of 65536) with 16-byte loads, queued on
 * `stream`; out_words (device, out_cap >= workgroups) receives one digest
 * per workgroup. A region of a few MiB stays in L2 and one of GiB streams
 * from HBM: bytes / time / CUs is the fetch rate of one CU from either. */
WELVET_API welvet_status welvet_fetch_probe(const void* buf, size_t region_bytes, int32_t iters,
                                            int32_t workgroups, uint32_t* out_words,
                                            size_t out_cap, void* stream);

/* Measurement extension, no reference counterpart: `workgroups` workgroups
 * of 4 waves each issue iters x 8 (shape 16: v_mfma_scale_f32_16x16x128_f8f6f4)
 * or iters x 4 (shape 32: the 32x32x64 form) independent scaled MFMAs with
 * operand formats fmt_a x fmt_b (0 E4M3, 1 E5M2, 2 FP6 E2M3, 4 FP4; built
 * pairs: 0x0, 2x0, 2x1, 2x4, 4x4, others code 2), queued on `stream`; out
 * (device, out_cap >= 256 * workgroups floats) receives the sums. The time
 * gives the instruction's issue rate per SIMD. */
WELVET_API welvet_status welvet_mfma_probe(int32_t fmt_a, int32_t fmt_b, int32_t shape,
                                           int32_t iters, int32_t workgroups, float* out,
                                           size_t out_cap, void* stream);

/* Measurement extension, no reference counterpart: a one-lane kernel queued
 * on `stream` (null: the default stream) writes the device's constant-rate
 * wall clock to *out (device memory). Two stamps captured into one graph
 * around a run of kernels time that run with no graph launch inside it;
 * welvet_clock_rate_khz gives the clock's rate (0 without a device). */
WELVET_API welvet_status welvet_clock_stamp(uint64_t* out, void* stream);
WELVET_API int64_t welvet_clock_rate_khz(void);

/* Segment backward of a Stack model of Dense / SwiGLU children (replaces reference
 * include/welvet_c.h:55, src/interop/model_session.cpp:435-455): the input
 * blob holds the tensors x and gy (model wire: rank, dims, float32 data);
 * the forward is recomputed and the output blob holds the input gradient and
 * the dW of the ops concatenated in op order (SwiGLU: Gate, Up, Down),
 * shape [1, n]. MHA children give code 3 ("gap?"), Grid roots code 1. */
WELVET_API welvet_status welvet_model_backward(welvet_model_session*, const uint8_t*, size_t,
                                               welvet_cuda_blob*);
/* Segment forward (replaces reference include/welvet_c.h:54,
 * model_session.cpp:420-434): x in; the blob holds the last op's
 * pre-activation and the output (Stack roots; a Dense last op here). */
WELVET_API welvet_status welvet_model_forward_pair(welvet_model_session*, const uint8_t*, size_t,
                                                   welvet_cuda_blob*);
/* Dense proxy of a Stack holding one Dense (replaces reference
 * include/welvet_c.h:52, model_session.cpp:475-493): x, gy, int32 flag, and
 * with flag 1 pre; gy is remapped to batch*out values (dense.cpp:121-139).
 * kind 0: the linear input gradient [batch, in]; kind 1: dW [out, in] with
 * act' at pre (zeros when absent or short). */
WELVET_API welvet_status welvet_model_dense_proxy(welvet_model_session*, int32_t, const uint8_t*,
                                                  size_t, welvet_cuda_blob*);
/* Segment SGD (replaces reference include/welvet_c.h:56, model_session.cpp:
 * 494-507): one tensor, the concatenated dW; every store becomes
 * quantize(f32(f64(W) - lr dW)) with the session's scale scheme. */
WELVET_API welvet_status welvet_model_apply_sgd(welvet_model_session*, double, const uint8_t*,
                                                size_t);
/* Dense NormalBP leaf (replaces reference include/welvet_c.h:69-79,
 * src/interop/c_abi.cpp:119-200): forward, then the gradient (grad_or_target
 * is gradOut, or with use_target = 1 an MSE target: loss = mean (post - t)^2),
 * the backward over the quantized weights (dX [batch*in], dW [out*in]) and,
 * if lr != 0, SGD on the quantized store: W <- quantize(f32(f64(W) - lr dW))
 * with the scale scheme in `backend` (0 = the reference's element re-encode).
 * W_after [out*in] is the resulting store dequantized to f32. Host buffers;
 * the call synchronizes. Codes: 1 bad arguments, 2 unsupported dtype/scheme. */
WELVET_API welvet_status welvet_dense_normalbp_f32(
    int32_t batch, int32_t in, int32_t out, int32_t act, int32_t dtype, int32_t backend,
    const float* W_init, const double* bias, size_t bias_len, const float* x,
    const float* grad_or_target, int32_t use_target, double lr, float* pre, float* post, float* dX,
    float* dW, float* W_after, double* loss);

/* SwiGLU NormalBP leaf (replaces reference include/welvet_c.h:137-146,
 * src/interop/c_abi.cpp:581-652): forward (pre = h [B*S*inter], post = y
 * [B*S*in]), the gradient (gradOut, or with use_target an MSE target), the
 * backward over the three quantized matrices (dX [B*S*in], dW = Gate | Up |
 * Down, 3*inter*in), SGD on each store if lr != 0, W_after in the same order,
 * dequantized. Scale scheme in `backend`. */
WELVET_API welvet_status welvet_swiglu_normalbp_f32(
    int32_t batch, int32_t seq, int32_t input_dim, int32_t intermediate_dim, int32_t dtype,
    int32_t backend, const float* Gate, const float* Up, const float* Down, const float* x,
    const float* grad_or_target, int32_t use_target, double lr, float* pre, float* post, float* dX,
    float* dW, float* W_after, double* loss);

/* ==== reference entry points outside this path: code 3 ("gap?") ====
 * Same signatures as reference include/welvet_c.h:50-59, 74-130, 142-162,
 * 175-386. */
WELVET_API welvet_status welvet_model_train_credit(welvet_model_session*, int32_t, double,
                                                   const uint8_t*, size_t);
WELVET_API welvet_status welvet_model_train_mse(welvet_model_session*, int32_t mode, double lr,
                                                int32_t ticks, const uint8_t*, size_t,
                                                double* loss);
WELVET_API welvet_status welvet_model_sync(welvet_model_session*, int32_t event);
WELVET_API welvet_status welvet_rmsnorm_forward_f32(int32_t batch, int32_t seq, int32_t dim,
                                                    double eps, int32_t dtype, int32_t backend,
                                                    const float* gamma, const float* x, float* pre,
                                                    float* post);
WELVET_API welvet_status welvet_rmsnorm_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, double eps, int32_t dtype, int32_t backend,
    const float* gamma_init, const float* x, const float* grad_or_target, int32_t use_target,
    double lr, float* pre, float* post, float* dX, float* dW, float* gamma_after, double* loss);
WELVET_API welvet_status welvet_layernorm_forward_f32(int32_t batch, int32_t seq, int32_t dim,
                                                      double eps, int32_t dtype, int32_t backend,
                                                      const float* gamma, const float* beta,
                                                      const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_layernorm_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, double eps, int32_t dtype, int32_t backend,
    const float* gamma_init, const float* beta_init, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW,
    float* gamma_after, float* beta_after, double* loss);
WELVET_API welvet_status welvet_softmax_forward_f32(
    int32_t n, int32_t dim, int32_t seq_len, int32_t kind, int32_t rows, int32_t cols,
    double temperature, double entmax_alpha, int32_t gumbel_seed, int32_t dtype, int32_t backend,
    int32_t rank, const int32_t* shape, const uint8_t* mask, int32_t mask_len, const int32_t* hier,
    int32_t hier_len, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_softmax_normalbp_f32(
    int32_t n, int32_t dim, int32_t seq_len, int32_t kind, int32_t rows, int32_t cols,
    double temperature, double entmax_alpha, int32_t gumbel_seed, int32_t dtype, int32_t backend,
    int32_t rank, const int32_t* shape, const uint8_t* mask, int32_t mask_len, const int32_t* hier,
    int32_t hier_len, const float* x, const float* grad_or_target, int32_t use_target, double lr,
    float* pre, float* post, float* dX, double* loss);
WELVET_API welvet_status welvet_embedding_forward_f32(
    int32_t batch, int32_t vocab, int32_t emb, int32_t seq_len, int32_t in_rank, int32_t in_last,
    int32_t act, int32_t dtype, int32_t backend, const float* W, const float* x, float* pre,
    float* post);
WELVET_API welvet_status welvet_embedding_normalbp_f32(
    int32_t batch, int32_t vocab, int32_t emb, int32_t seq_len, int32_t in_rank, int32_t in_last,
    int32_t act, int32_t dtype, int32_t backend, const float* W_init, const float* x,
    const float* grad_or_target, int32_t use_target, double lr, float* pre, float* post, float* dX,
    float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_mha_normalbp_f32(
    int32_t batch, int32_t seq, int32_t d_model, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t max_seq_len, int32_t mask, int32_t pos, int32_t dtype, int32_t backend,
    const float* Q, const float* K, const float* V, const float* O, const float* x,
    const float* grad_or_target, int32_t use_target, double lr, float* pre, float* post, float* dX,
    float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_cnn1_forward_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t seq_len, int32_t kernel, int32_t stride,
    int32_t padding, int32_t act, int32_t dtype, int32_t backend, const float* W, const double* bias,
    size_t bias_len, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_cnn1_normalbp_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t seq_len, int32_t kernel, int32_t stride,
    int32_t padding, int32_t act, int32_t dtype, int32_t backend, const float* W, const double* bias,
    size_t bias_len, const float* x, const float* grad_or_target, int32_t use_target, double lr,
    float* pre, float* post, float* dX, float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_cnn2_forward_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t height, int32_t width, int32_t kernel,
    int32_t stride, int32_t padding, int32_t act, int32_t dtype, int32_t backend, const float* W,
    const double* bias, size_t bias_len, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_cnn2_normalbp_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t height, int32_t width, int32_t kernel,
    int32_t stride, int32_t padding, int32_t act, int32_t dtype, int32_t backend, const float* W,
    const double* bias, size_t bias_len, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_cnn3_forward_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t depth, int32_t height, int32_t width,
    int32_t kernel, int32_t stride, int32_t padding, int32_t act, int32_t dtype, int32_t backend,
    const float* W, const double* bias, size_t bias_len, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_cnn3_normalbp_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t depth, int32_t height, int32_t width,
    int32_t kernel, int32_t stride, int32_t padding, int32_t act, int32_t dtype, int32_t backend,
    const float* W, const double* bias, size_t bias_len, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_convt1_forward_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t seq_len, int32_t kernel, int32_t stride,
    int32_t padding, int32_t output_padding, int32_t act, int32_t dtype, int32_t backend,
    const float* W, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_convt1_normalbp_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t seq_len, int32_t kernel, int32_t stride,
    int32_t padding, int32_t output_padding, int32_t act, int32_t dtype, int32_t backend,
    const float* W, const float* x, const float* grad_or_target, int32_t use_target, double lr,
    float* pre, float* post, float* dX, float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_convt2_forward_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t height, int32_t width, int32_t kernel,
    int32_t stride, int32_t padding, int32_t output_padding, int32_t act, int32_t dtype,
    int32_t backend, const float* W, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_convt2_normalbp_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t height, int32_t width, int32_t kernel,
    int32_t stride, int32_t padding, int32_t output_padding, int32_t act, int32_t dtype,
    int32_t backend, const float* W, const float* x, const float* grad_or_target, int32_t use_target,
    double lr, float* pre, float* post, float* dX, float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_convt3_forward_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t depth, int32_t height, int32_t width,
    int32_t kernel, int32_t stride, int32_t padding, int32_t output_padding, int32_t act,
    int32_t dtype, int32_t backend, const float* W, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_convt3_normalbp_f32(
    int32_t batch, int32_t in_c, int32_t filters, int32_t depth, int32_t height, int32_t width,
    int32_t kernel, int32_t stride, int32_t padding, int32_t output_padding, int32_t act,
    int32_t dtype, int32_t backend, const float* W, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_rnn_forward_f32(
    int32_t batch, int32_t input_size, int32_t hidden_size, int32_t seq_len, int32_t dtype,
    int32_t backend, const float* packed, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_rnn_normalbp_f32(
    int32_t batch, int32_t input_size, int32_t hidden_size, int32_t seq_len, int32_t dtype,
    int32_t backend, const float* packed, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_lstm_forward_f32(
    int32_t batch, int32_t input_size, int32_t hidden_size, int32_t seq_len, int32_t dtype,
    int32_t backend, const float* packed, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_lstm_normalbp_f32(
    int32_t batch, int32_t input_size, int32_t hidden_size, int32_t seq_len, int32_t dtype,
    int32_t backend, const float* packed, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_sequential_forward_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t depth, int32_t child_act, int32_t dtype,
    int32_t backend, const float* packed, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_sequential_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t depth, int32_t child_act, int32_t dtype,
    int32_t backend, const float* packed, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_residual_forward_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t depth, int32_t child_act, int32_t dtype,
    int32_t backend, const float* packed, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_residual_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t depth, int32_t child_act, int32_t dtype,
    int32_t backend, const float* packed, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_stack_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t n_children, int32_t child_act, int32_t dtype,
    int32_t backend, const float* packed, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_mamba_normalbp_f32(
    int32_t batch, int32_t seq, int32_t d_model, int32_t d_state, int32_t expand, int32_t dtype,
    int32_t backend, const float* packed, const float* x, const float* grad_or_target,
    int32_t use_target, double lr, float* pre, float* post, float* dX, float* dW, float* W_after,
    double* loss);
WELVET_API welvet_status welvet_metacognition_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t dtype, int32_t backend, const float* packed,
    const float* x, const float* grad_or_target, int32_t use_target, double lr, float* pre,
    float* post, float* dX, float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_gdn_normalbp_f32(
    int32_t batch, int32_t seq, int32_t hidden, int32_t num_key_heads, int32_t num_value_heads,
    int32_t key_head_dim, int32_t value_head_dim, int32_t conv_kernel, int32_t dtype, int32_t backend,
    const float* packed, const float* x, const float* grad_or_target, int32_t use_target, double lr,
    float* pre, float* post, float* dX, float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_kmeans_normalbp_f32(
    int32_t batch, int32_t seq, int32_t num_clusters, int32_t feature_dim, int32_t output_mode,
    int32_t act, double temperature, int32_t dtype, int32_t backend, const float* W, const float* x,
    const float* grad_or_target, int32_t use_target, double lr, float* pre, float* post, float* dX,
    float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_parallel_normalbp_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t out_feat, int32_t branches, int32_t combine,
    int32_t sparse_k, int32_t dtype, int32_t backend, double disagree_beta, const float* packed,
    const float* x, const float* grad_or_target, int32_t use_target, double lr, float* pre,
    float* post, float* dX, float* dW, float* W_after, double* loss);
WELVET_API welvet_status welvet_mamba_forward_f32(
    int32_t batch, int32_t seq, int32_t d_model, int32_t d_state, int32_t expand, int32_t dtype,
    int32_t backend, const float* packed, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_metacognition_forward_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t dtype, int32_t backend, const float* packed,
    const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_gdn_forward_f32(
    int32_t batch, int32_t seq, int32_t hidden, int32_t num_key_heads, int32_t num_value_heads,
    int32_t key_head_dim, int32_t value_head_dim, int32_t conv_kernel, int32_t dtype, int32_t backend,
    const float* packed, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_kmeans_forward_f32(
    int32_t n, int32_t feature_dim, int32_t num_clusters, int32_t output_mode, int32_t act,
    double temperature, int32_t dtype, int32_t backend, int32_t rank, const int32_t* shape,
    const float* W, const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_parallel_forward_f32(
    int32_t batch, int32_t seq, int32_t dim, int32_t out_feat, int32_t branches, int32_t combine,
    int32_t sparse_k, int32_t dtype, int32_t backend, double disagree_beta, const float* packed,
    const float* x, float* pre, float* post);
WELVET_API welvet_status welvet_seqmix_kind_name(int32_t kind, char* buf, int32_t buf_len);
WELVET_API int32_t welvet_seqmix_mha_kind(void);
WELVET_API int32_t welvet_seqmix_mamba_kind(void);
WELVET_API int32_t welvet_seqmix_gdn_kind(void);

#ifdef __cplusplus
}
#endif

#endif /* WELVET_C_H */
