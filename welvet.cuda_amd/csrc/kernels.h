// Host-side launchers of the device kernels.
#pragma once

#include "common.h"

namespace wv {

// ---- mount-time quantization (quant.hip) ----
// Quantizes the device fp32 matrix dW [rows x cols] into dw (allocates it) and,
// if d_raw is set, writes the reference FormatNone payload there.
// Builds DeviceWeights::codes_frag from the codes (operand-order copy read
// by the 5..32-row GEMM when present).
Status build_codes_frag(DeviceWeights* dw, hipStream_t st);
Status quantize_to_device(const float* dW, int dtype, int scheme, int rows, int cols,
                          DeviceWeights* dw, uint8_t* d_raw, hipStream_t st);
// Builds dw from a reference payload already on the device plus optional
// scales (row scales [rows]; E8M0 bytes [rows][ceil(cols/32)]).
Status relayout_to_device(const uint8_t* d_raw, int dtype, int scheme, int rows, int cols,
                          const float* d_row_scale, const uint8_t* d_blk_rows,
                          DeviceWeights* dw, hipStream_t st);
// Encoder digests over all f32 patterns of the given 2^20-pattern chunks.
Status codec_sweep(int dtype, uint32_t first_chunk, uint32_t n_chunks, int64_t* host_out,
                   hipStream_t st);

// ---- weight rows with non-finite codes (special.hip) ----
// Fills dw->nf_rows / nf_host with the rows holding E5M2 inf/NaN codes.
Status find_nonfinite_rows(DeviceWeights* dw, hipStream_t st);
// Dequantized f32 of elements [e0, e0 + n) of a row-major rows x cols
// FormatNone payload (FP4: element i in byte i / 2, odd i in the high
// nibble): decode times the row scale, or times 2^e of the element's
// 32-column block. `bytes` starts at the byte of element e0 (e0 / 2 for
// FP4); row_scale (or null: 1) and blk ([row][nb] E8M0 bytes, or null) start
// at row e0 / cols.
Status launch_decode_store(const uint8_t* bytes, int dtype, int64_t e0, int64_t n, int cols,
                           const float* row_scale, const uint8_t* blk, int nb, float* out,
                           hipStream_t st);
// Device copy of a row list (out is reset; left empty for an empty list).
Status upload_rows(const std::vector<int>& rows, DevBuf* out, hipStream_t st);
// Recomputes the listed output rows of a product (decoded weights, f64 sum)
// and applies the epilogue: bias / activation (mats 1) or the SwiGLU product
// of matrices 0 and 1 into pre (mats 2).
struct NfArgs {
  const int* rows = nullptr;
  int n = 0;
  int dtype = 0, mats = 1;
  const uint8_t* codes[2] = {nullptr, nullptr};
  const float* scale[2] = {nullptr, nullptr};
  const uint8_t* blk[2] = {nullptr, nullptr};
  int pitch = 0, nblk = 0, cols = 0;
  const float* x = nullptr;
  int x_stride = 0, batch = 0;
  float* pre = nullptr;
  float* post = nullptr;
  int out_stride = 0;
  int act = kLinear;
  int need_epi = 0;
  const double* bias = nullptr;
  int bias_len = 0;
};
Status launch_nf_fix(const NfArgs& a, hipStream_t st);

// ---- streaming read of a buffer (probe.hip): the read floor ----
// Words of `out` a read of `bytes` writes (one per workgroup).
size_t read_probe_words(size_t bytes);
Status launch_read_probe(const uint8_t* buf, size_t bytes, uint32_t* out, hipStream_t st);
// the device wall clock into *out (one lane of one workgroup)
Status launch_clock_stamp(uint64_t* out, hipStream_t st);
// `workgroups` workgroups of 256 lanes each read `iters` 64 KiB regions of
// buf[0, region_bytes); out: one word per workgroup
Status launch_fetch_probe(const uint8_t* buf, size_t region_bytes, int iters, int workgroups,
                          uint32_t* out, hipStream_t st);
// `workgroups` workgroups of 4 waves each issue iters x 8 (shape 16) or x 4
// (shape 32) scaled MFMAs with operand formats fmt_a / fmt_b (0 E4M3, 1
// E5M2, 2 FP6 E2M3, 4 FP4); out: workgroups x 256 floats
Status launch_mfma_probe(int fmt_a, int fmt_b, int shape, int iters, int workgroups, float* out,
                         hipStream_t st);

// ---- small-batch GEMV (gemv.hip) ----
struct GemvArgs {
  const uint8_t* codes[2] = {nullptr, nullptr};
  const float* scale[2] = {nullptr, nullptr};
  const uint8_t* blk[2] = {nullptr, nullptr};
  int mats = 1;
  int pitch = 0, nblk = 0, kpad = 0, cols = 0, rows = 0;
  const float* x = nullptr;
  int x_stride = 0;
  float* pre = nullptr;
  float* post = nullptr;
  int out_stride = 0;
  int act = kLinear;
  int need_epi = 0;
  const double* bias = nullptr;
  int bias_len = 0;
};
// Rows per workgroup (2, 4, 8, 16) and waves per workgroup (1, 2, 4, or 3, 6,
// 8 with 8 rows; they split K).
struct GemvTile {
  int rows = 8;
  int waves = 4;
};
GemvTile gemv_tile(int dtype, int kpad, int rows, int mats, int cus);
Status launch_gemv(const GemvArgs& a, int dtype, bool blk, int batch, GemvTile tile,
                   hipStream_t st);

// ---- small-batch GEMV on the scaled MFMA (mxv.hip) ----
constexpr int kMxvMaxBatch = 4;
struct MxvArgs {
  const uint8_t* codes[2] = {nullptr, nullptr};
  const float* scale[2] = {nullptr, nullptr};
  const uint8_t* blk[2] = {nullptr, nullptr};
  int mats = 1;
  int pitch = 0, nblk = 0, kpad = 0, cols = 0, rows = 0;
  const float* x = nullptr;
  int x_stride = 0;
  int batch = 1;
  float* pre = nullptr;
  float* post = nullptr;
  int out_stride = 0;
  int act = kLinear;
  int need_epi = 0;
  const double* bias = nullptr;
  int bias_len = 0;
};
Status launch_mxv(const MxvArgs& a, int dtype, bool blk, hipStream_t st);

// ---- 1-4-row GEMV on the scaled MFMA over operand-order weights (gemv_mx.hip) ----
// x as three E4M3 terms per 16-element piece in the rows of the A operand;
// the weights from DeviceWeights::codes_frag (and blk_frag). The pre-split
// input image (asplit / next) holds, per K chunk of 128, the term codes
// [3][4 lane groups][32 B] (piece p of the chunk at lane group p & 3, byte
// 16 (p >> 2)), and after all `steps` chunks the exponents [steps][3][8]
// (E8M0 + 127 per term and piece; 0xFF marks a non-finite piece).
struct GemvMxArgs {
  const uint8_t* codesf[2] = {nullptr, nullptr};
  const uint8_t* blkf[2] = {nullptr, nullptr};
  const float* scale[2] = {nullptr, nullptr};
  int mats = 1;
  int kpad = 0, cols = 0, rows = 0;
  int nb = 1;  // batch rows, 1..kGemvMxMaxRows
  // fp32 input [nb][cols], 16-byte aligned with cols % 4 == 0 unless asplit
  // is given (then read only by the non-finite fallback)
  const float* x = nullptr;
  // pre-split x (one matrix): one image of asplit_steps chunks per batch
  // row, back to back; or null
  const uint8_t* asplit = nullptr;
  int asplit_steps = 0;
  // two matrices: the split of h written here (one image of next_steps
  // chunks per batch row), or null
  uint8_t* next = nullptr;
  int next_steps = 0;
  float* pre = nullptr;   // [nb][rows]
  float* post = nullptr;  // [nb][rows]
  int act = kLinear;
  int need_epi = 0;
  const double* bias = nullptr;
  int bias_len = 0;
};
constexpr int kGemvMxMaxRows = 4;
// Shapes the kernel runs: FP8/FP4, at least 256 row blocks of 16, 16..128
// K chunks of 128 (96 for 4 batch rows), 1..4 batch rows.
bool gemv_mx_fits(int dtype, int rows, int kpad, int mats, int nb);
// Bytes of one batch row's pre-split input image over kpad columns.
size_t gemv_mx_split_bytes(int kpad);
Status launch_gemv_mx(const GemvMxArgs& a, int dtype, bool blk, hipStream_t st);

// ---- batched GEMM on the scaled MFMA (mxg.hip) ----
// Activations are split into kTerms terms with per-32 E8M0 scales (two or one
// for one-matrix products that ask for them: less residual precision, less
// matrix-core work and fewer activation bytes). Three-term splits hold FP6
// E2M3 terms ((block, chunk) slices of 3 x 1.5 KiB), the others E4M3 terms
// (NT x 2 KiB). The split buffer is always sized
// for kTerms E4M3 terms; the exponents sit at the same offset in every
// format.
constexpr int kTerms = 3;
struct MxgArgs {
  // term codes in MFMA operand order, [mpad/16][kpad/128][kTerms][2][64][16]
  // (FP6 terms: [mpad/16][kpad/128][kTerms][1536], 16 B of lane l at 16 l,
  // then 8 B at 1024 + 8 l)
  // (16-row block, K chunk, term, operand half, lane, byte)
  const uint8_t* a = nullptr;
  // E8M0 exponents, [mpad/16][kpad/128][64] dwords; byte t is term t's
  const uint8_t* as = nullptr;
  int M = 0, mpad = 0;
  const uint8_t* codes[2] = {nullptr, nullptr};
  const float* scale[2] = {nullptr, nullptr};
  const uint8_t* blk[2] = {nullptr, nullptr};
  int mats = 1;
  int pitch = 0, nblk = 0, kpad = 0, N = 0;
  float* pre = nullptr;
  float* post = nullptr;
  int out_stride = 0;
  int act = kLinear;
  int need_epi = 0;
  const double* bias = nullptr;
  int bias_len = 0;
  // small-M products split along K: raw partial sums (mxg_part_bytes)
  float* part = nullptr;
  // block exponents in lane order (DeviceWeights::blk_frag), BLOCK32 only
  const uint8_t* blkf[2] = {nullptr, nullptr};
  // codes in operand order (DeviceWeights::codes_frag) or null; the 5..32-row
  // GEMM reads them instead of `codes` when every matrix has them
  const uint8_t* codesf[2] = {nullptr, nullptr};
  // small M (mxg_block_m(M) == 16): the fp32 input [M][cols] (row stride
  // x_stride), split into terms by the GEMM kernel itself (a / as unused);
  // x_vec: x 16-byte aligned, cols and x_stride multiples of 4
  const float* x = nullptr;
  int x_stride = 0, cols = 0, x_vec = 0;
  // large tiles, one matrix, no bias or activation: when set, the epilogue
  // applies RoPE to the output (row m = token position m, heads of rope_hd
  // columns, 128 % rope_hd == 0): pairs (d, d + rope_hd/2) rotated by the
  // (cos, sin) table [token][pair] in f64, as build_rope_table makes it
  const double* rope_tab = nullptr;
  int rope_hd = 0;
  // large tiles, one matrix, N a multiple of 256: when set, the epilogue also
  // writes the split of post here, laid out as the split buffer of a layer
  // with the same rows (mpad) and kpad = N (the next layer of a chain, which
  // uses the same number of terms)
  uint8_t* next = nullptr;
  // activation terms: kTerms, or 1 or 2 for one-matrix products (1: above
  // 32 rows only)
  int terms = kTerms;
  // large tiles: 1 when the next launch reads the output (the MHA Q, K, V
  // and SwiGLU gate+up products): plain stores, which leave it in the
  // caches; 0: streaming stores
  int keep_out = 0;
};
int mxg_block_m(int M);
// Bytes of the K-split partial buffer the product of M rows with N outputs
// (per matrix) needs; 0 when it takes no split.
size_t mxg_part_bytes(int M, int kpad, int N, int mats);
// Bytes of the split buffer for M rows of kpad columns.
size_t split_bytes(int M, int kpad);
// x [M][cols] (row stride x_stride) -> split terms in buf.
// Three-term splits hold FP6 (E2M3) terms, two- and one-term splits E4M3
// terms; the product's kernel reads the same format.
Status launch_split(const float* x, int x_stride, int M, int cols, int kpad, uint8_t* buf,
                    hipStream_t st, int terms = kTerms);
Status launch_mxg(const MxgArgs& p, int dtype, bool blk, hipStream_t st);
// Adds the ksplit partial planes of a split product (rows: the product's
// weight rows per workgroup, which pad the planes) and applies the epilogue
// (reduce.hip); mats 2: the SwiGLU gate+up pair. Launch errors are left for
// the caller's hipGetLastError.
void launch_mxs_reduce(const MxgArgs& p, int ksplit, int rows, int mats, hipStream_t st);
// The reduce of a split large-tile product of one matrix (N a multiple of
// 256, pre and post 16-byte aligned, out_stride a multiple of 4) that also
// writes the split of post to p.next for the next layer of a chain
// (reduce.hip).
void launch_reduce_split(const MxgArgs& p, int ksplit, hipStream_t st);
// Grouped forms over n members that share every shape field: `jobs` / `tab`
// are device arrays of n entries (one split input and buffer / one GEMM
// argument block per member). One launch covers all members.
struct SplitJob {
  const float* x = nullptr;
  uint8_t* buf = nullptr;
};
Status launch_split_group(const SplitJob* jobs, int n, bool vec, int x_stride, int M, int cols,
                          int kpad, hipStream_t st, int terms = kTerms);
// Members must take the large-tile GEMM (M above 32 rows).
Status launch_mxg_group(const MxgArgs* tab, const MxgArgs& shape, int n, int dtype, bool blk,
                        hipStream_t st);

// ---- attention core (attention.hip) ----
struct AttnArgs {
  const float* q = nullptr;  // [tokens][heads*hd], rotated in place when rope
  const float* k = nullptr;  // [tokens][kv_heads*hd], rotated in place when rope
  const float* v = nullptr;  // [tokens][kv_heads*hd]
  float* out = nullptr;      // [tokens][heads*hd]
  int tokens = 0, seq = 0, heads = 0, kv_heads = 0, hd = 0, msl = 0;
  int mask = 1, window = 0, prefix_len = 0, window_causal = 1;
  int rope = 0, alibi = 0, sigmoid = 0;
  double rope_theta = 10000.0, scale = 0.125;
  // optional (cos, sin) per [token][pair] in f64 (build_rope_table); without
  // it the rotation angles are computed per call
  const double* rope_tab = nullptr;
  // optional (attention_writes_split): the kernel also writes the
  // three-term FP6 split of out, laid out as the split buffer of a layer
  // with split_mpad rows and kpad = heads * hd (the O projection's input)
  uint8_t* split = nullptr;
  int split_mpad = 0;
};
Status launch_attention(const AttnArgs& a, hipStream_t st);
// True when the matrix-core attention runs for `a` and can write the split
// of its output: head_dim 32, 64 or 128, heads * hd a multiple of 256, seq
// a multiple of 16 (each wave's 16 queries are one aligned row block).
bool attention_writes_split(const AttnArgs& a);
// (cos, sin) of t / theta^(2d/hd) for tokens t < tokens and pairs d < hd/2,
// in f64: tab[2 * (t * (hd/2) + d) + {0, 1}].
Status build_rope_table(double* tab, int tokens, int hd, double theta, hipStream_t st);

// ---- Dense backward and SGD (backward.hip) ----
// d_pre = f32(f64(gy) * act'(f64 pre)) over n = batch * out elements; with
// use_target, g holds the target and gy = f32(2/n (post - target)), and
// loss_part[dpre_blocks(n)] receives the per-block sums of (post - target)^2.
int64_t dpre_blocks(int64_t n);
Status launch_dpre(const float* g, const float* post, const float* pre, int act, int use_target,
                   int64_t n, float* dpre, double* loss_part, hipStream_t st);
struct GemvtArgs {
  const uint8_t* codes = nullptr;  // device codes [rpad][pitch]
  const float* scale = nullptr;    // [rpad]
  const uint8_t* blk = nullptr;    // [rpad][nblk] E8M0, scheme 3
  int pitch = 0, nblk = 0, kpad = 0, in = 0, out = 0;
  const float* dpre = nullptr;     // [batch][out]
};
// Bytes of the f64 partial buffer launch_backward_products needs.
size_t gemvt_part_bytes(int in, int out);
// dX [batch][in] = W^T d_pre (f64 accumulation, rounded once to f32) and dW
// [out][in] (the reference's per-batch-row f32 accumulation) from d_pre.
// With dpre_out set, a.dpre is gy of a Linear layer without a target (d_pre
// equals it) and the launch also stores it to dpre_out [batch][out].
Status launch_backward_products(const GemvtArgs& a, int dtype, bool blk, int batch,
                                const float* x, float* dw, double* part, float* dx,
                                float* dpre_out, hipStream_t st);
// SwiGLU backward product (d_up, d_gate from gate_pre, up_post, grad_h) and
// the f64 sum of two gradients, rounded to f32.
Status launch_swiglu_bwd(const float* gate_pre, const float* up_post, const float* grad_h,
                         float* d_up, float* d_gate, int64_t n, hipStream_t st);
Status launch_add_f64(const float* a, const float* b, float* out, int64_t n, hipStream_t st);
// w_next [rows][cols] = f32(f64(dequant(W)) - lr * f64(dW)).
Status launch_sgd(const DeviceWeights& d, const float* dw, double lr, float* w_next,
                  hipStream_t st);
Status launch_sgd(const DeviceWeights& d, const double* dw, double lr, float* w_next,
                  hipStream_t st);
// W as f32 [rows][cols]: decode times the scales.
Status launch_dequant(const DeviceWeights& d, float* w, hipStream_t st);

// ---- packed block formats (formats.hip) ----
// QuantFormat ids: the reference's enum (include/welvet/weights.hpp:12-15)
// holds only None; the other values follow the order of its format table
// (README.md:361-383).
enum QuantFormat : int32_t {
  kFmtNone = 0, kQ8_0 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 4, kQ5_1 = 5, kQ2_K = 6, kQ3_K = 7,
  kQ4_K = 8, kQ5_K = 9, kQ6_K = 10, kIQ4_NL = 16, kIQ4_XS = 17, kFmtLast = 20
};
// Elements and packed bytes per block; bytes per 32-element sub-block of the
// resident code (q), high-bit (h) and scale (s) arrays, and of the per-256
// array e (Q6_K's d).
struct FmtGeom {
  int qk, bb, qb, hb, sb, eb;
};
constexpr FmtGeom fmt_geom(int fmt) {
  return fmt == kQ8_0   ? FmtGeom{32, 34, 32, 0, 2, 0}
         : fmt == kQ4_0 ? FmtGeom{32, 18, 16, 0, 2, 0}
         : fmt == kQ4_1 ? FmtGeom{32, 20, 16, 0, 4, 0}
         : fmt == kQ5_0 ? FmtGeom{32, 22, 16, 4, 2, 0}
         : fmt == kQ5_1 ? FmtGeom{32, 24, 16, 4, 4, 0}
         : fmt == kQ2_K ? FmtGeom{256, 84, 8, 0, 2, 4}
         : fmt == kQ3_K ? FmtGeom{256, 110, 8, 4, 2, 0}
         : fmt == kQ4_K ? FmtGeom{256, 144, 16, 0, 2, 0}
         : fmt == kQ5_K ? FmtGeom{256, 176, 16, 4, 2, 0}
         : fmt == kQ6_K ? FmtGeom{256, 210, 16, 8, 2, 2}
         : fmt == kIQ4_NL ? FmtGeom{32, 18, 16, 0, 2, 0}
         : fmt == kIQ4_XS ? FmtGeom{256, 136, 16, 0, 1, 0}
                        : FmtGeom{0, 0, 0, 0, 0, 0};
}
struct FmtArgs {
  const uint8_t* q = nullptr;  // [rpad][nsub][qb]
  const uint8_t* h = nullptr;  // [rpad][nsub][hb]
  const uint8_t* s = nullptr;  // [rpad][nsub][sb]
  const uint8_t* e = nullptr;  // [rpad][nsub / 8][eb] (Q2_K d, dmin; Q6_K d)
  int rows = 0, cols = 0, nsub = 0;  // nsub = cols / 32
  const float* x = nullptr;
  int x_stride = 0;
  float* pre = nullptr;
  float* post = nullptr;
  int out_stride = 0, act = -1, bias_len = 0;
  bool need_epi = false;
  const double* bias = nullptr;
};
// Packed blocks of n row-major elements (a multiple of the format's block)
// from fp32 W (device): Q8_0, Q4_0, Q4_1, Q5_0 and Q5_1 with ggml's
// reference quantizers; the K and IQ4 formats with the library's one-pass
// quantizers (formats.hip).
Status format_quantize(int fmt, const float* W, int64_t n, uint8_t* out, hipStream_t st);
// Packed blocks of rows x cols -> the resident arrays of a (q, h, s, e set).
Status format_relayout(int fmt, const FmtArgs& a, const uint8_t* blocks, int rows, hipStream_t st);
// The resident arrays -> f32 [rows][cols] (the format's dequantization).
Status format_dequant(int fmt, const FmtArgs& a, int rows, float* out, hipStream_t st);
// y = W x for every one of `batch` rows of x (a.x, a.x_stride), with the Dense
// epilogue into a.pre / a.post.
Status launch_format_gemv(int fmt, const FmtArgs& a, int batch, hipStream_t st);

}  // namespace wv
