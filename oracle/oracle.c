/*
 * CPU oracle for the quantized-weight Dense path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference numerical contract (welvet.cuda
 * 0.79). Only tests, the smoke check and the benchmark's CPU-baseline leg use
 * it. Build flags follow the reference host flags: -O2 -ffp-contract=off
 * (reference CMakeLists.txt:102-106), so every f32/f64 operation below rounds
 * exactly once, in program order.
 */
#define _POSIX_C_SOURCE 200809L
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* ------------------------------------------------------------------------- */
/* E4M3 (float_codecs.cpp:57-97). Rules: zero/NaN -> 0x00; sign from f < 0;  */
/* |f| > 448 -> S|0x7E; biased exponent E = exp + 7; E < -2 -> S; E in       */
/* [-2, 0] -> truncated subnormal mantissa; E >= 15 -> S|0x7E; otherwise     */
/* 3-bit mantissa rounded half-away on bit 19 alone, with carry into E.      */
uint8_t or_enc_e4m3(float f) {
  if (isnan(f) || f == 0.0f) return 0x00;
  const uint8_t s = (f < 0.0f) ? 0x80 : 0x00;
  const float a = (f < 0.0f) ? -f : f;
  if (a > 448.0f) return (uint8_t)(s | 0x7E);
  const uint32_t bits = f2u(a);
  const uint32_t frac = bits & 0x7FFFFFu;
  int E = (int)(bits >> 23) - 127 + 7;
  if (E <= 0) {
    if (E < -2) return s;
    const uint32_t sub = (frac | 0x800000u) >> (uint32_t)(21 - E);
    return (uint8_t)(s | (sub & 7u));
  }
  if (E >= 15) return (uint8_t)(s | 0x7E);
  uint32_t m = (frac >> 20) & 7u;
  if ((frac >> 19) & 1u) {
    m += 1u;
    if (m == 8u) {
      m = 0u;
      E += 1;
      if (E >= 15) return (uint8_t)(s | 0x7E);
    }
  }
  return (uint8_t)(s | ((uint32_t)E << 3) | m);
}

/* float_codecs.cpp:99-117: E == 0 decodes to signed zero for every mantissa; */
/* 0x7F/0xFF decode to +-448; the rest is the exact normal value.            */
float or_dec_e4m3(uint8_t b) {
  const uint32_t s = (b & 0x80u) ? 0x80000000u : 0u;
  const uint32_t E = (b >> 3) & 15u, m = b & 7u;
  if (E == 0u) return u2f(s);
  if (E == 15u && m == 7u) return u2f(s | f2u(448.0f));
  return u2f(s | ((E + 120u) << 23) | (m << 20));
}

/* E5M2 (float_codecs.cpp:119-158): NaN -> 0x7E; sign from f < 0 or signbit; */
/* +-inf -> S|0x7C; zero -> S; E = exp + 15 <= 0 -> S (flush); E >= 31 ->    */
/* S|0x7C; 2-bit mantissa rounded half-away on bit 20 with carry.            */
uint8_t or_enc_e5m2(float f) {
  if (isnan(f)) return 0x7E;
  const uint8_t s = (f < 0.0f || signbit(f)) ? 0x80 : 0x00;
  const float a = (f < 0.0f) ? -f : f;
  if (isinf(a)) return (uint8_t)(s | 0x7C);
  if (a == 0.0f) return s;
  const uint32_t bits = f2u(a);
  const uint32_t frac = bits & 0x7FFFFFu;
  int E = (int)(bits >> 23) - 127 + 15;
  if (E <= 0) return s;
  if (E >= 31) return (uint8_t)(s | 0x7C);
  uint32_t m = (frac >> 21) & 3u;
  if ((frac >> 20) & 1u) {
    m += 1u;
    if (m == 4u) {
      m = 0u;
      E += 1;
      if (E >= 31) return (uint8_t)(s | 0x7C);
    }
  }
  return (uint8_t)(s | ((uint32_t)E << 2) | m);
}

/* float_codecs.cpp:160-182: E == 0 -> signed zero; E == 31 -> inf (m == 0)  */
/* or sign|0x7FC00000; else exact normal.                                   */
float or_dec_e5m2(uint8_t b) {
  const uint32_t s = (b & 0x80u) ? 0x80000000u : 0u;
  const uint32_t E = (b >> 2) & 31u, m = b & 3u;
  if (E == 0u) return u2f(s);
  if (E == 31u) return u2f(s | (m ? 0x7FC00000u : 0x7F800000u));
  return u2f(s | ((E + 112u) << 23) | (m << 21));
}

/* E2M1 value table, code order S EE M (float_codecs.cpp:184). */
static const float kE2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

/* float_codecs.cpp:187-198: first code (lowest index) with the strictly     */
/* smallest f32 |f - value|, searched from best_err = FLT_MAX. The f32        */
/* subtraction is part of the contract (it decides ties and huge inputs).    */
uint8_t or_enc_fp4(float f) {
  float best_err = FLT_MAX;
  uint8_t best = 0;
  for (uint8_t c = 0; c < 16; ++c) {
    const float d = fabsf(f - kE2M1[c]);
    if (d < best_err) {
      best_err = d;
      best = c;
    }
  }
  return best;
}

float or_dec_fp4(uint8_t c) { return kE2M1[c & 15u]; }

uint8_t or_encode(int dtype, float f) {
  switch (dtype) {
  case OR_FP8E4M3: return or_enc_e4m3(f);
  case OR_FP8E5M2: return or_enc_e5m2(f);
  case OR_FP4: return or_enc_fp4(f);
  }
  return 0;
}

float or_decode(int dtype, uint8_t code) {
  switch (dtype) {
  case OR_FP8E4M3: return or_dec_e4m3(code);
  case OR_FP8E5M2: return or_dec_e5m2(code);
  case OR_FP4: return or_dec_fp4(code);
  }
  return NAN;
}

/* ------------------------------------------------------------------------- */
typedef struct {
  int dtype;
  uint32_t first, count;
  int64_t* out;
} sweep_job;

static void* sweep_worker(void* p) {
  sweep_job* j = (sweep_job*)p;
  for (uint32_t c = 0; c < j->count; ++c) {
    const uint32_t chunk = j->first + c;
    int64_t s1 = 0, s2 = 0;
    for (uint32_t i = 0; i < (1u << 20); ++i) {
      const uint32_t u = (chunk << 20) | i;
      const int64_t code = or_encode(j->dtype, u2f(u));
      s1 += code;
      s2 += code * (int64_t)i;
    }
    j->out[2 * (size_t)c] = s1;
    j->out[2 * (size_t)c + 1] = s2;
  }
  return NULL;
}

void or_sweep_digest(int dtype, uint32_t first_chunk, uint32_t n_chunks, int64_t* out,
                     int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if ((uint32_t)nthreads > n_chunks) nthreads = (int)(n_chunks ? n_chunks : 1);
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  sweep_job* jobs = (sweep_job*)calloc((size_t)nthreads, sizeof(sweep_job));
  uint32_t start = 0;
  for (int t = 0; t < nthreads; ++t) {
    const uint32_t cnt = n_chunks / (uint32_t)nthreads + ((uint32_t)t < n_chunks % (uint32_t)nthreads);
    jobs[t].dtype = dtype;
    jobs[t].first = first_chunk + start;
    jobs[t].count = cnt;
    jobs[t].out = out + 2 * (size_t)start;
    start += cnt;
    pthread_create(&th[t], NULL, sweep_worker, &jobs[t]);
  }
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(th);
  free(jobs);
}

/* ------------------------------------------------------------------------- */
/* FormatNone payload (native_codec.cpp:193-211): FP8 one byte per element,   */
/* row-major [out][in]; FP4 two codes per byte over the flattened matrix,     */
/* element i in byte i/2, even i in the low nibble, (n+1)/2 bytes.            */
size_t or_native_bytes(int dtype, int64_t n) {
  return dtype == OR_FP4 ? (size_t)((n + 1) / 2) : (size_t)n;
}

void or_pack(int dtype, const float* w, int64_t n, uint8_t* out) {
  if (dtype != OR_FP4) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_encode(dtype, w[i]);
    return;
  }
  memset(out, 0, (size_t)((n + 1) / 2));
  for (int64_t i = 0; i < n; ++i) {
    const uint8_t c = or_enc_fp4(w[i]) & 15u;
    out[i >> 1] |= (uint8_t)((i & 1) ? (c << 4) : c);
  }
}

/* native_codec.cpp:534-549 */
float or_weight_at(int dtype, const uint8_t* raw, int64_t i) {
  if (dtype == OR_FP4) {
    const uint8_t b = raw[i >> 1];
    return or_dec_fp4((i & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15u));
  }
  return or_decode(dtype, raw[i]);
}

/* ------------------------------------------------------------------------- */
float or_maxrep(int dtype) {
  switch (dtype) {
  case OR_FP8E4M3: return 240.0f;
  case OR_FP8E5M2: return 57344.0f;
  case OR_FP4: return 6.0f;
  }
  return 1.0f;
}

int or_maxrep_ok(int dtype) {
  return dtype == OR_FP8E4M3 || dtype == OR_FP8E5M2 || dtype == OR_FP4;
}

/* Least e in [-127, 127] with amax <= maxrep * 2^e; amax == 0 (or NaN) -> 0. */
int or_e8m0_exponent(float amax, float maxrep) {
  if (!(amax > 0.0f)) return 0;
  if (isinf(amax)) return 127;
  int e = ilogbf(amax) - ilogbf(maxrep) - 1; /* maxrep*2^e < amax here */
  if (e < -127) e = -127;
  while (e < 127 && !(amax <= ldexpf(maxrep, e))) ++e;
  return e;
}

/* Magnitude maximum with the reference's NaN-skipping '>' scan
 * (native_codec.cpp:20-27). */
static float amax_of(const float* w, int64_t n, int64_t stride) {
  float m = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    const float a = fabsf(w[i * stride]);
    if (a > m) m = a;
  }
  return m;
}

static float scale_from_amax(float amax, float maxrep) {
  float s = amax / maxrep;
  if (s == 0.0f) s = 1.0f;
  return s;
}

void or_quantize(int dtype, int scheme, int rows, int cols, const float* W, uint8_t* native,
                 float* row_scale, uint8_t* blk_exp) {
  const int64_t n = (int64_t)rows * cols;
  const float maxrep = or_maxrep(dtype);
  const int nblk = (cols + 31) / 32;
  float* q = (float*)malloc((size_t)n * sizeof(float));
  if (scheme == OR_SCHEME_TENSOR) {
    const float s = scale_from_amax(amax_of(W, n, 1), maxrep);
    for (int r = 0; r < rows; ++r) row_scale[r] = s;
    for (int64_t i = 0; i < n; ++i) q[i] = W[i] / s;
  } else if (scheme == OR_SCHEME_ROW) {
    for (int r = 0; r < rows; ++r) {
      const float* wr = W + (int64_t)r * cols;
      const float s = scale_from_amax(amax_of(wr, cols, 1), maxrep);
      row_scale[r] = s;
      for (int c = 0; c < cols; ++c) q[(int64_t)r * cols + c] = wr[c] / s;
    }
  } else if (scheme == OR_SCHEME_BLOCK32) {
    for (int r = 0; r < rows; ++r) {
      row_scale[r] = 1.0f;
      for (int b = 0; b < nblk; ++b) {
        const int c0 = b * 32, len = (cols - c0) < 32 ? (cols - c0) : 32;
        const float* wb = W + (int64_t)r * cols + c0;
        const int e = or_e8m0_exponent(amax_of(wb, len, 1), maxrep);
        blk_exp[(int64_t)r * nblk + b] = (uint8_t)(e + 127);
        const float inv = ldexpf(1.0f, -e);
        for (int c = 0; c < len; ++c) q[(int64_t)r * cols + c0 + c] = wb[c] * inv;
      }
    }
  } else {
    for (int r = 0; r < rows; ++r) row_scale[r] = 1.0f;
    memcpy(q, W, (size_t)n * sizeof(float));
  }
  or_pack(dtype, q, n, native);
  free(q);
}

void or_dequant(int dtype, int scheme, int rows, int cols, const uint8_t* native,
                const float* row_scale, const uint8_t* blk_exp, float* W_dq) {
  const int nblk = (cols + 31) / 32;
  for (int r = 0; r < rows; ++r) {
    for (int c = 0; c < cols; ++c) {
      const int64_t i = (int64_t)r * cols + c;
      const float d = or_weight_at(dtype, native, i);
      if (scheme == OR_SCHEME_BLOCK32) {
        const int e = (int)blk_exp[(int64_t)r * nblk + c / 32] - 127;
        W_dq[i] = d * ldexpf(1.0f, e);
      } else {
        W_dq[i] = d * row_scale[r];
      }
    }
  }
}

/* ------------------------------------------------------------------------- */
/* activate.cpp:7-29 (ids: activate.hpp:8-17). */
double or_activate(int act, double x) {
  switch (act) {
  case -1: return x;
  case 0: return x < 0.0 ? 0.0 : x;
  case 1: return x / (1.0 + exp(-x));
  case 2: {
    const double k = 0.7978845608028654;
    return 0.5 * x * (1.0 + tanh(k * (x + 0.044715 * x * x * x)));
  }
  case 3: return tanh(x);
  case 4: return 1.0 / (1.0 + exp(-x));
  case 5: return x < 0.0 ? 0.01 * x : x;
  case 6: return x < 0.0 ? 0.0 : x * x;
  }
  return x;
}

typedef struct {
  int batch, in, out, act, bias_len, o0, o1;
  const float* W;
  const double* W64;
  const double* bias;
  const float* x;
  float *pre, *post;
} dense_job;

static void dense_rows(const dense_job* j) {
  const int need_epi = (j->act != -1) || (j->bias != NULL && j->bias_len > 0);
  for (int b = 0; b < j->batch; ++b) {
    const float* xb = j->x + (int64_t)b * j->in;
    for (int o = j->o0; o < j->o1; ++o) {
      double acc = 0.0;
      if (j->W64) {
        const double* wr = j->W64 + (int64_t)o * j->in;
        for (int k = 0; k < j->in; ++k) acc += wr[k] * (double)xb[k];
      } else {
        const float* wr = j->W + (int64_t)o * j->in;
        for (int k = 0; k < j->in; ++k) acc += (double)wr[k] * (double)xb[k];
      }
      const int64_t idx = (int64_t)b * j->out + o;
      float y = (float)acc;
      if (need_epi) {
        double v = (double)y;
        if (j->bias && o < j->bias_len) {
          v += j->bias[o];
          y = (float)v;
        }
        j->pre[idx] = y;
        j->post[idx] = (float)or_activate(j->act, v);
      } else {
        j->pre[idx] = y;
        j->post[idx] = y;
      }
    }
  }
}

static void* dense_worker(void* p) {
  dense_rows((const dense_job*)p);
  return NULL;
}

static void dense_run(dense_job base, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > base.out) nthreads = base.out;
  if (nthreads == 1) {
    base.o0 = 0;
    base.o1 = base.out;
    dense_rows(&base);
    return;
  }
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  dense_job* jobs = (dense_job*)calloc((size_t)nthreads, sizeof(dense_job));
  for (int t = 0; t < nthreads; ++t) {
    jobs[t] = base;
    jobs[t].o0 = (int)((int64_t)base.out * t / nthreads);
    jobs[t].o1 = (int)((int64_t)base.out * (t + 1) / nthreads);
    pthread_create(&th[t], NULL, dense_worker, &jobs[t]);
  }
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(th);
  free(jobs);
}

void or_dense_forward(int batch, int in, int out, int act, const float* W, const double* bias,
                      int bias_len, const float* x, float* pre, float* post, int nthreads) {
  dense_job j;
  memset(&j, 0, sizeof j);
  j.batch = batch;
  j.in = in;
  j.out = out;
  j.act = act;
  j.bias_len = bias_len;
  j.W = W;
  j.bias = bias;
  j.x = x;
  j.pre = pre;
  j.post = post;
  dense_run(j, nthreads);
}

/* kernels.cu:296-304 */
void or_swiglu_product(const float* g, const float* u, float* h, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float silu = (float)or_activate(1, (double)g[i]);
    h[i] = (float)((double)silu * (double)u[i]);
  }
}

/* ------------------------------------------------------------------------- */
/* activate_deriv_dev, kernels.cu:48-81 (activate.cpp:31-63 on the host). */
double or_act_deriv(int act, double x) {
  switch (act) {
  case -1: return 1.0;
  case 0: return x > 0.0 ? 1.0 : 0.0;
  case 6: return x > 0.0 ? 2.0 * x : 0.0;
  case 5: return x > 0.0 ? 1.0 : 0.01;
  case 1: {
    const double sg = 1.0 / (1.0 + exp(-x));
    return sg * (1.0 + x * (1.0 - sg));
  }
  case 2: {
    const double k = 0.7978845608028654;
    const double u = k * (x + 0.044715 * x * x * x);
    const double th = tanh(u);
    const double du = k * (1.0 + 3.0 * 0.044715 * x * x);
    return 0.5 * (1.0 + th) + 0.5 * x * (1.0 - th * th) * du;
  }
  case 3: {
    const double t = tanh(x);
    return 1.0 - t * t;
  }
  case 4: {
    const double sg = 1.0 / (1.0 + exp(-x));
    return sg * (1.0 - sg);
  }
  }
  return 1.0;
}

typedef struct {
  int batch, in, out, i0, i1;
  const float *W, *dpre;
  float* dX;
} matvect_job;

/* dense_matvect_f64_batch, kernels.cu:92-107: columns [i0, i1). */
static void* matvect_cols(void* p) {
  const matvect_job* j = (const matvect_job*)p;
  for (int b = 0; b < j->batch; ++b)
    for (int i = j->i0; i < j->i1; ++i) {
      double sum = 0.0;
      for (int o = 0; o < j->out; ++o)
        sum += (double)j->W[(int64_t)o * j->in + i] * (double)j->dpre[(int64_t)b * j->out + o];
      j->dX[(int64_t)b * j->in + i] = (float)sum;
    }
  return NULL;
}

void or_dense_backward(int batch, int in, int out, int act, const float* W, const float* gy,
                       const float* pre, const float* x, float* dpre, float* dX, float* dW,
                       int nthreads) {
  /* dense_act_deriv, kernels.cu:83-90 */
  for (int64_t i = 0; i < (int64_t)batch * out; ++i)
    dpre[i] = (float)((double)gy[i] * or_act_deriv(act, (double)pre[i]));
  if (nthreads < 1) nthreads = 1;
  if (nthreads > in) nthreads = in;
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  matvect_job* jobs = (matvect_job*)calloc((size_t)nthreads, sizeof(matvect_job));
  for (int t = 0; t < nthreads; ++t) {
    matvect_job j = {batch, in, out, (int)((int64_t)in * t / nthreads),
                     (int)((int64_t)in * (t + 1) / nthreads), W, dpre, dX};
    jobs[t] = j;
    pthread_create(&th[t], NULL, matvect_cols, &jobs[t]);
  }
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(th);
  free(jobs);
  /* dense_outer_f64_batch, kernels.cu:109-127 */
  for (int o = 0; o < out; ++o)
    for (int i = 0; i < in; ++i) {
      float acc = 0.0f;
      for (int b = 0; b < batch; ++b)
        acc = (float)((double)acc + (double)dpre[(int64_t)b * out + o] * (double)x[(int64_t)b * in + i]);
      dW[(int64_t)o * in + i] = acc;
    }
}

/* training.cpp:44-56 */
double or_mse(int64_t n, const float* pred, const float* target) {
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double d = (double)pred[i] - (double)target[i];
    sum += d * d;
  }
  return sum / (double)n;
}

/* training.cpp:58-69 */
void or_mse_grad(int64_t n, const float* pred, const float* target, float* grad) {
  const double scale = 2.0 / (double)n;
  for (int64_t i = 0; i < n; ++i) grad[i] = (float)(scale * ((double)pred[i] - (double)target[i]));
}

/* native_codec.cpp:1123-1127 */
void or_sgd(int64_t n, const float* w, const float* dW, double lr, float* next) {
  for (int64_t i = 0; i < n; ++i) next[i] = (float)((double)w[i] - lr * (double)dW[i]);
}

/* kernels.cu:307-320 */
void or_swiglu_bwd_product(const float* g, const float* u, const float* gh, float* d_up,
                           float* d_gate, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const double gp = (double)g[i];
    const float s = (float)or_activate(1, gp);
    const float ds = (float)or_act_deriv(1, gp);
    const double dh = (double)gh[i], up = (double)u[i];
    d_up[i] = (float)(dh * (double)s);
    d_gate[i] = (float)(dh * up * (double)ds);
  }
}

/* ------------------------------------------------------------------------- */
/* kernels.cu:470-485 */
static int attn_allow(int qp, int kp, int mask, int window, int msl, int prefix_len,
                      int window_causal) {
  if (mask == 2) return 1;
  if (mask == 3) {
    const int w = window > 0 ? window : msl;
    if (window_causal) return kp <= qp && kp >= qp - w + 1;
    const int d = qp > kp ? qp - kp : kp - qp;
    return d < w;
  }
  if (mask == 4) {
    if (qp < prefix_len && kp < prefix_len) return 1;
    return kp <= qp;
  }
  return kp <= qp;
}

/* kernels.cu:487-504: rotate pairs (d, d + hd/2) of every head by pos/theta^(2d/hd). */
static void rope_rotate(double* v, int pos, int heads, int hd, double theta) {
  const int half = hd / 2;
  if (half <= 0 || theta <= 0.0) return;
  for (int h = 0; h < heads; ++h) {
    double* b = v + (int64_t)h * hd;
    for (int d = 0; d < half; ++d) {
      const double ang = (double)pos / pow(theta, (double)(2 * d) / (double)hd);
      const double c = cos(ang), s = sin(ang);
      const double a0 = b[d], a1 = b[d + half];
      b[d] = a0 * c - a1 * s;
      b[d + half] = a0 * s + a1 * c;
    }
  }
}

/* kernels.cu:526-533 */
static double alibi(int head, int heads, int qp, int kp, int on) {
  if (!on) return 0.0;
  const int n = heads > 0 ? heads : 1;
  const double slope = pow(2.0, -(double)(head + 1) * 8.0 / (double)n);
  const int d = qp > kp ? qp - kp : kp - qp;
  return -slope * (double)d;
}

/* The attention of one set of query heads (h = h0, h0 + hstep, ...). Each
 * head's arithmetic is the reference's loop (kernels.cu:536-631) restricted
 * to that head: the ring rows of its KV head and its query rows, rotated per
 * head as the reference rotates them (heads are rotated independently), so
 * the result does not depend on how heads are spread over threads. */
typedef struct {
  const float *q, *k, *v;
  float* attn;
  int batch, seq, num_heads, num_kv, head_dim, msl, mask, pos_kind, softmax_kind, window,
      prefix_len, window_causal;
  double rope_theta, scale_override;
  int h0, hstep;
} attn_job;

static void attn_heads(const attn_job* j) {
  const int batch = j->batch, seq = j->seq, num_heads = j->num_heads, num_kv = j->num_kv;
  const int head_dim = j->head_dim, msl = j->msl;
  const int qd = num_heads * head_dim, kvd = num_kv * head_dim;
  const int per_kv = num_heads / num_kv;
  const double scale = j->scale_override > 0.0 ? j->scale_override : 1.0 / sqrt((double)head_dim);
  const int rope = (j->pos_kind == 0 || j->pos_kind == 3);
  const int use_alibi = (j->pos_kind == 2 || j->pos_kind == 3);
  double* ck = (double*)calloc((size_t)msl * kvd, sizeof(double));
  double* cv = (double*)calloc((size_t)msl * kvd, sizeof(double));
  double* Q = (double*)malloc((size_t)seq * qd * sizeof(double));
  const int64_t max_kv = (int64_t)batch * seq;
  double* sc = (double*)malloc((size_t)max_kv * sizeof(double));
  int* kpos = (int*)malloc((size_t)max_kv * sizeof(int));
  for (int b = 0; b < batch; ++b) {
    const int base = b * seq;
    for (int s = 0; s < seq; ++s) {
      const int pos = base + s;
      const int64_t tok = (int64_t)b * seq + s;
      for (int i = 0; i < qd; ++i) Q[(int64_t)s * qd + i] = (double)j->q[tok * qd + i];
      double* kr = ck + (int64_t)(pos % msl) * kvd;
      double* vr = cv + (int64_t)(pos % msl) * kvd;
      for (int i = 0; i < kvd; ++i) {
        kr[i] = (double)j->k[tok * kvd + i];
        vr[i] = (double)j->v[tok * kvd + i];
      }
      if (rope) {
        for (int h = j->h0; h < num_heads; h += j->hstep)
          rope_rotate(Q + (int64_t)s * qd + (int64_t)h * head_dim, pos, 1, head_dim, j->rope_theta);
        for (int kh = 0; kh < num_kv; ++kh)
          rope_rotate(kr + (int64_t)kh * head_dim, pos, 1, head_dim, j->rope_theta);
      }
    }
    const int kv_len = base + seq;
    for (int s = 0; s < seq; ++s) {
      const int qp = base + s;
      for (int h = j->h0; h < num_heads; h += j->hstep) {
        const int kvh = h / per_kv;
        const double* qv = Q + (int64_t)s * qd + (int64_t)h * head_dim;
        float* out = j->attn + ((int64_t)b * seq + s) * qd + (int64_t)h * head_dim;
        int n = 0;
        double mx = -1e9;
        for (int kp = 0; kp < kv_len; ++kp) {
          if (!attn_allow(qp, kp, j->mask, j->window, msl, j->prefix_len, j->window_causal))
            continue;
          const double* kr = ck + (int64_t)(kp % msl) * kvd + (int64_t)kvh * head_dim;
          double dot = 0.0;
          for (int d = 0; d < head_dim; ++d) dot += qv[d] * kr[d];
          const double score = dot * scale + alibi(h, num_heads, qp, kp, use_alibi);
          sc[n] = score;
          kpos[n] = kp;
          if (score > mx) mx = score;
          ++n;
        }
        if (n == 0) {
          for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
          continue;
        }
        if (j->softmax_kind == 1) {
          for (int i = 0; i < n; ++i) sc[i] = 1.0 / (1.0 + exp(-sc[i]));
        } else {
          double sum = 0.0;
          for (int i = 0; i < n; ++i) {
            sc[i] = exp(sc[i] - mx);
            sum += sc[i];
          }
          const double inv = 1.0 / sum;
          for (int i = 0; i < n; ++i) sc[i] *= inv;
        }
        for (int d = 0; d < head_dim; ++d) {
          double acc = 0.0;
          for (int i = 0; i < n; ++i)
            acc += sc[i] * cv[(int64_t)(kpos[i] % msl) * kvd + (int64_t)kvh * head_dim + d];
          out[d] = (float)acc;
        }
      }
    }
  }
  free(ck);
  free(cv);
  free(Q);
  free(sc);
  free(kpos);
}

static void* attn_worker(void* p) {
  attn_heads((const attn_job*)p);
  return NULL;
}

void or_mha_attention_mt(const float* q, const float* k, const float* v, float* attn, int batch,
                         int seq, int num_heads, int num_kv, int head_dim, int msl, int mask,
                         int pos_kind, int softmax_kind, int window, int prefix_len,
                         int window_causal, double rope_theta, double scale_override,
                         int nthreads) {
  attn_job base = {q, k, v, attn, batch, seq, num_heads, num_kv, head_dim, msl, mask, pos_kind,
                   softmax_kind, window, prefix_len, window_causal, rope_theta, scale_override,
                   0, 1};
  if (nthreads < 1) nthreads = 1;
  if (nthreads > num_heads) nthreads = num_heads;
  if (nthreads == 1) {
    attn_heads(&base);
    return;
  }
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  attn_job* jobs = (attn_job*)calloc((size_t)nthreads, sizeof(attn_job));
  for (int t = 0; t < nthreads; ++t) {
    jobs[t] = base;
    jobs[t].h0 = t;
    jobs[t].hstep = nthreads;
    pthread_create(&th[t], NULL, attn_worker, &jobs[t]);
  }
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(th);
  free(jobs);
}

void or_mha_attention(const float* q, const float* k, const float* v, float* attn, int batch,
                      int seq, int num_heads, int num_kv, int head_dim, int msl, int mask,
                      int pos_kind, int softmax_kind, int window, int prefix_len, int window_causal,
                      double rope_theta, double scale_override) {
  or_mha_attention_mt(q, k, v, attn, batch, seq, num_heads, num_kv, head_dim, msl, mask, pos_kind,
                      softmax_kind, window, prefix_len, window_causal, rope_theta, scale_override,
                      1);
}

/* ------------------------------------------------------------------------- */
static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

double or_cpu_dense_bench(int dtype, int scheme, int batch, int in, int out, const uint8_t* native,
                          const float* row_scale, const uint8_t* blk_exp, const float* x,
                          float* y, int nthreads, int warmup, int iters, double* mount_s) {
  const double t0 = now_s();
  const int64_t n = (int64_t)out * in;
  float* wdq = (float*)malloc((size_t)n * sizeof(float));
  or_dequant(dtype, scheme, out, in, native, row_scale, blk_exp, wdq);
  double* w64 = (double*)malloc((size_t)n * sizeof(double));
  for (int64_t i = 0; i < n; ++i) w64[i] = (double)wdq[i];
  free(wdq);
  if (mount_s) *mount_s = now_s() - t0;
  float* post = (float*)malloc((size_t)batch * out * sizeof(float));
  dense_job j;
  memset(&j, 0, sizeof j);
  j.batch = batch;
  j.in = in;
  j.out = out;
  j.act = -1;
  j.W64 = w64;
  j.x = x;
  j.pre = y;
  j.post = post;
  for (int i = 0; i < warmup; ++i) dense_run(j, nthreads);
  const double t1 = now_s();
  for (int i = 0; i < iters; ++i) dense_run(j, nthreads);
  const double per = (now_s() - t1) / (iters > 0 ? iters : 1);
  free(post);
  free(w64);
  return per;
}
