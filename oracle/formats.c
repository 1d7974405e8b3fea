/*
 * CPU oracle for the packed block weight formats (QuantFormat).
 *
 * TEST INFRASTRUCTURE ONLY: the reference for the library's block-format
 * kernels; the product never links or calls it.
 *
 * The reference reserves the QuantFormat enum (include/welvet/weights.hpp:
 * 12-15, "all other quant.Format values from welvet/quant") and lists the
 * formats (README.md:361-383) without implementing any of them; the Go
 * package that defines them is not part of the reference tree. The layouts
 * and rules restated here are ggml's published block formats (llama.cpp
 * ggml-common.h block_q8_0 .. block_q6_K, ggml-quants.c quantize_row_*_ref
 * and dequantize_row_*; GGUF v3 layouts), the de-facto definition of those
 * names. Arithmetic is plain f32 with no contraction (built with
 * -ffp-contract=off), left to right as written below.
 *
 * Format ids follow the README's table order: 1 Q8_0, 2 Q4_0, 3 Q4_1,
 * 4 Q5_0, 5 Q5_1, 6 Q2_K, 7 Q3_K, 8 Q4_K, 9 Q5_K, 10 Q6_K, 16 IQ4_NL,
 * 17 IQ4_XS.
 */
#include <float.h>
#include <math.h>
#include <string.h>

#include "oracle.h"

/* IEEE binary16 -> binary32: exact. */
float or_f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31;
  const int e = (h >> 10) & 0x1F;
  const uint32_t m = h & 0x3FF;
  uint32_t bits;
  if (e == 0x1F) {
    bits = s | 0x7F800000u | (m << 13);
  } else if (e == 0) {
    if (m == 0) {
      bits = s;
    } else {
      /* subnormal: m * 2^-24, exact in f32 */
      float v = (float)m * 0x1p-24f;
      memcpy(&bits, &v, 4);
      bits |= s;
    }
  } else {
    bits = s | ((uint32_t)(e - 15 + 127) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* binary32 -> binary16, round to nearest even; overflow -> inf, NaN -> quiet
 * NaN. */
uint16_t or_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t s = (uint16_t)((u >> 16) & 0x8000);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return s | 0x7E00;
  if (a >= 0x47800000u) {
    /* >= 65536: inf; [65520, 65536) rounds to inf too (handled below) */
    return s | 0x7C00;
  }
  const int e = (int)(a >> 23) - 127;
  if (e < -14) {
    /* subnormal half (or zero): value / 2^-24 rounded to an integer, RNE */
    if (e < -25) return s; /* below half the smallest subnormal */
    const uint32_t m = (a & 0x7FFFFF) | 0x800000; /* 24-bit significand */
    const int shift = -e - 14 + 13;               /* to units of 2^-24 */
    const uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1);
    const uint32_t half = 1u << (shift - 1);
    uint32_t r = q + (rem > half || (rem == half && (q & 1)));
    return s | (uint16_t)r; /* r may carry into the smallest normal: right */
  }
  uint32_t m = a & 0x7FFFFF;
  uint32_t q = ((uint32_t)(e + 15) << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) ++q; /* carries into exponent */
  return s | (uint16_t)q;                                /* 0x7C00 on overflow */
}

int or_fmt_block_elems(int fmt) {
  switch (fmt) {
  case OR_FMT_Q8_0: case OR_FMT_Q4_0: case OR_FMT_Q4_1: case OR_FMT_Q5_0: case OR_FMT_Q5_1:
  case OR_FMT_IQ4_NL:
    return 32;
  case OR_FMT_Q2_K: case OR_FMT_Q3_K: case OR_FMT_Q4_K: case OR_FMT_Q5_K: case OR_FMT_Q6_K:
  case OR_FMT_IQ4_XS:
    return 256;
  default:
    return 0;
  }
}

int or_fmt_block_bytes(int fmt) {
  switch (fmt) {
  case OR_FMT_Q8_0: return 34;  /* f16 d, int8 qs[32] */
  case OR_FMT_Q4_0: return 18;  /* f16 d, qs[16] */
  case OR_FMT_Q4_1: return 20;  /* f16 d, f16 m, qs[16] */
  case OR_FMT_Q5_0: return 22;  /* f16 d, qh[4], qs[16] */
  case OR_FMT_Q5_1: return 24;  /* f16 d, f16 m, qh[4], qs[16] */
  case OR_FMT_Q2_K: return 84;  /* scales[16], qs[64], f16 d, f16 dmin */
  case OR_FMT_Q3_K: return 110; /* hmask[32], qs[64], scales[12], f16 d */
  case OR_FMT_Q4_K: return 144; /* f16 d, f16 dmin, scales[12], qs[128] */
  case OR_FMT_Q5_K: return 176; /* f16 d, f16 dmin, scales[12], qh[32], qs[128] */
  case OR_FMT_Q6_K: return 210; /* ql[128], qh[64], int8 scales[16], f16 d */
  case OR_FMT_IQ4_NL: return 18; /* f16 d, qs[16] (indices into the 16-value table) */
  case OR_FMT_IQ4_XS: return 136; /* f16 d, u16 scales_h, scales_l[4], qs[128] */
  default: return 0;
  }
}

static void put16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
}
static uint16_t get16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static int imin(int a, int b) { return a < b ? a : b; }

/* quantize_row_q8_0_ref: d = amax / 127, q = roundf(x / d) via x * (1/d). */
static void q8_0_block(const float* x, uint8_t* y) {
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put16(y, or_f32_to_f16(d));
  for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

/* The element of largest magnitude (the first one on ties), with its sign. */
static float signed_amax(const float* x) {
  float amax = 0.0f, max = 0.0f;
  for (int j = 0; j < 32; ++j) {
    if (amax < fabsf(x[j])) {
      amax = fabsf(x[j]);
      max = x[j];
    }
  }
  return max;
}

/* quantize_row_q4_0_ref: d = max / -8; q = min(15, (int8)(x / d + 8.5));
 * element j in the low nibble of qs[j], element j + 16 in the high one. */
static void q4_0_block(const float* x, uint8_t* y) {
  const float max = signed_amax(x);
  const float d = max / -8.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put16(y, or_f32_to_f16(d));
  for (int j = 0; j < 16; ++j) {
    const int q0 = imin(15, (int8_t)(x[j] * id + 8.5f));
    const int q1 = imin(15, (int8_t)(x[16 + j] * id + 8.5f));
    y[2 + j] = (uint8_t)(q0 | (q1 << 4));
  }
}

/* quantize_row_q4_1_ref: d = (max - min) / 15, m = min;
 * q = min(15, (int8)((x - min) / d + 0.5)). */
static void q4_1_block(const float* x, uint8_t* y) {
  float mn = FLT_MAX, mx = -FLT_MAX;
  for (int j = 0; j < 32; ++j) {
    if (x[j] < mn) mn = x[j];
    if (x[j] > mx) mx = x[j];
  }
  const float d = (mx - mn) / 15.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put16(y, or_f32_to_f16(d));
  put16(y + 2, or_f32_to_f16(mn));
  for (int j = 0; j < 16; ++j) {
    const int q0 = imin(15, (int8_t)((x[j] - mn) * id + 0.5f));
    const int q1 = imin(15, (int8_t)((x[16 + j] - mn) * id + 0.5f));
    y[4 + j] = (uint8_t)(q0 | (q1 << 4));
  }
}

/* quantize_row_q5_0_ref: d = max / -16; q = min(31, (int8)(x / d + 16.5));
 * low 4 bits as Q4_0, bit 4 of element e in bit e of the little-endian qh. */
static void q5_0_block(const float* x, uint8_t* y) {
  const float max = signed_amax(x);
  const float d = max / -16.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put16(y, or_f32_to_f16(d));
  uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    const int q0 = imin(31, (int8_t)(x[j] * id + 16.5f));
    const int q1 = imin(31, (int8_t)(x[16 + j] * id + 16.5f));
    y[6 + j] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
    qh |= (uint32_t)((q0 & 0x10) >> 4) << j;
    qh |= (uint32_t)((q1 & 0x10) >> 4) << (j + 16);
  }
  memcpy(y + 2, &qh, 4);
}

/* quantize_row_q5_1_ref: d = (max - min) / 31, m = min;
 * q = (uint8)((x - min) / d + 0.5). */
static void q5_1_block(const float* x, uint8_t* y) {
  float mn = FLT_MAX, mx = -FLT_MAX;
  for (int j = 0; j < 32; ++j) {
    if (x[j] < mn) mn = x[j];
    if (x[j] > mx) mx = x[j];
  }
  const float d = (mx - mn) / 31.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put16(y, or_f32_to_f16(d));
  put16(y + 2, or_f32_to_f16(mn));
  uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    const int q0 = (uint8_t)((x[j] - mn) * id + 0.5f);
    const int q1 = (uint8_t)((x[16 + j] - mn) * id + 0.5f);
    y[8 + j] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
    qh |= (uint32_t)((q0 & 0x10) >> 4) << j;
    qh |= (uint32_t)((q1 & 0x10) >> 4) << (j + 16);
  }
  memcpy(y + 4, &qh, 4);
}

/* ggml's non-linear 4-bit code book of IQ4_NL and IQ4_XS (kvalues_iq4nl). */
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1,    13,   25,  38,  53,  69,  89,  113};

/* ---- The library's quantizers of the K and IQ4 formats.
 * ggml's own (make_qkx2_quants, make_q3_quants, make_qx_quants and the IQ4
 * scale search) refine the scales with a weighted least-squares search;
 * ggml is not in this image, so these are the library's own one-pass
 * quantizers into the same block layouts (the restatement of the device
 * code in formats.hip, which must give the same bytes):
 *  - affine formats (Q2_K, Q4_K, Q5_K): per sub-block, scale = (max - mn) /
 *    qmax and offset = -mn with mn = min(0, min); the super-block's scales
 *    and offsets are quantized to lmax levels of d = max scale / lmax and
 *    dmin = max offset / lmax; codes q = round((x + dmin * lm) / (d * ls));
 *  - signed formats (Q3_K, Q6_K): per sub-block s = m / qdiv with m the
 *    element of largest magnitude (so m takes the code qdiv exactly); the
 *    super-block's scales are integers of d = ms / ldiv, ms the s of largest
 *    magnitude; q = round(x / (d * l));
 *  - IQ4_NL / IQ4_XS: the scale maps the element of largest magnitude to
 *    the code book's -127 (IQ4_XS: per sub-block, with the 6-bit integer
 *    scales of d = ms / -32); each element takes the nearest code-book entry
 *    (the first on ties).
 * d and dmin are rounded to f16 before the codes are chosen, so the codes fit
 * the stored scales. Plain f32 arithmetic in the order written, no
 * contraction. */
static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
static float f16r(float v) { return or_f16_to_f32(or_f32_to_f16(v)); }
/* nearest integer of v clamped to [lo, hi] (half away from zero) */
static int qround(float v, int lo, int hi) {
  return clampi((int)roundf(fminf(fmaxf(v, (float)lo), (float)hi)), lo, hi);
}
static float signed_amax_n(const float* x, int n) {
  float amax = 0.0f, max = 0.0f;
  for (int j = 0; j < n; ++j) {
    if (amax < fabsf(x[j])) {
      amax = fabsf(x[j]);
      max = x[j];
    }
  }
  return max;
}

/* Affine super-block: nsub sub-blocks of sub elements; qmax code levels,
 * lmax scale / offset levels. ls, lm: integer scales and offsets; q: codes;
 * d, dmin: the f32 super-block scales (stored as f16). */
static void affine_k(const float* x, int nsub, int sub, int qmax, int lmax, int* ls, int* lm,
                     int* q, float* d, float* dmin) {
  float scale[16], off[16];
  float max_scale = 0.0f, max_off = 0.0f;
  for (int j = 0; j < nsub; ++j) {
    const float* v = x + sub * j;
    float mn = v[0], mx = v[0];
    for (int i = 1; i < sub; ++i) {
      mn = v[i] < mn ? v[i] : mn;
      mx = v[i] > mx ? v[i] : mx;
    }
    /* the offset is -min(min, 0); comparisons, not fmaxf, so that an all-zero
     * or constant sub-block gives +0 (fmaxf may return either signed zero) */
    off[j] = mn < 0.0f ? -mn : 0.0f;
    scale[j] = (mx + off[j]) / (float)qmax;
    if (scale[j] > max_scale) max_scale = scale[j];
    if (off[j] > max_off) max_off = off[j];
  }
  const float inv_s = max_scale > 0.0f ? (float)lmax / max_scale : 0.0f;
  const float inv_m = max_off > 0.0f ? (float)lmax / max_off : 0.0f;
  *d = max_scale / (float)lmax;
  *dmin = max_off / (float)lmax;
  const float dd = f16r(*d), dm = f16r(*dmin);
  for (int j = 0; j < nsub; ++j) {
    ls[j] = qround(inv_s * scale[j], 0, lmax);
    lm[j] = qround(inv_m * off[j], 0, lmax);
    const float ds = dd * (float)ls[j];
    const float dmn = dm * (float)lm[j];
    const float id = ds > 0.0f ? 1.0f / ds : 0.0f;
    for (int i = 0; i < sub; ++i) q[sub * j + i] = qround((x[sub * j + i] + dmn) * id, 0, qmax);
  }
}

/* Signed super-block: sub-block scales m / qdiv as integers of d = ms / ldiv
 * in [lmin, lmax]; codes in [qlo, qhi]. */
static void signed_k(const float* x, int nsub, int sub, float qdiv, int qlo, int qhi, float ldiv,
                     int lmin, int lmax, int* l, int* q, float* d) {
  float s[16];
  for (int j = 0; j < nsub; ++j) s[j] = signed_amax_n(x + sub * j, sub) / qdiv;
  const float ms = signed_amax_n(s, nsub);
  *d = ms / ldiv;
  const float id = *d != 0.0f ? 1.0f / *d : 0.0f;
  const float dd = f16r(*d);
  for (int j = 0; j < nsub; ++j) {
    l[j] = qround(s[j] * id, lmin, lmax);
    const float ds = dd * (float)l[j];
    const float is = ds != 0.0f ? 1.0f / ds : 0.0f;
    for (int i = 0; i < sub; ++i) q[sub * j + i] = qround(x[sub * j + i] * is, qlo, qhi);
  }
}

/* index of the code-book entry nearest t (the first on ties) */
static int iq4_index(float t) {
  int best = 0;
  float err = fabsf(t - (float)kIq4nl[0]);
  for (int k = 1; k < 16; ++k) {
    const float e = fabsf(t - (float)kIq4nl[k]);
    if (e < err) {
      err = e;
      best = k;
    }
  }
  return best;
}

static void q4k_block(const float* x, uint8_t* y, int k5) {
  int ls[8], lm[8], q[256];
  float d, dmin;
  affine_k(x, 8, 32, k5 ? 31 : 15, 63, ls, lm, q, &d, &dmin);
  memset(y, 0, k5 ? 176 : 144);
  put16(y, or_f32_to_f16(d));
  put16(y + 2, or_f32_to_f16(dmin));
  uint8_t* sc = y + 4;
  for (int j = 0; j < 8; ++j) {
    if (j < 4) {
      sc[j] |= (uint8_t)(ls[j] & 63);
      sc[j + 4] |= (uint8_t)(lm[j] & 63);
    } else {
      sc[j + 4] = (uint8_t)((ls[j] & 15) | ((lm[j] & 15) << 4));
      sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
      sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
    }
  }
  uint8_t* qh = y + 16;
  uint8_t* qs = y + (k5 ? 48 : 16);
  for (int i = 0; i < 4; ++i)
    for (int l = 0; l < 32; ++l) {
      const int a = q[64 * i + l], b = q[64 * i + 32 + l];
      qs[32 * i + l] = (uint8_t)((a & 15) | ((b & 15) << 4));
      if (k5) qh[l] |= (uint8_t)(((a >> 4) << (2 * i)) | ((b >> 4) << (2 * i + 1)));
    }
}
static void q4_k_block(const float* x, uint8_t* y) { q4k_block(x, y, 0); }
static void q5_k_block(const float* x, uint8_t* y) { q4k_block(x, y, 1); }

static void q2_k_block(const float* x, uint8_t* y) {
  int ls[16], lm[16], q[256];
  float d, dmin;
  affine_k(x, 16, 16, 3, 15, ls, lm, q, &d, &dmin);
  memset(y, 0, 84);
  for (int j = 0; j < 16; ++j) y[j] = (uint8_t)(ls[j] | (lm[j] << 4));
  for (int n = 0; n < 2; ++n)
    for (int j = 0; j < 4; ++j)
      for (int l = 0; l < 32; ++l) y[16 + 32 * n + l] |= (uint8_t)(q[128 * n + 32 * j + l] << (2 * j));
  put16(y + 80, or_f32_to_f16(d));
  put16(y + 82, or_f32_to_f16(dmin));
}

static void q3_k_block(const float* x, uint8_t* y) {
  int l[16], q[256];
  float d;
  signed_k(x, 16, 16, -4.0f, -4, 3, -32.0f, -32, 31, l, q, &d);
  memset(y, 0, 110);
  uint8_t* hm = y;
  uint8_t* qs = y + 32;
  uint8_t* sc = y + 96;
  for (int n = 0; n < 2; ++n)
    for (int j = 0; j < 4; ++j)
      for (int i = 0; i < 32; ++i) {
        const int v = q[128 * n + 32 * j + i] + 4;
        qs[32 * n + i] |= (uint8_t)((v & 3) << (2 * j));
        hm[i] |= (uint8_t)((v >> 2) << (4 * n + j));
      }
  for (int s = 0; s < 16; ++s) {
    const int v = l[s] + 32, g = s >> 2, i = s & 3;
    sc[(g & 1) * 4 + i] |= (uint8_t)((v & 15) << ((g >> 1) * 4));
    sc[8 + i] |= (uint8_t)((v >> 4) << (2 * g));
  }
  put16(y + 108, or_f32_to_f16(d));
}

static void q6_k_block(const float* x, uint8_t* y) {
  int l[16], q[256];
  float d;
  signed_k(x, 16, 16, -32.0f, -32, 31, -128.0f, -128, 127, l, q, &d);
  memset(y, 0, 210);
  uint8_t* ql = y;
  uint8_t* qh = y + 128;
  for (int n = 0; n < 2; ++n)
    for (int t = 0; t < 4; ++t)
      for (int i = 0; i < 32; ++i) {
        const int v = q[128 * n + 32 * t + i] + 32;
        ql[64 * n + 32 * (t & 1) + i] |= (uint8_t)((v & 15) << (4 * (t >> 1)));
        qh[32 * n + i] |= (uint8_t)((v >> 4) << (2 * t));
      }
  for (int s = 0; s < 16; ++s) y[192 + s] = (uint8_t)(int8_t)l[s];
  put16(y + 208, or_f32_to_f16(d));
}

/* the 32 code-book indices of one sub-block at scale ds into qs[16] */
static void iq4_sub(const float* x, float ds, uint8_t* qs) {
  const float id = ds != 0.0f ? 1.0f / ds : 0.0f;
  for (int j = 0; j < 16; ++j)
    qs[j] = (uint8_t)(iq4_index(x[j] * id) | (iq4_index(x[16 + j] * id) << 4));
}

static void iq4_nl_block(const float* x, uint8_t* y) {
  const float d = signed_amax_n(x, 32) / -127.0f;
  put16(y, or_f32_to_f16(d));
  iq4_sub(x, f16r(d), y + 2);
}

static void iq4_xs_block(const float* x, uint8_t* y) {
  float s[8];
  for (int j = 0; j < 8; ++j) s[j] = signed_amax_n(x + 32 * j, 32) / -127.0f;
  const float ms = signed_amax_n(s, 8);
  const float d = ms / -32.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const float dd = f16r(d);
  memset(y, 0, 136);
  put16(y, or_f32_to_f16(d));
  int sh = 0;
  for (int j = 0; j < 8; ++j) {
    const int l = qround(s[j] * id, -32, 31);
    const int ls = l + 32;
    y[4 + j / 2] |= (uint8_t)((ls & 15) << (4 * (j & 1)));
    sh |= (ls >> 4) << (2 * j);
    iq4_sub(x + 32 * j, dd * (float)l, y + 8 + 16 * j);
  }
  put16(y + 2, (uint16_t)sh);
}

int or_fmt_quantize(int fmt, int64_t n, const float* x, uint8_t* out) {
  void (*blk)(const float*, uint8_t*) = NULL;
  switch (fmt) {
  case OR_FMT_Q8_0: blk = q8_0_block; break;
  case OR_FMT_Q4_0: blk = q4_0_block; break;
  case OR_FMT_Q4_1: blk = q4_1_block; break;
  case OR_FMT_Q5_0: blk = q5_0_block; break;
  case OR_FMT_Q5_1: blk = q5_1_block; break;
  case OR_FMT_Q2_K: blk = q2_k_block; break;
  case OR_FMT_Q3_K: blk = q3_k_block; break;
  case OR_FMT_Q4_K: blk = q4_k_block; break;
  case OR_FMT_Q5_K: blk = q5_k_block; break;
  case OR_FMT_Q6_K: blk = q6_k_block; break;
  case OR_FMT_IQ4_NL: blk = iq4_nl_block; break;
  case OR_FMT_IQ4_XS: blk = iq4_xs_block; break;
  default: return -1;
  }
  const int qk = or_fmt_block_elems(fmt);
  if (n % qk) return -1;
  const int bb = or_fmt_block_bytes(fmt);
  for (int64_t b = 0; b < n / qk; ++b) blk(x + qk * b, out + bb * b);
  return 0;
}

/* get_scale_min_k4: 6-bit scale and min of sub-block j (0..7) from the 12
 * packed bytes of a Q4_K/Q5_K super-block. */
static void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

/* The 16 6-bit scales of a Q3_K super-block from its 12 packed bytes, as
 * signed values (scale - 32): scale s = 4 g + i takes the low (g = 0, 1) or
 * high (g = 2, 3) nibble of byte i (g even) or byte 4 + i (g odd), and bits
 * 4-5 from bits 2g, 2g + 1 of byte 8 + i. */
static int scale_q3k(int s, const uint8_t* q) {
  const int g = s >> 2, i = s & 3;
  const int lo = (q[(g & 1) * 4 + i] >> ((g >> 1) * 4)) & 0xF;
  const int hi = (q[8 + i] >> (2 * g)) & 3;
  return (lo | (hi << 4)) - 32;
}


static void dequant_block(int fmt, const uint8_t* b, float* y) {
  switch (fmt) {
  case OR_FMT_Q8_0: { /* y = q * d */
    const float d = or_f16_to_f32(get16(b));
    for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
    break;
  }
  case OR_FMT_Q4_0: { /* y = (q - 8) * d */
    const float d = or_f16_to_f32(get16(b));
    for (int j = 0; j < 16; ++j) {
      y[j] = (float)((b[2 + j] & 0x0F) - 8) * d;
      y[j + 16] = (float)((b[2 + j] >> 4) - 8) * d;
    }
    break;
  }
  case OR_FMT_Q4_1: { /* y = q * d + m */
    const float d = or_f16_to_f32(get16(b)), m = or_f16_to_f32(get16(b + 2));
    for (int j = 0; j < 16; ++j) {
      y[j] = (float)(b[4 + j] & 0x0F) * d + m;
      y[j + 16] = (float)(b[4 + j] >> 4) * d + m;
    }
    break;
  }
  case OR_FMT_Q5_0: { /* y = (q - 16) * d */
    const float d = or_f16_to_f32(get16(b));
    uint32_t qh;
    memcpy(&qh, b + 2, 4);
    for (int j = 0; j < 16; ++j) {
      const int h0 = ((qh >> j) << 4) & 0x10, h1 = (qh >> (j + 12)) & 0x10;
      y[j] = (float)(((b[6 + j] & 0x0F) | h0) - 16) * d;
      y[j + 16] = (float)(((b[6 + j] >> 4) | h1) - 16) * d;
    }
    break;
  }
  case OR_FMT_Q5_1: { /* y = q * d + m */
    const float d = or_f16_to_f32(get16(b)), m = or_f16_to_f32(get16(b + 2));
    uint32_t qh;
    memcpy(&qh, b + 4, 4);
    for (int j = 0; j < 16; ++j) {
      const int h0 = ((qh >> j) << 4) & 0x10, h1 = (qh >> (j + 12)) & 0x10;
      y[j] = (float)((b[8 + j] & 0x0F) | h0) * d + m;
      y[j + 16] = (float)((b[8 + j] >> 4) | h1) * d + m;
    }
    break;
  }
  case OR_FMT_Q4_K: case OR_FMT_Q5_K: {
    /* 8 sub-blocks of 32: y = (d * sc) * q - (dmin * m); sub-block 2i takes
     * the low nibbles of qs[32i .. 32i + 31], 2i + 1 the high ones; Q5_K adds
     * 16 when bit (sub-block) of qh[l] is set */
    const int k5 = fmt == OR_FMT_Q5_K;
    const float d = or_f16_to_f32(get16(b)), dmin = or_f16_to_f32(get16(b + 2));
    const uint8_t* sc = b + 4;
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + (k5 ? 48 : 16);
    for (int i = 0; i < 4; ++i) {
      int s0, m0, s1, m1;
      scale_min_k4(2 * i, sc, &s0, &m0);
      scale_min_k4(2 * i + 1, sc, &s1, &m1);
      const float d1 = d * (float)s0, mm1 = dmin * (float)m0;
      const float d2 = d * (float)s1, mm2 = dmin * (float)m1;
      for (int l = 0; l < 32; ++l) {
        const int hi0 = k5 && ((qh[l] >> (2 * i)) & 1) ? 16 : 0;
        const int hi1 = k5 && ((qh[l] >> (2 * i + 1)) & 1) ? 16 : 0;
        y[64 * i + l] = d1 * (float)((qs[32 * i + l] & 0xF) + hi0) - mm1;
        y[64 * i + 32 + l] = d2 * (float)((qs[32 * i + l] >> 4) + hi1) - mm2;
      }
    }
    break;
  }
  case OR_FMT_Q2_K: {
    /* element 128 n + 32 j + l: 2-bit code j of qs[32 n + l] (bits 2j, 2j+1),
     * scale byte sc = scales[8 n + 2 j + l / 16]:
     * y = (d * (sc & 15)) * q - (dmin * (sc >> 4)) */
    const uint8_t* sc = b;
    const uint8_t* qs = b + 16;
    const float d = or_f16_to_f32(get16(b + 80)), dmin = or_f16_to_f32(get16(b + 82));
    for (int n = 0; n < 2; ++n)
      for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) {
          const int s = sc[8 * n + 2 * j + l / 16];
          const float dl = d * (float)(s & 15), ml = dmin * (float)(s >> 4);
          const int q = (qs[32 * n + l] >> (2 * j)) & 3;
          y[128 * n + 32 * j + l] = dl * (float)q - ml;
        }
    break;
  }
  case OR_FMT_Q3_K: {
    /* element 128 n + 32 j + l: low bits from bits 2j, 2j+1 of qs[32 n + l],
     * minus 4 unless bit 4n + j of hmask[l] is set; scale 8 n + 2 j + l / 16:
     * y = (d * scale) * q */
    const uint8_t* hm = b;
    const uint8_t* qs = b + 32;
    const uint8_t* sc = b + 96;
    const float d = or_f16_to_f32(get16(b + 108));
    for (int n = 0; n < 2; ++n)
      for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) {
          const float dl = d * (float)scale_q3k(8 * n + 2 * j + l / 16, sc);
          const int lo = (qs[32 * n + l] >> (2 * j)) & 3;
          const int q = lo - (((hm[l] >> (4 * n + j)) & 1) ? 0 : 4);
          y[128 * n + 32 * j + l] = dl * (float)q;
        }
    break;
  }
  case OR_FMT_IQ4_NL: { /* y = d * table[index]; element j low nibble of qs[j], j + 16 high */
    const float d = or_f16_to_f32(get16(b));
    for (int j = 0; j < 16; ++j) {
      y[j] = d * (float)kIq4nl[b[2 + j] & 15];
      y[j + 16] = d * (float)kIq4nl[b[2 + j] >> 4];
    }
    break;
  }
  case OR_FMT_IQ4_XS: {
    /* 8 sub-blocks of 32: 6-bit scale ls = nibble (ib & 1) of scales_l[ib / 2]
     * | bits 2ib, 2ib+1 of scales_h << 4; y = (d * (ls - 32)) * table[index],
     * indices of sub-block ib in qs[16 ib ..] as IQ4_NL */
    const float d = or_f16_to_f32(get16(b));
    const int sh = get16(b + 2);
    for (int ib = 0; ib < 8; ++ib) {
      const int ls = ((b[4 + ib / 2] >> (4 * (ib & 1))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
      const float dl = d * (float)(ls - 32);
      const uint8_t* qs = b + 8 + 16 * ib;
      for (int j = 0; j < 16; ++j) {
        y[32 * ib + j] = dl * (float)kIq4nl[qs[j] & 15];
        y[32 * ib + j + 16] = dl * (float)kIq4nl[qs[j] >> 4];
      }
    }
    break;
  }
  case OR_FMT_Q6_K: {
    /* two halves of 128: element 128n + 32t + l has low 4 bits from
     * ql[64n + 32(t & 1) + l] (nibble t >> 1), high 2 bits from bits 2t..2t+1
     * of qh[32n + l]; y = (d * sc[8n + 2t + l / 16]) * (q - 32) */
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = or_f16_to_f32(get16(b + 208));
    for (int n = 0; n < 2; ++n)
      for (int t = 0; t < 4; ++t)
        for (int l = 0; l < 32; ++l) {
          const int lo = (ql[64 * n + 32 * (t & 1) + l] >> (4 * (t >> 1))) & 0xF;
          const int hi = (qh[32 * n + l] >> (2 * t)) & 3;
          const int q = (lo | (hi << 4)) - 32;
          y[128 * n + 32 * t + l] = d * (float)sc[8 * n + 2 * t + l / 16] * (float)q;
        }
    break;
  }
  default: break;
  }
}

int or_fmt_dequant(int fmt, int64_t n, const uint8_t* in, float* out) {
  const int qk = or_fmt_block_elems(fmt), bb = or_fmt_block_bytes(fmt);
  if (!qk || n % qk) return -1;
  for (int64_t b = 0; b < n / qk; ++b) dequant_block(fmt, in + bb * b, out + qk * b);
  return 0;
}
