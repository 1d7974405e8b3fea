/*
 * CPU oracle for the packed block weight formats (QuantFormat).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the library's block-format
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

int or_fmt_quantize(int fmt, int64_t n, const float* x, uint8_t* out) {
  void (*blk)(const float*, uint8_t*) = NULL;
  switch (fmt) {
  case OR_FMT_Q8_0: blk = q8_0_block; break;
  case OR_FMT_Q4_0: blk = q4_0_block; break;
  case OR_FMT_Q4_1: blk = q4_1_block; break;
  case OR_FMT_Q5_0: blk = q5_0_block; break;
  case OR_FMT_Q5_1: blk = q5_1_block; break;
  default: return -1; /* the K formats' quantizers (an rmse search) are not restated */
  }
  if (n % 32) return -1;
  const int bb = or_fmt_block_bytes(fmt);
  for (int64_t b = 0; b < n / 32; ++b) blk(x + 32 * b, out + bb * b);
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

/* ggml's non-linear 4-bit code book of IQ4_NL and IQ4_XS (kvalues_iq4nl). */
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1,    13,   25,  38,  53,  69,  89,  113};

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
