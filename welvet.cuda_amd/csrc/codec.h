// FP8 (E4M3 / E5M2) and FP4 (E2M1) element codecs with the reference's
// rounding and special-value rules, usable from host and device code.
//
// Reference semantics (src/core/float_codecs.cpp):
//   E4M3 encode :57-97  — ties away from zero on one guard bit, truncated
//                         subnormals, |x| in [248, inf] -> 448 (0x7E), NaN -> 0.
//   E4M3 decode :99-117 — subnormal codes decode to signed zero, 0x7F -> 448.
//   E5M2 encode :119-158 — ties away, flush below 2^-14, overflow -> inf, NaN -> 0x7E.
//   E5M2 decode :160-182 — subnormal codes decode to signed zero.
//   FP4 encode  :184-198 — first table entry with strictly smallest f32 |x - v|.
//
// The encoders here work on the f32 bit pattern with integer operations, so
// they do not depend on the device's denormal mode. The rounding carry is
// taken by adding one to the (exponent|mantissa) field, which carries into the
// exponent exactly as the reference's explicit carry does.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define WV_HD __host__ __device__ inline __attribute__((always_inline))
#else
#define WV_HD inline
#endif

namespace wv {

enum DType : int32_t { kE4M3 = 4, kE5M2 = 5, kFP4 = 16 };
enum Scheme : int32_t { kSchemeRef = 0, kSchemeTensor = 1, kSchemeRow = 2, kSchemeBlock32 = 3 };

WV_HD uint32_t bits_of(float f) {
  union {
    float f;
    uint32_t u;
  } c;
  c.f = f;
  return c.u;
}
WV_HD float float_of(uint32_t u) {
  union {
    float f;
    uint32_t u;
  } c;
  c.u = u;
  return c.f;
}

WV_HD uint8_t encode_e4m3(float f) {
  const uint32_t u = bits_of(f);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a == 0u || a > 0x7F800000u) return 0x00;       // +-0 and NaN
  const uint32_t s = (u >> 24) & 0x80u;
  if (a > 0x43E00000u) return (uint8_t)(s | 0x7Eu);  // |f| > 448, incl. inf
  const int E = (int)(a >> 23) - 120;                // exponent rebiased to 7
  if (E <= 0) {
    if (E < -2) return (uint8_t)s;
    const uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
    return (uint8_t)(s | ((sig >> (uint32_t)(21 - E)) & 7u));
  }
  if (E >= 15) return (uint8_t)(s | 0x7Eu);
  uint32_t field = ((uint32_t)E << 3) | ((a >> 20) & 7u);
  field += (a >> 19) & 1u;                           // half-away, carry into E
  if (field >= (15u << 3)) return (uint8_t)(s | 0x7Eu);
  return (uint8_t)(s | field);
}

WV_HD float decode_e4m3(uint8_t b) {
  const uint32_t s = (uint32_t)(b & 0x80u) << 24;
  const uint32_t field = b & 0x7Fu;
  if (field < 8u) return float_of(s);                // exponent 0: signed zero
  if (field == 0x7Fu) return float_of(s | 0x43E00000u);
  return float_of(s | ((field << 20) + (120u << 23)));
}

WV_HD uint8_t encode_e5m2(float f) {
  const uint32_t u = bits_of(f);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return 0x7E;                  // NaN
  const uint32_t s = (u >> 24) & 0x80u;              // -0 keeps its sign
  if (a == 0x7F800000u) return (uint8_t)(s | 0x7Cu);
  const int E = (int)(a >> 23) - 112;                // exponent rebiased to 15
  if (E <= 0) return (uint8_t)s;                     // zero and flush range
  if (E >= 31) return (uint8_t)(s | 0x7Cu);
  uint32_t field = ((uint32_t)E << 2) | ((a >> 21) & 3u);
  field += (a >> 20) & 1u;
  if (field >= (31u << 2)) return (uint8_t)(s | 0x7Cu);
  return (uint8_t)(s | field);
}

WV_HD float decode_e5m2(uint8_t b) {
  const uint32_t s = (uint32_t)(b & 0x80u) << 24;
  const uint32_t field = b & 0x7Fu;
  if (field < 4u) return float_of(s);
  if (field >= 0x7Cu) return float_of(s | (field == 0x7Cu ? 0x7F800000u : 0x7FC00000u));
  return float_of(s | ((field << 21) + (112u << 23)));
}

// Magnitudes of E2M1 codes 0..7; codes 8..15 are the negatives.
WV_HD float fp4_magnitude(uint32_t c) {
  // 0, .5, 1, 1.5, 2, 3, 4, 6 — built from bits to stay constexpr-free on device.
  const uint32_t tbl[8] = {0x00000000u, 0x3F000000u, 0x3F800000u, 0x3FC00000u,
                           0x40000000u, 0x40400000u, 0x40800000u, 0x40C00000u};
  return float_of(tbl[c & 7u]);
}

// Nearest magnitude searched in table order with a strict '<' from FLT_MAX,
// using the same f32 differences as the reference. For negative inputs the
// reference visits the positive entries first, whose errors are never
// strictly smaller than |x| (the error of code 0), so only code 0 and the
// negative entries 9..15 can win; by symmetry their errors equal those of the
// positive entries for |x|.
WV_HD uint8_t encode_fp4(float f) {
  const uint32_t u = bits_of(f);
  const float m = float_of(u & 0x7FFFFFFFu);
  float best_err = float_of(0x7F7FFFFFu);
  uint32_t best = 0;
  for (uint32_t c = 0; c < 8u; ++c) {
    float d = m - fp4_magnitude(c);
    d = float_of(bits_of(d) & 0x7FFFFFFFu);
    if (d < best_err) {
      best_err = d;
      best = c;
    }
  }
  const bool neg = f < 0.0f;
  return (uint8_t)((neg && best != 0u) ? (best | 8u) : best);
}

WV_HD float decode_fp4(uint8_t c) {
  const float m = fp4_magnitude(c);
  return (c & 8u) ? -m : m;
}

WV_HD uint8_t encode(int dtype, float f) {
  return dtype == kE4M3 ? encode_e4m3(f) : dtype == kE5M2 ? encode_e5m2(f) : encode_fp4(f);
}

WV_HD float decode(int dtype, uint8_t c) {
  return dtype == kE4M3 ? decode_e4m3(c) : dtype == kE5M2 ? decode_e5m2(c) : decode_fp4(c);
}

// Device-operand canonical form: a code with the same reference value whose
// OCP hardware interpretation (gfx950 cvt / MFMA) is that value. E4M3:
// exponent-0 codes -> signed zero, 0x7F/0xFF -> 0x7E/0xFE. E5M2: exponent-0
// codes -> signed zero. FP4 already agrees.
WV_HD uint8_t canonical(int dtype, uint8_t c) {
  if (dtype == kE4M3) {
    if ((c & 0x78u) == 0u) return (uint8_t)(c & 0x80u);
    if ((c & 0x7Fu) == 0x7Fu) return (uint8_t)(c - 1u);
    return c;
  }
  if (dtype == kE5M2) {
    if ((c & 0x7Cu) == 0u) return (uint8_t)(c & 0x80u);
    return c;
  }
  return (uint8_t)(c & 15u);
}

// Largest value a scaled code may take before the reference encoder
// saturates: E4M3 240 (inputs >= 248 jump to 448), E5M2 57344, FP4 6.
WV_HD float max_representable(int dtype) {
  return dtype == kE4M3 ? 240.0f : dtype == kE5M2 ? 57344.0f : 6.0f;
}

// Per-tensor / per-row scale: amax / maxrep, with 0 -> 1.
WV_HD float scale_for(float amax, float maxrep) {
  const float s = amax / maxrep;
  return s == 0.0f ? 1.0f : s;
}

// Least e in [-127, 127] with amax <= maxrep * 2^e (amax == 0 or NaN -> 0;
// inf -> 127). With amax = A * 2^qa and maxrep = R * 2^qr (A, R in [1, 2)),
// the answer is qa - qr + (A > R), clamped. Written without branches (it
// runs per block in the activation split). A subnormal amax (below 2^-126)
// gives at most -126 - qr, which clamps to -127 for every maxrep >= 2 (the
// FP8 / FP4 maxima), so its significand is never normalized.
WV_HD int e8m0_exponent(float amax, float maxrep) {
  const uint32_t a = bits_of(amax) & 0x7FFFFFFFu;
  const uint32_t r = bits_of(maxrep);
  int e = (int)(a >> 23) - (int)(r >> 23) + ((a & 0x7FFFFFu) > (r & 0x7FFFFFu) ? 1 : 0);
  e = e < -127 ? -127 : e > 127 ? 127 : e;
  e = a == 0x7F800000u ? 127 : e;
  return a == 0u || a > 0x7F800000u ? 0 : e;
}

// 2^e as f32 for e in [-127, 127] (2^-127 is the subnormal 0x00400000).
WV_HD float pow2f(int e) {
  return e >= -126 ? float_of((uint32_t)(e + 127) << 23) : float_of(0x00400000u);
}

}  // namespace wv
