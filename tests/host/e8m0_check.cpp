// Host build of the library's E8M0 block-exponent rule (codec.h) checked
// against the oracle's or_e8m0_exponent over non-negative f32 patterns:
// every pattern when the first argument is "all", else every 61st pattern
// plus the 256 powers of two and their neighbours. Prints the first
// mismatch and exits 1, or prints the count checked.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "codec.h"

extern "C" int or_e8m0_exponent(float amax, float maxrep);

static int check(uint32_t a, float maxrep) {
  const float f = wv::float_of(a);
  const int got = wv::e8m0_exponent(f, maxrep), want = or_e8m0_exponent(f, maxrep);
  if (got != want) {
    printf("mismatch: amax bits 0x%08x maxrep %g: %d, oracle %d\n", a, maxrep, got, want);
    return 1;
  }
  return 0;
}

int main(int argc, char** argv) {
  const bool all = argc > 1 && strcmp(argv[1], "all") == 0;
  const float reps[] = {448.0f, 240.0f, 57344.0f, 6.0f};
  uint64_t n = 0;
  for (float r : reps) {
    const uint32_t step = all ? 1u : 61u;
    for (uint64_t a = 0; a <= 0x7FFFFFFFull; a += step, ++n)
      if (check((uint32_t)a, r)) return 1;
    for (uint32_t e = 0; e < 256; ++e)
      for (int d = -2; d <= 2; ++d) {
        const int64_t a = ((int64_t)e << 23) + d;
        if (a < 0 || a > 0x7FFFFFFF) continue;
        if (check((uint32_t)a, r)) return 1;
        ++n;
      }
  }
  printf("checked %llu\n", (unsigned long long)n);
  return 0;
}
