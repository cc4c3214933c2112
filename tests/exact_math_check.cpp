// Host check of rai_amd/csrc/exact_math.h: expf_glibc() against the C
// library's expf, over the float bit patterns of [lo, hi] taken with a stride.
// Prints "<checked> <mismatches> <first mismatching input or nan>".
// Built and run by tests/test_cpu_pins.py (test infrastructure only).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "exact_math.h"

static float from_bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

int main(int argc, char **argv) {
  if (argc != 4) return 2;
  const float lo = std::strtof(argv[1], nullptr), hi = std::strtof(argv[2], nullptr);
  const uint32_t stride = (uint32_t)std::strtoul(argv[3], nullptr, 10);
  unsigned long long checked = 0, bad = 0;
  float first = NAN;
  // Walk the positive and the negative halves by bit pattern.
  for (int sign = 0; sign < 2; ++sign) {
    for (uint64_t u = 0; u < 0x7f800000ull; u += stride) {
      const float x = from_bits((uint32_t)u | (sign ? 0x80000000u : 0u));
      if (!(x >= lo && x <= hi)) continue;
      ++checked;
      const float a = rai_exact::expf_glibc(x), b = expf(x);
      uint32_t ua, ub;
      std::memcpy(&ua, &a, 4);
      std::memcpy(&ub, &b, 4);
      if (ua != ub) {
        if (!bad) first = x;
        ++bad;
      }
    }
  }
  std::printf("%llu %llu %.9g\n", checked, bad, first);
  return 0;
}
