// Exact scalar math shared by the HIP kernels and host-side checks.
//
// rai's AVX2 path (rai-infer/src/layers.rs) uses two exponentials:
//   * the 8-wide bodies of SiLU and the attention softmax use Schraudolph's
//     bit trick (layers.rs:855-876, 1317-1331);
//   * scalar tails (n % 8 leftovers) and the MoE router softmax call Rust's
//     f32::exp, i.e. the C library's expf (glibc 2.35 on the reference
//     platform and on this build's hosts).
// To reproduce the reference bit for bit, the GPU evaluates both exactly as
// the CPU does.  expf_glibc() restates the published algorithm that glibc
// (since 2.28) ships as expf: ARM Optimized Routines' exp by a 32-entry
// 2^(i/32) table and a cubic polynomial in double precision (Szabolcs Nagy,
// 2017), with the multiply-adds fused as in glibc's FMA build, which is the
// variant x86-64 hosts with FMA select at run time.  The table holds the
// correctly rounded doubles 2^(i/32), minus i << 47.  tests/ checks this
// function against the host's expf on every float in [-110, 89].
#ifndef RAI_EXACT_MATH_H
#define RAI_EXACT_MATH_H

#include <stdint.h>

#include <cmath>
#include <cstring>

#if defined(__HIPCC__)
#define RAI_HD __host__ __device__ __forceinline__
#else
#define RAI_HD inline
#endif

namespace rai_exact {

RAI_HD uint32_t f2u(float f) {
  uint32_t u;
#if defined(__HIP_DEVICE_COMPILE__)
  u = __float_as_uint(f);
#else
  std::memcpy(&u, &f, 4);
#endif
  return u;
}
RAI_HD float u2f(uint32_t u) {
  float f;
#if defined(__HIP_DEVICE_COMPILE__)
  f = __uint_as_float(u);
#else
  std::memcpy(&f, &u, 4);
#endif
  return f;
}
RAI_HD uint64_t d2u(double d) {
  uint64_t u;
#if defined(__HIP_DEVICE_COMPILE__)
  u = (uint64_t)__double_as_longlong(d);
#else
  std::memcpy(&u, &d, 8);
#endif
  return u;
}
RAI_HD double u2d(uint64_t u) {
  double d;
#if defined(__HIP_DEVICE_COMPILE__)
  d = __longlong_as_double((long long)u);
#else
  std::memcpy(&d, &u, 8);
#endif
  return d;
}

RAI_HD double fma_d(double a, double b, double c) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __fma_rn(a, b, c);
#else
  return std::fma(a, b, c);
#endif
}

RAI_HD uint64_t exp2_tab(uint32_t i) {
  // 2^(i/32) rounded to nearest double, as bits, minus (i << 47).
  switch (i & 31u) {
    case 0: return 0x3ff0000000000000ULL;  case 1: return 0x3fefd9b0d3158574ULL;
    case 2: return 0x3fefb5586cf9890fULL;  case 3: return 0x3fef9301d0125b51ULL;
    case 4: return 0x3fef72b83c7d517bULL;  case 5: return 0x3fef54873168b9aaULL;
    case 6: return 0x3fef387a6e756238ULL;  case 7: return 0x3fef1e9df51fdee1ULL;
    case 8: return 0x3fef06fe0a31b715ULL;  case 9: return 0x3feef1a7373aa9cbULL;
    case 10: return 0x3feedea64c123422ULL; case 11: return 0x3feece086061892dULL;
    case 12: return 0x3feebfdad5362a27ULL; case 13: return 0x3feeb42b569d4f82ULL;
    case 14: return 0x3feeab07dd485429ULL; case 15: return 0x3feea47eb03a5585ULL;
    case 16: return 0x3feea09e667f3bcdULL; case 17: return 0x3fee9f75e8ec5f74ULL;
    case 18: return 0x3feea11473eb0187ULL; case 19: return 0x3feea589994cce13ULL;
    case 20: return 0x3feeace5422aa0dbULL; case 21: return 0x3feeb737b0cdc5e5ULL;
    case 22: return 0x3feec49182a3f090ULL; case 23: return 0x3feed503b23e255dULL;
    case 24: return 0x3feee89f995ad3adULL; case 25: return 0x3feeff76f2fb5e47ULL;
    case 26: return 0x3fef199bdd85529cULL; case 27: return 0x3fef3720dcef9069ULL;
    case 28: return 0x3fef5818dcfba487ULL; case 29: return 0x3fef7c97337b9b5fULL;
    case 30: return 0x3fefa4afa2a490daULL; default: return 0x3fefd0765b6e4540ULL;
  }
}

// expf as glibc computes it (see the file comment).
RAI_HD float expf_glibc(float x) {
  const uint32_t ix = f2u(x);
  const uint32_t abstop = (ix >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88, inf or nan
    if (ix == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);  // overflow to +inf
    if (x < -0x1.9fe368p6f) return 0.0f;             // underflow to +0
  }
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32768.0;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 1024.0;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = (double)x;
  double kd = fma_d(inv_ln2_n, xd, shift);
  const uint64_t ki = d2u(kd);
  kd -= shift;
  const double r = fma_d(inv_ln2_n, xd, -kd);
  uint64_t t = exp2_tab((uint32_t)(ki % 32u));
  t += ki << 47;
  const double s = u2d(t);
  const double z = fma_d(c0, r, c1);
  const double r2 = r * r;
  double y = fma_d(c2, r, 1.0);
  y = fma_d(z, r2, y);
  y = y * s;
  return (float)y;
}

// One lane of the AVX2 Schraudolph exponential (layers.rs:855-876):
// t = 12102203*x + (1065353216 - 486411) in f32, unfused; clamp with the
// operand order of _mm256_min_ps / _mm256_max_ps; round to nearest even;
// reinterpret the integer as float bits.
RAI_HD float schraudolph(float x) {
  const float a = 12102203.0f;
  const float b = 1064866816.0f;  // f32(1065353216 - 486411), rounded in f32
#if defined(__HIP_DEVICE_COMPILE__)
  float t = __fadd_rn(__fmul_rn(a, x), b);
#else
  float t = a * x + b;
#endif
  t = (t < 2139095040.0f) ? t : 2139095040.0f;  // _mm256_min_ps(t, hi)
  t = (t > 0.0f) ? t : 0.0f;                    // _mm256_max_ps(t, lo)
#if defined(__HIP_DEVICE_COMPILE__)
  const int32_t i = __float2int_rn(t);
#else
  const int32_t i = (int32_t)std::nearbyint(t);
#endif
  return u2f((uint32_t)i);
}

}  // namespace rai_exact

#endif
