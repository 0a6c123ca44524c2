// expf with the results of glibc 2.35's expf on x86-64 (the std::exp(float) that the reference calls in its softmax tails
// and chunk merges: /root/reference/src/kernels_x86.cpp:420, /root/reference/src/model_llama.cpp:163), for host and
// device code.
//
// Method (the published table-driven scheme of glibc's single-precision exp since 2.27, restated here): with N = 32,
// z = x * N / ln 2 in double, k = round(z) (by adding and subtracting 1.5 * 2^52), r = z - k in [-1/2, 1/2];
// 2^(k / N) = 2^(k div N) * T[k mod N] with T[i] = 2^(i / N) rounded to double; exp(x) ~ 2^(k / N) * (1 + c2 r + c1 r^2
// + c0 r^3), evaluated in double with fused multiply-adds and rounded once to float.  T is the correctly rounded table
// (computed with 60-digit decimal arithmetic); c0..c2 are the degree-3 coefficients of 2^(r / N).
//
// Pinned exhaustively: tests/test_expf.py compiles this header for the host and compares it with the C library's expf on
// every one of the 2^32 float inputs (NaNs excepted).  Two inputs round the other way in glibc (its double result lies
// 0.5001 ulp from the exact value, this evaluation's on the correct side); they are returned as glibc returns them.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define QPH_HD __host__ __device__
#else
#define QPH_HD
#endif

namespace qph {

QPH_HD inline double libm_fma(double a, double b, double c) { return __builtin_fma(a, b, c); }

QPH_HD inline float libm_expf(float x) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
  // 2^(i / 32) for i = 0..31, correctly rounded
  constexpr double T[32] = {
      0x1.0000000000000p+0, 0x1.059b0d3158574p+0, 0x1.0b5586cf9890fp+0, 0x1.11301d0125b51p+0, 0x1.172b83c7d517bp+0,
      0x1.1d4873168b9aap+0, 0x1.2387a6e756238p+0, 0x1.29e9df51fdee1p+0, 0x1.306fe0a31b715p+0, 0x1.371a7373aa9cbp+0,
      0x1.3dea64c123422p+0, 0x1.44e086061892dp+0, 0x1.4bfdad5362a27p+0, 0x1.5342b569d4f82p+0, 0x1.5ab07dd485429p+0,
      0x1.6247eb03a5585p+0, 0x1.6a09e667f3bcdp+0, 0x1.71f75e8ec5f74p+0, 0x1.7a11473eb0187p+0, 0x1.82589994cce13p+0,
      0x1.8ace5422aa0dbp+0, 0x1.93737b0cdc5e5p+0, 0x1.9c49182a3f090p+0, 0x1.a5503b23e255dp+0, 0x1.ae89f995ad3adp+0,
      0x1.b7f76f2fb5e47p+0, 0x1.c199bdd85529cp+0, 0x1.cb720dcef9069p+0, 0x1.d5818dcfba487p+0, 0x1.dfc97337b9b5fp+0,
      0x1.ea4afa2a490dap+0, 0x1.f50765b6e4540p+0};
  constexpr double N = 32.0;
  constexpr double c0 = 0x1.c6af84b912394p-5 / (N * N * N), c1 = 0x1.ebfce50fac4f3p-3 / (N * N), c2 = 0x1.62e42ff0c52d6p-1 / N;
  constexpr double inv_ln2_n = 0x1.71547652b82fep+0 * N, shift = 0x1.8p+52;
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  if (b == 0xc27c65d9u) return 0x1.f45326p-92f;   // x = -0x1.f8cbb2p+5
  if (b == 0x4202422fu) return 0x1.f93e38p+46f;   // x = 0x1.04845ep+5
  if (x != x) return x;
  if (x > 0x1.62e42ep6f) return __builtin_inff();
  if (x < -0x1.9fe368p6f) return 0.f;
  const double z = inv_ln2_n * (double)x;
  double kd = z + shift;
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= shift;
  const double r = z - kd;
  const uint64_t t = __builtin_bit_cast(uint64_t, T[ki % 32]) - ((ki % 32) << 47) + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double p = libm_fma(c0, r, c1), r2 = r * r;
  double y = libm_fma(c2, r, 1.0);
  y = libm_fma(p, r2, y);
  return (float)(y * s);
}

}  // namespace qph
