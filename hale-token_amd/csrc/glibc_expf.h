/*
 * glibc_expf.h -- single-precision exp that returns glibc's expf bits.
 *
 * Hale-Token computes SiLU and softmax with Rust's f32::exp
 * (src/ops/activation.rs:6,15), which on x86_64 Linux is a call to glibc's
 * expf.  glibc (>= 2.28) uses the ARM optimized-routines expf: with
 * N = 32, z = x*N/ln2 is split as k + r (k an integer, |r| <= 1/2),
 * 2^(k/N) comes from a 32-entry table of 2^(i/N) with the integer part of
 * k/N added to the exponent field, and 2^(r/N) from a degree-3 polynomial,
 * all in double precision, rounded once to float at the end.  On x86_64 the
 * glibc build selected on CPUs with FMA contracts the range reduction and
 * the polynomial into fused multiply-adds, which this function does too.
 *
 * The table holds round-to-nearest doubles of 2^(i/32), stored minus
 * i << 47 so that adding k << 47 scales by 2^(k/32).  The polynomial
 * coefficients are the published least-squares fit of 2^(r/32) on
 * [-1/2, 1/2] (1/ln2 = 0x1.71547652b82fep0).
 *
 * tests/test_expf.py compiles this header for the host and compares it with
 * the host glibc expf on all 2^32 float inputs.
 *
 * The same text compiles as C (host test) and as HIP device code; the
 * includer sets HALE_EXPF_FN / HALE_EXPF_TABLE to add __device__ qualifiers.
 */
#ifndef HALE_GLIBC_EXPF_H
#define HALE_GLIBC_EXPF_H

#include <stdint.h>

#ifndef HALE_EXPF_FN
#define HALE_EXPF_FN static inline
#endif
#ifndef HALE_EXPF_TABLE
#define HALE_EXPF_TABLE static const
#endif

HALE_EXPF_TABLE uint64_t hale_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

/* Range reduction and special cases.  Returns 1 with the final result in
 * *res for |x| >= 88, inf and nan; otherwise returns 0 with the table index
 * (*ki % 32), ki and r for hale_expf_finish. */
HALE_EXPF_FN int hale_expf_reduce(float x, float *res, uint64_t *ki_out, double *r_out) {
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
  const double shift = 0x1.8p+52;
  uint32_t ix;
  __builtin_memcpy(&ix, &x, 4);
  uint32_t abstop = (ix >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) { /* |x| >= 88, or inf / nan */
    if (ix == 0xff800000u) { *res = 0.0f; return 1; }             /* -inf */
    if (abstop >= 0x7f8u) { *res = x + x; return 1; }             /* inf or nan */
    if (x > 0x1.62e42ep6f) { *res = __builtin_huge_valf(); return 1; } /* overflow */
    if (x < -0x1.9fe368p6f) { *res = 0.0f; return 1; }            /* underflow */
  }
  double xd = (double)x;
  double kd = __builtin_fma(inv_ln2_n, xd, shift);
  uint64_t ki;
  __builtin_memcpy(&ki, &kd, 8);
  kd -= shift;
  *ki_out = ki;
  *r_out = __builtin_fma(inv_ln2_n, xd, -kd);
  return 0;
}

/* 2^(k/32) from the table entry of ki % 32, times the polynomial for r. */
HALE_EXPF_FN float hale_expf_finish(uint64_t ki, double r, uint64_t tab_entry) {
  const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  uint64_t t = tab_entry + (ki << 47);
  double s;
  __builtin_memcpy(&s, &t, 8);
  double z = __builtin_fma(c0, r, c1);
  double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

HALE_EXPF_FN float hale_expf(float x) {
  float res;
  uint64_t ki;
  double r;
  if (hale_expf_reduce(x, &res, &ki, &r)) return res;
  return hale_expf_finish(ki, r, hale_exp2_tab[ki % 32]);
}

#endif /* HALE_GLIBC_EXPF_H */
