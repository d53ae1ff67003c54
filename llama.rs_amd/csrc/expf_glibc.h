// expf_glibc.h — expf with the results of the host glibc expf, which the
// reference reaches through f32::exp (softmax_inplace ops.rs:410, silu
// ops.rs:394) on x86-64 linux-gnu.
//
// Method (glibc's expf for FMA-capable x86-64, taken from ARM's published
// optimized-routines): x * 32/ln2 = k + r with |r| <= 1/2,
// exp(x) = 2^(k/32) * p(r) where p is a cubic evaluated in double with
// FMAs and 2^(k/32) is built from a 32-entry table T[i] = bits(2^(i/32)) -
// (i << 47) plus k << 47 in the exponent field. |x| >= 88 and NaN take the
// special cases (overflow to +inf above 0x1.62e42ep6, 0 below -0x1.9fe368p6,
// x + x for NaN and +inf, 0 for -inf).
//
// The includer defines RLH_EXPF_QUAL (the function qualifiers: `__device__
// __forceinline__` in the kernels, `inline` in host code) before including
// this header. The table is passed in as `tab` (anything indexable by
// uint64_t: a __constant__ array, an LDS copy, a host array).
// The includer provides uint32_t / uint64_t (<cstdint>); the header may be
// included inside a namespace.
#pragma once

#ifndef RLH_EXPF_QUAL
#error "define RLH_EXPF_QUAL before including expf_glibc.h"
#endif
// RLH_EXPF_KEEP(v): an optional barrier the includer may define that makes
// the compiler compute v where it stands, for every input (in GPU code an
// empty asm that reads and writes v's register; the compiler would
// otherwise move the main path into a branch around the special cases).
#ifndef RLH_EXPF_KEEP
#define RLH_EXPF_KEEP(v) ((void)0)
#endif

// T[i] = bits(2^(i/32)) - (i << 47), i = 0..31 (as an initializer list).
#define RLH_EXP2_TABLE_INIT                                                                                   \
  {0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,               \
   0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,               \
   0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,               \
   0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,               \
   0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,               \
   0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,               \
   0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,               \
   0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL}

// Coefficients: 32/ln2, the rounding shift 1.5 * 2^52, and the cubic's
// coefficients of r^3, r^2, r scaled by 32^-3, 32^-2, 32^-1.
#define RLH_EXPF_INV_LN2_N (0x1.71547652b82fep+0 * 32.0)
#define RLH_EXPF_SHIFT 0x1.8p+52
#define RLH_EXPF_C0 (0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0)
#define RLH_EXPF_C1 (0x1.ebfce50fac4f3p-3 / 32.0 / 32.0)
#define RLH_EXPF_C2 (0x1.62e42ff0c52d6p-1 / 32.0)

// The main path runs for every x and the special cases replace its value
// after it by selects (no branch: in a GPU loop the branches cost more than
// the arithmetic). For NaN, infinite or huge x the main path's value is
// discarded; its integer arithmetic wraps and its table index stays in 0..31.
template <class Tab>
RLH_EXPF_QUAL float expf_glibc_t(float x, Tab tab) {
  const uint32_t ux = __builtin_bit_cast(uint32_t, x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  const double xd = (double)x;
  double kd = __builtin_fma(RLH_EXPF_INV_LN2_N, xd, RLH_EXPF_SHIFT);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= RLH_EXPF_SHIFT;
  const double r = __builtin_fma(RLH_EXPF_INV_LN2_N, xd, -kd);
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double z = __builtin_fma(RLH_EXPF_C0, r, RLH_EXPF_C1);
  const double r2 = r * r;
  double y = __builtin_fma(RLH_EXPF_C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  // |x| >= 88 or NaN (below 88 none of these conditions holds): underflow
  // below -0x1.9fe368p6 (and -inf) gives 0, overflow above 0x1.62e42ep6
  // +inf, +inf and NaN x + x; one select each, on the bit patterns (so that
  // NaN results keep x + x's payload)
  uint32_t rb = __builtin_bit_cast(uint32_t, (float)y), nb = __builtin_bit_cast(uint32_t, x + x);
  RLH_EXPF_KEEP(rb);
  RLH_EXPF_KEEP(nb);
  rb = x < -0x1.9fe368p6f ? 0u : rb;
  rb = x > 0x1.62e42ep6f ? 0x7f800000u : rb;
  rb = ((abstop >= 0x7f8) & (ux != 0xff800000u)) ? nb : rb;
  return __builtin_bit_cast(float, rb);
}
