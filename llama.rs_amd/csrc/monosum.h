// monosum.h — the f32 sum ((0 + x0) + x1) + ... of non-negative floats,
// bit for bit as the sequential loop rounds it, evaluated in parallel.
//
// While the running sum s stays below the top of its binade H, every value
// it can take is a multiple of the binade's spacing U = 2^u: s = N * U with
// an integer N < 2^24 (H = 2^24 * U). Adding x >= 0 rounds to
//   N' = N + floor(x / U) + r,  r = 1 if the remainder is above U/2,
//   0 if below, and at exactly U/2 (ties to even) 1 when N + floor(x/U) is odd.
// The increment depends on N only through its parity, so a run of additions
// is a function of the starting parity: a pair of increments (even start,
// odd start). Pairs compose associatively (mono_then), so a parallel prefix
// over them gives every partial sum inside the binade exactly. The first
// addition that would make N reach 2^24 leaves the binade: it is done as a
// real f32 add, and the prefix restarts from it with the new spacing. The
// region below 2^-125 (subnormals and the first normal binade) has the
// uniform spacing 2^-149 and is one "binade" here.
//
// The includer defines RLH_MONO_QUAL (`__device__ __forceinline__` in the
// kernels, `inline` in host code) and provides uint32_t (<cstdint>).
#pragma once

#ifndef RLH_MONO_QUAL
#error "define RLH_MONO_QUAL before including monosum.h"
#endif

// An increment pair saturates here: far beyond 2^24, where only "the sum
// left the binade" matters.
#define RLH_MONO_SAT (1u << 30)
#define RLH_MONO_TOP (1u << 24)

struct MonoFn {
  uint32_t a0, a1;  // increments of N for an even / an odd starting N
};

RLH_MONO_QUAL uint32_t mono_sat(uint32_t x) { return x < RLH_MONO_SAT ? x : RLH_MONO_SAT; }

RLH_MONO_QUAL MonoFn mono_identity() { return MonoFn{0u, 0u}; }

// f, then g
RLH_MONO_QUAL MonoFn mono_then(MonoFn f, MonoFn g) {
  MonoFn h;
  h.a0 = mono_sat(f.a0 + ((f.a0 & 1u) ? g.a1 : g.a0));
  h.a1 = mono_sat(f.a1 + ((f.a1 & 1u) ? g.a0 : g.a1));
  return h;
}

// The increment pair of adding x (finite, >= 0) at spacing 2^u.
RLH_MONO_QUAL MonoFn mono_elem(float x, int u) {
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  const uint32_t ef = b >> 23;
  const uint32_t m = ef ? ((b & 0x7fffffu) | 0x800000u) : b;
  if (m == 0) return MonoFn{0u, 0u};
  const int ee = ef ? (int)ef - 150 : -149;  // x = m * 2^ee
  const int sh = u - ee;                     // x / U = m * 2^-sh
  if (sh <= 0) {                             // a whole multiple of U
    if (sh <= -7) return MonoFn{RLH_MONO_SAT, RLH_MONO_SAT};
    const uint32_t q = mono_sat(m << (uint32_t)(-sh));
    return MonoFn{q, q};
  }
  if (sh > 25) return MonoFn{0u, 0u};  // x < U / 4
  const uint32_t q = m >> (uint32_t)sh, rem = m & ((1u << (uint32_t)sh) - 1u), half = 1u << (uint32_t)(sh - 1);
  const uint32_t up = rem > half ? 1u : 0u, tie = rem == half ? 1u : 0u;
  return MonoFn{q + up + (tie & (q & 1u)), q + up + (tie & ((q & 1u) ^ 1u))};
}

// Spacing exponent u and integer N of a running sum s >= 0 (finite).
RLH_MONO_QUAL void mono_state(float s, int* u, uint32_t* n) {
  const uint32_t b = __builtin_bit_cast(uint32_t, s), ef = b >> 23;
  if (ef <= 1u) {
    *u = -149;
    *n = b;
  } else {
    *u = (int)ef - 150;
    *n = (b & 0x7fffffu) | 0x800000u;
  }
}

// The state for a run of subtractions: as mono_state, except that a power of
// two 2^23 * U is written 2^24 * (U/2), in the binade below, whose spacing
// every subtraction from it rounds to.
RLH_MONO_QUAL void mono_state_dec(float s, int* u, uint32_t* n) {
  mono_state(s, u, n);
  if (*u > -149 && *n == (RLH_MONO_TOP >> 1)) {
    *u -= 1;
    *n = RLH_MONO_TOP;
  }
}

// The sum N * 2^u (N <= 2^24, N >= 2^23 unless u = -149).
RLH_MONO_QUAL float mono_value(int u, uint32_t n) {
  return __builtin_bit_cast(float, ((uint32_t)(u + 149) << 23) + n);
}

// The increment for a starting N.
RLH_MONO_QUAL uint32_t mono_apply(MonoFn f, uint32_t n) { return (n & 1u) ? f.a1 : f.a0; }

// Subtraction. r - x with x >= 0 from r = N * U rounds to N - d where d is
// the same pair's entry: the exact value N - x/U rounds down by one more
// than floor(x/U) when the remainder is above U/2, and at exactly U/2 when
// N - floor(x/U) is odd, which has the parity of N + floor(x/U). A run of
// subtractions is exact in the model while every intermediate value stays
// above the binade's floor: 2^23 in a normal binade (a result of exactly
// 2^23 may have come from a value just below, where the spacing halves),
// 0 in the region below 2^-125 (there every difference of floats is exact).
// Its state comes from mono_state_dec, so that N is above the floor unless
// the value is 0.

// True when a run that starts at N and adds `inc` in total may leave the
// binade: the run is then finished with real f32 adds.
RLH_MONO_QUAL bool mono_inc_leaves(uint32_t n, uint32_t inc) { return n + inc >= RLH_MONO_TOP; }

// The same for a run of subtractions of `dec` in total from N at spacing 2^u.
RLH_MONO_QUAL bool mono_dec_leaves(int u, uint32_t n, uint32_t dec) {
  const uint32_t floor_n = u == -149 ? 0u : (RLH_MONO_TOP >> 1);
  return dec >= n - floor_n;
}

// The softmax-sum walk (the attention softmax's sum over positions): the
// terms are split into runs; each run's pair is made at the binade that an
// approximate prefix sum predicts for its start (mono_binade of that
// estimate). Walking the runs in order, a run's pair applies when the exact
// state lies in that binade and the run does not leave it; otherwise its
// terms are added with f32 adds from mono_value(u, N) and the new state is
// taken with mono_state. The prediction only chooses between the two
// paths, never the result.
RLH_MONO_QUAL int mono_binade(float s) {
  int u;
  uint32_t n;
  mono_state(s, &u, &n);
  return u;
}

template <typename P>
RLH_MONO_QUAL MonoFn mono_run_pair(P x, uint32_t k, int u) {
  MonoFn f = mono_identity();
  for (uint32_t i = 0; i < k; i++) f = mono_then(f, mono_elem(x[i], u));
  return f;
}

