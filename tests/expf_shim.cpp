// Test helper (built by tests/test_host_expf.py with g++): exposes librlh's
// two host-compiled expf restatements — the AVX2 path of the sampler's
// softmax (exp_shift_avx2, sampler.cpp) and expf_glibc_t (expf_glibc.h, the
// source the kernels compile) — and compares them with the C library's expf
// over a range of float bit patterns.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../llama.rs_amd/csrc/sampler.cpp"

// sampler.cpp reports argument errors through the engine's error slot.
int rlh::set_error(int code, const char*) { return code; }

namespace {

const uint64_t kTab[32] = RLH_EXP2_TABLE_INIT;

bool same_bits(float a, float b) {
  uint32_t x, y;
  std::memcpy(&x, &a, 4);
  std::memcpy(&y, &b, 4);
  return x == y || (a != a && b != b);
}

float from_bits(uint64_t u) {
  const uint32_t b = (uint32_t)u;
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

}  // namespace

extern "C" {

// Single values: which = 0 the AVX2 softmax path (x - 0), 1 expf_glibc_t,
// 2 the C library.
float shim_expf(float x, int which) {
  if (which == 0) {
    float v[4] = {x, x, x, x};
    rlh::exp_shift_avx2(v, 4, 0.0f);
    return v[0];
  }
  if (which == 1) return expf_glibc_t(x, kTab);
  return expf(x);
}

// Bit patterns [lo, hi) compared with the C library's expf; returns the
// number of differing results and the first differing pattern (or hi).
uint64_t shim_expf_mismatches(uint64_t lo, uint64_t hi, int which, int nthreads, uint64_t* first_bad) {
  if (nthreads < 1) nthreads = 1;
  std::vector<uint64_t> bad(nthreads, 0), first(nthreads, hi);
  std::vector<std::thread> th;
  const uint64_t span = (hi - lo + nthreads - 1) / nthreads;
  for (int t = 0; t < nthreads; t++) {
    th.emplace_back([&, t] {
      const uint64_t a = lo + span * t, b = std::min(hi, a + span);
      std::vector<float> buf(4096);
      for (uint64_t base = a; base < b; base += buf.size()) {
        const uint64_t n = std::min<uint64_t>(buf.size(), b - base);
        for (uint64_t i = 0; i < n; i++) buf[i] = from_bits(base + i);
        if (which == 0)
          rlh::exp_shift_avx2(buf.data(), n, 0.0f);
        else
          for (uint64_t i = 0; i < n; i++) buf[i] = expf_glibc_t(buf[i], kTab);
        for (uint64_t i = 0; i < n; i++) {
          if (!same_bits(buf[i], expf(from_bits(base + i)))) {
            if (!bad[t]) first[t] = base + i;
            bad[t]++;
          }
        }
      }
    });
  }
  for (auto& x : th) x.join();
  uint64_t total = 0, fb = hi;
  for (int t = 0; t < nthreads; t++) {
    total += bad[t];
    if (first[t] < fb) fb = first[t];
  }
  if (first_bad) *first_bad = fb;
  return total;
}

}  // extern "C"
