// Test helper (built by tests/test_monosum.py with g++): the exact parallel
// evaluation of sequential f32 sums and differences of non-negative terms
// (llama.rs_amd/csrc/monosum.h), run step by step as the device chains in
// sampler_dev.hip run it, next to the plain sequential loop it must equal.
//
// shim_chain:   wave_chain — T lanes of E consecutive terms per pass; an
//               exclusive scan of increment pairs; the first lane that may
//               leave the binade or reach the stop threshold replays its
//               terms with real f32 steps; the next pass starts after it.
// shim_softwalk: the attention softmax's sum (block_softmax_sum): 256 runs
//               of K terms (K a multiple of 4), each run's pair at the
//               binade its approximate f32 prefix predicts (mode 1 / 2 move
//               every prediction one binade up / down, mode 3 alternates, to
//               force the replay path); the runs are taken 64 at a time: a
//               scan of their pairs at the current binade, the first run that
//               misses it or may leave it replayed with f32 adds, the scan
//               resumed after it.
// shim_runwalk: k_run_pairs + k_run_walk — runs of R terms with pairs at the
//               three candidate binades from the f64 prefix estimate, walked
//               T runs per pass; the first run that may leave the binade, or
//               whose candidates miss it (cu_shift moves every candidate
//               window to force that path), is replayed by wave_chain over
//               its terms (E = 1, R lanes) from its exact start.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#define RLH_MONO_QUAL inline
#include "../llama.rs_amd/csrc/monosum.h"

namespace {

const uint32_t kNone = 0xffffffffu;
enum { STOP_NONE = 0, STOP_GE = 1, STOP_LE0 = 2 };

bool stop_at(int kind, float r, float thr) {
  return kind == STOP_GE ? r >= thr : (kind == STOP_LE0 ? r <= 0.0f : false);
}

void state(bool dec, float s, int* u, uint32_t* n) {
  if (dec)
    mono_state_dec(s, u, n);
  else
    mono_state(s, u, n);
}

uint64_t inc_limit(int u, int stop, float thr) {
  uint64_t lim = RLH_MONO_TOP;
  if (stop == STOP_GE) {
    const double q = std::ldexp((double)thr, -u);
    if (q < (double)RLH_MONO_TOP) lim = q <= 0.0 ? 0ull : (uint64_t)std::ceil(q);
  }
  return lim;
}

// One pass structure shared by both levels: lanes' functions f[0..T) from
// lane l0 on (identity before), start (u, N). Returns the first lane that may
// leave (T when none) and each lane's starting N in nl; *tot = the whole
// composition.
int scan_pass(bool dec, const std::vector<MonoFn>& f, int T, int l0, int u, uint32_t N, int stop, float thr,
              std::vector<uint32_t>* nl, MonoFn* tot) {
  MonoFn acc = mono_identity();
  int lc = T;
  for (int l = 0; l < T; l++) {
    const uint32_t a = mono_apply(acc, N);
    (*nl)[l] = dec ? N - a : N + a;
    const uint32_t b = mono_apply(f[l], (*nl)[l]);
    const bool leaves = dec ? mono_dec_leaves(u, N, a + b) : (uint64_t)N + a + b >= inc_limit(u, stop, thr);
    if (l >= l0 && leaves && lc == T) lc = l;
    acc = mono_then(acc, f[l]);
  }
  *tot = acc;
  return lc;
}

uint32_t chain(bool dec, const float* y, uint32_t len, float s0, int T, int E, int stop, float thr, float* val,
               uint64_t* passes) {
  float s = s0;
  std::vector<MonoFn> f(T);
  std::vector<uint32_t> nl(T);
  for (uint64_t base = 0; base < len; base += (uint64_t)T * E) {
    auto term = [&](int l, int k) {
      const uint64_t i = base + (uint64_t)l * E + k;
      return i < len ? y[i] : 0.0f;
    };
    int l0 = 0;
    for (;;) {
      (*passes)++;
      int u;
      uint32_t N;
      state(dec, s, &u, &N);
      for (int l = 0; l < T; l++) {
        MonoFn g = mono_identity();
        if (l >= l0)
          for (int k = 0; k < E; k++) g = mono_then(g, mono_elem(term(l, k), u));
        f[l] = g;
      }
      MonoFn tot;
      const int lc = scan_pass(dec, f, T, l0, u, N, stop, thr, &nl, &tot);
      if (lc == T) {
        const uint32_t t = mono_apply(tot, N);
        s = mono_value(u, dec ? N - t : N + t);
        break;
      }
      float r = mono_value(u, nl[lc]);
      for (int k = 0; k < E; k++) {
        r = dec ? r - term(lc, k) : r + term(lc, k);
        const uint64_t i = base + (uint64_t)lc * E + k;
        if (i < len && stop_at(stop, r, thr)) {
          *val = r;
          return (uint32_t)i;
        }
      }
      s = r;
      if (lc == T - 1) break;
      l0 = lc + 1;
    }
  }
  *val = s;
  return len;
}

}  // namespace

extern "C" {

// s_j = s_{j-1} + y_j (dec: - y_j) from s_{-1} = s0; the first j with the stop
// condition (1: s_j >= thr, 2: s_j <= 0), or len; *val = s_j there (the last
// value when none, s0 when len is 0).
uint32_t shim_seq(int dec, const float* y, uint32_t len, float s0, int stop_kind, float thr, float* val) {
  float s = s0;
  for (uint32_t j = 0; j < len; j++) {
    s = dec ? s - y[j] : s + y[j];
    if (stop_at(stop_kind, s, thr)) {
      *val = s;
      return j;
    }
  }
  *val = s;
  return len;
}

uint32_t shim_chain(int dec, const float* y, uint32_t len, float s0, int T, int E, int stop_kind, float thr,
                    float* val, uint64_t* passes) {
  *passes = 0;
  return chain(dec != 0, y, len, s0, T, E, stop_kind, thr, val, passes);
}

uint32_t shim_runwalk(int dec, const float* y, uint32_t len, float s0, int T, int R, int stop, float thr,
                      int cu_shift, float* val, uint64_t* passes, uint64_t* misses) {
  *passes = 0;
  *misses = 0;
  const uint32_t n_runs = (uint32_t)((len + R - 1) / R);
  // k_run_pairs: f64 run sums, prefix estimate, candidates, pairs
  std::vector<int> cu(n_runs);
  std::vector<MonoFn> pr(3 * (size_t)n_runs);
  double pre = 0.0;
  for (uint32_t r = 0; r < n_runs; r++) {
    const double est = dec ? (double)s0 - pre : (double)s0 + pre;
    const float fe = (float)est;
    int ug = -149;
    if (fe > 0.0f && std::isfinite(fe)) {
      uint32_t nn;
      mono_state(fe, &ug, &nn);
    }
    cu[r] = std::max(-149, ug - 1) + cu_shift;
    double rs = 0.0;
    for (int c = 0; c < 3; c++) {
      MonoFn g = mono_identity();
      for (int j = 0; j < R; j++) {
        const uint64_t i = (uint64_t)r * R + j;
        g = mono_then(g, mono_elem(i < len ? y[i] : 0.0f, cu[r] + c));
      }
      pr[3 * (size_t)r + c] = g;
    }
    for (int j = 0; j < R; j++) {
      const uint64_t i = (uint64_t)r * R + j;
      rs += i < len ? (double)y[i] : 0.0;
    }
    pre += rs;
  }
  // k_run_walk
  float s = s0;
  std::vector<MonoFn> f(T);
  std::vector<uint32_t> nl(T);
  for (uint32_t cb = 0; cb < n_runs; cb += T) {
    int l0 = 0;
    for (;;) {
      (*passes)++;
      int u;
      uint32_t N;
      state(dec != 0, s, &u, &N);
      std::vector<char> miss(T, 0);
      for (int l = 0; l < T; l++) {
        const uint32_t r = cb + l;
        f[l] = mono_identity();
        if (r >= n_runs || l < l0) continue;
        const int d = u - cu[r];
        if (d >= 0 && d <= 2) {
          f[l] = pr[3 * (size_t)r + d];
        } else {
          (*misses)++;
          miss[l] = 1;
        }
      }
      MonoFn tot;
      int lc = scan_pass(dec != 0, f, T, l0, u, N, stop, thr, &nl, &tot);
      for (int l = l0; l < lc; l++)
        if (miss[l]) {  // a miss counts as a run that may leave
          lc = l;
          break;
        }
      if (lc < T && cb + lc >= n_runs) lc = T;
      if (lc == T) {
        const uint32_t t = mono_apply(tot, N);
        s = mono_value(u, dec ? N - t : N + t);
        break;
      }
      const uint32_t run = cb + lc;
      const uint32_t rlen = (uint32_t)std::min<uint64_t>(R, len - (uint64_t)run * R);
      float v;
      const uint32_t j = chain(dec != 0, y + (size_t)run * R, rlen, mono_value(u, nl[lc]), R, 1, stop, thr, &v,
                               passes);
      if (j < rlen) {
        *val = v;
        return run * R + j;
      }
      s = v;
      if (lc == T - 1 || run + 1 >= n_runs) break;
      l0 = lc + 1;
    }
  }
  *val = s;
  return len;
}

uint32_t shim_softwalk(const float* x, uint32_t n, int mode, float* out, uint64_t* replays) {
  const uint32_t K = (((n + 255) / 256) + 3) & ~3u;
  const uint32_t nr = (n + K - 1) / K;
  std::vector<float> loc(nr), pre(nr);
  std::vector<MonoFn> f(nr);
  std::vector<int> ur(nr);
  for (uint32_t r = 0; r < nr; r++) {
    float a = 0.0f;
    for (uint32_t j = r * K; j < std::min(n, r * K + K); j++) a += x[j];
    loc[r] = a;
  }
  float acc = 0.0f;  // approximate exclusive prefix (any order would do)
  for (uint32_t r = 0; r < nr; r++) {
    pre[r] = acc;
    acc += loc[r];
    ur[r] = mono_binade(pre[r]);
    if (mode == 1 || (mode == 3 && (r & 1))) ur[r] += 1;
    if (mode == 2 || (mode == 3 && !(r & 1))) ur[r] -= 1;
    const uint32_t j0 = r * K;
    f[r] = mono_run_pair(x + j0, std::min(n, j0 + K) - j0, ur[r]);
  }
  int u = -149;
  uint32_t N = 0;
  *replays = 0;
  for (uint32_t gb = 0; gb < nr; gb += 64) {
    const uint32_t gl = std::min<uint32_t>(64, nr - gb);
    uint32_t l0 = 0;
    while (l0 < gl) {
      // the scan: lanes l0.. in order, each run's start state while every run
      // before it hits the binade and stays in it
      MonoFn pre_f = mono_identity();
      uint32_t lc = gl;
      uint32_t nl_c = 0;
      for (uint32_t l = l0; l < gl; l++) {
        const uint32_t r = gb + l;
        const uint32_t nl = N + mono_apply(pre_f, N);
        const bool hit = ur[r] == u;
        if (!hit || mono_inc_leaves(nl, mono_apply(f[r], nl))) {
          lc = l;
          nl_c = nl;
          break;
        }
        pre_f = mono_then(pre_f, f[r]);
      }
      if (lc == gl) {
        N += mono_apply(pre_f, N);
        break;
      }
      const uint32_t k0 = (gb + lc) * K;
      float sv = mono_value(u, nl_c);
      for (uint32_t j = k0; j < std::min(n, k0 + K); j++) sv = sv + x[j];
      mono_state(sv, &u, &N);
      ++*replays;
      l0 = lc + 1;
    }
  }
  *out = mono_value(u, N);
  return nr;
}

}  // extern "C"
