// sampler_dev.hip — the token sampler (src/sampler.rs:56-163) and the
// softmax it runs (ops::softmax_inplace, src/ops.rs:398-419) on device-resident
// logits, giving the tokens and probabilities of the host restatement
// (sampler.cpp) bit for bit, so a sampled decode loop never copies the
// vocabulary's logits to the host.
//
// Steps (one HIP stream, no host round trip until the token is read):
//   scale    x = pen(logit) * (1/temperature): the repetition penalty on the
//            distinct ids of the window (sampler.rs:82-102, a sorted id list
//            the host builds) and the temperature (115-118); block maxima
//   exp      e = expf(x - max) with glibc's expf (ops.rs:402-410), max by the
//            reference's rule (x[0] when it is NaN, else the largest non-NaN);
//            f64 sums of every run of 64 terms
//   sum      the index-order f32 sum of e (ops.rs:411-414), exact: increment
//            pairs of every run at three candidate binades (monosum.h; the
//            f64 prefix fixes the candidates), then one wave scans the runs
//            and replays the few runs that leave a binade with real f32 adds
//   norm     p = e * (1/sum) when sum > 0 (ops.rs:415-418); a histogram of the
//            top 8 bits of p (exponent and first mantissa bit), with the f64
//            mass of each bin
//   top-k    candidates: every p whose digit is at least a threshold chosen
//            from the histogram, an exact prefix of the sorted order that
//            holds the k wanted (top-p alone: whose mass surely reaches top_p);
//            sorted by (p descending, id ascending) on chip. Lists that do not
//            fit 4096, and top_k 0 without top-p, take a device radix sort.
//   pick     the top-p running sum (sampler.rs:135-146) and the draw
//            r = u * sum, r -= p until r <= 0 (148-162), both exact chains;
//            u is the host's xorshift64* draw (sampler.rs:40-54), passed in.
// Equal probabilities are ordered by id, as in the host restatement (the
// reference leaves their order to select_nth_unstable).
#include <hip/hip_runtime.h>

#include <rocprim/device/device_radix_sort.hpp>

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "../../include/rlh.h"
#include "kernels.h"
#include "rlh_device.h"
#include "sampler.h"
#include "sampler_dev.h"

#define RLH_MONO_QUAL __device__ __forceinline__
#include "monosum.h"
#include "monosum_wave.h"

namespace rlh {

namespace {

constexpr uint32_t kEwThreads = 256;                  // elementwise kernels
constexpr uint32_t kEwPer = 4;                        // elements per thread
constexpr uint32_t kEwBlock = kEwThreads * kEwPer;    // elements per block
constexpr uint32_t kRun = 64;                         // terms per run of a long chain
constexpr uint32_t kRunsPerBlock = 16;                // k_run_pairs: 4 waves x 4 runs
constexpr uint32_t kCandMax = 4096;                   // candidates sorted on chip
constexpr uint32_t kNone = 0xffffffffu;
constexpr double kTopPMargin = 1e-3;                  // relative; see k_sd_candidates

enum : uint32_t { F_NAN = 1, F_OVERFLOW = 2, F_SHORT = 4 };
enum : int { STOP_NONE = 0, STOP_GE = 1, STOP_LE0 = 2 };
enum : int { OUT_SUM = 0, OUT_TOPP = 1, OUT_DRAW = 2 };

// Device-side state of one call.
struct SdState {
  float sum;         // softmax sum (NaN when an exponential is NaN)
  uint32_t flags;    // F_*
  uint32_t n_cand;   // candidates written
  uint32_t token;
  uint32_t rng_used; // the draw consumed the uniform (sum > 0)
  uint32_t cutoff;   // kept list length after top-p
  float kept_sum;    // sum of the kept list
  float x0;          // x[0] after penalty and temperature (the max rule reads it)
};

// Increment pairs of the runs of a long chain at three consecutive candidate
// binades cu, cu + 1, cu + 2, laid out per chunk of 64 runs as 8 rows of 64:
// cu, a0 and a1 of each candidate, one unused row; the walk copies a chunk's
// 2 KB in one piece.
constexpr uint32_t kPairRows = 8;
__device__ __forceinline__ uint32_t pair_at(uint32_t run, uint32_t row) {
  return (run >> 6) * (kPairRows * 64) + row * 64 + (run & 63);
}

__device__ __forceinline__ uint32_t lower_bound_u32(const uint32_t* a, uint32_t n, uint32_t key) {
  uint32_t lo = 0, hi = n;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (a[mid] < key)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// Largest non-NaN value of the block (v > m never holds for a NaN v).
__device__ __forceinline__ float block_max256(float m, float* red) {
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(m, off);
    m = o > m ? o : m;
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = m;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < (int)(kEwThreads / 64); i++) r = red[i] > r ? red[i] : r;
  return r;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// x = pen(in) * inv_t (scale set) or pen(in); per-block maxima. Block 0 also
// clears the call's state, the digit histogram and its masses (kernels below
// run after it on the same stream).
__global__ void __launch_bounds__(kEwThreads)
    k_sd_scale(const float* in, float* x, uint32_t n, float inv_t, int scale, float rp, const uint32_t* pen,
               uint32_t n_pen, float* part_max, SdState* st, uint32_t* hist, double* mass) {
  __shared__ float red[kEwThreads / 64];
  const uint32_t t = threadIdx.x, lo = blockIdx.x * kEwBlock;
  if (blockIdx.x == 0) {
    hist[t] = 0;
    mass[t] = 0.0;
    if (t == 0) {
      st->flags = 0;
      st->n_cand = 0;
      st->token = 0;
      st->rng_used = 0;
      st->cutoff = 0;
      st->kept_sum = 0.0f;
    }
  }
  const uint32_t hi = min(n, lo + kEwBlock);
  uint32_t j0 = 0, j1 = 0;
  if (n_pen) {
    j0 = lower_bound_u32(pen, n_pen, lo);
    j1 = lower_bound_u32(pen, n_pen, hi);
  }
  float m = -__int_as_float(0x7f800000);
#pragma unroll
  for (uint32_t k = 0; k < kEwPer; k++) {
    const uint32_t i = lo + k * kEwThreads + t;
    if (i < n) {
      float v = in[i];
      if (j1 > j0) {
        const uint32_t j = j0 + lower_bound_u32(pen + j0, j1 - j0, i);
        if (j < j1 && pen[j] == i) v = v > 0.0f ? v / rp : v * rp;  // sampler.rs:96-100
      }
      if (scale) v = v * inv_t;
      x[i] = v;
      if (i == 0) st->x0 = v;
      m = v > m ? v : m;
    }
  }
  m = block_max256(m, red);
  if (t == 0) part_max[blockIdx.x] = m;
}

// a - b with the NaN results of the x86 subtraction the reference runs
// (SSE subss/subps): a NaN operand comes out quieted (the first one when
// both are NaN), and an invalid difference (inf - inf) is the negative
// "indefinite" NaN 0xffc00000. The GPU's own NaN results differ in sign and
// payload; finite and infinite results are the same IEEE difference.
__device__ __forceinline__ float sub_x86(float a, float b) {
  const float d = a - b;
  if (d == d) return d;
  if (a != a) return __uint_as_float(__float_as_uint(a) | 0x00400000u);
  if (b != b) return __uint_as_float(__float_as_uint(b) | 0x00400000u);
  return __uint_as_float(0xffc00000u);
}

// e = expf(x - max), in place; F_NAN when any e is NaN; rs[r] = f64 sum of
// run r (64 consecutive terms: one wave's slice of one of the block's rows).
__global__ void __launch_bounds__(kEwThreads)
    k_sd_exp(float* x, uint32_t n, const float* part_max, uint32_t nb, SdState* st, double* rs) {
  __shared__ float red[kEwThreads / 64];
  const uint32_t t = threadIdx.x, lo = blockIdx.x * kEwBlock;
  float m = -__int_as_float(0x7f800000);
  for (uint32_t i = t; i < nb; i += kEwThreads) {
    const float v = part_max[i];
    m = v > m ? v : m;
  }
  m = block_max256(m, red);
  const float x0 = st->x0;  // x[0] itself may already hold its exponential
  const float mx = x0 != x0 ? x0 : m;  // ops.rs:402-407
  bool nan = false;
#pragma unroll
  for (uint32_t k = 0; k < kEwPer; k++) {
    const uint32_t i = lo + k * kEwThreads + t;
    float e = 0.0f;
    if (i < n) {
      e = expf_glibc(sub_x86(x[i], mx));
      x[i] = e;
      nan |= e != e;
    }
    const double rsum = wave_sum_f64((double)e);
    const uint32_t run = (lo + k * kEwThreads + (t & ~63u)) / kRun;
    if ((t & 63) == 0 && run * kRun < n) rs[run] = rsum;
  }
  if (__ballot(nan) != 0 && (t & 63) == 0) atomicOr(&st->flags, F_NAN);
}

// rs[r] = f64 sum of run r of y[0..len) (for chains over arrays no earlier
// kernel summed).
__global__ void __launch_bounds__(kEwThreads) k_run_sums(const float* y, uint32_t len, double* rs) {
  const uint32_t t = threadIdx.x, lo = blockIdx.x * kEwBlock;
#pragma unroll
  for (uint32_t k = 0; k < kEwPer; k++) {
    const uint32_t i = lo + k * kEwThreads + t;
    const double rsum = wave_sum_f64(i < len ? (double)y[i] : 0.0);
    const uint32_t run = (lo + k * kEwThreads + (t & ~63u)) / kRun;
    if ((t & 63) == 0 && run * kRun < len) rs[run] = rsum;
  }
}

// ---- exact chains ------------------------------------------------------------
//
// A chain is s_j = s_{j-1} + y_j (DEC: - y_j), j < len, from s_{-1} = s0, with
// the values of the sequential f32 loop (all y_j >= 0), stopping at the first
// j where the stop condition holds (STOP_GE: s_j >= thr; STOP_LE0: s_j <= 0).
// Inside a binade the model of monosum.h is exact; a term that may leave the
// binade, or reach the stop condition, is done as a real f32 step.

template <bool DEC>
__device__ __forceinline__ void chain_state(float s, int* u, uint32_t* n) {
  if (DEC)
    mono_state_dec(s, u, n);
  else
    mono_state(s, u, n);
}

// For an increasing chain: the N (at spacing 2^u) from which a run must be
// replayed: the binade's top, or the first N whose value reaches thr.
__device__ __forceinline__ uint64_t inc_limit(int u, int stop, float thr) {
  uint64_t lim = RLH_MONO_TOP;
  if (stop == STOP_GE) {
    const double q = ldexp((double)thr, -u);  // exact: a power-of-two scaling
    if (q < (double)RLH_MONO_TOP) lim = q <= 0.0 ? 0ull : (uint64_t)ceil(q);
  }
  return lim;
}

__device__ __forceinline__ bool stop_at(int stop, float r, float thr) {
  return stop == STOP_GE ? r >= thr : (stop == STOP_LE0 ? r <= 0.0f : false);
}

// One wave, E terms per lane per pass (lane l: terms base + l*E .. + E).
// Each pass forms every lane's increment pair at the current binade, scans
// them, and finds the first lane whose terms may leave the binade or reach
// the stop condition; lanes before it are exact in the model, that lane
// replays its terms with real f32 steps, and the next pass starts after it.
// Returns the stop index (len when none) and *val = s there (the last value
// when none). All 64 lanes call it with uniform arguments.
template <bool DEC, int E, class Load>
__device__ uint32_t wave_chain(Load y, uint32_t len, float s0, int stop, float thr, float* val) {
  const int lane = threadIdx.x & 63;
  float s = s0;
  for (uint32_t base = 0; base < len; base += 64u * E) {
    const uint32_t i0 = base + (uint32_t)lane * E;
    float v[E];
#pragma unroll
    for (int k = 0; k < E; k++) v[k] = i0 + k < len ? y(i0 + k) : 0.0f;
    int l0 = 0;
    for (;;) {
      int u;
      uint32_t N;
      chain_state<DEC>(s, &u, &N);
      MonoFn f = mono_identity();
      if (lane >= l0) {
#pragma unroll
        for (int k = 0; k < E; k++) f = mono_then(f, mono_elem(v[k], u));
      }
      const MonoFn incl = wave_scan_fn(f);
      const uint32_t a = mono_apply(wave_excl_fn(incl), N);
      const uint32_t nl = DEC ? N - a : N + a;
      const uint32_t b = mono_apply(f, nl);
      bool leaves;
      if (DEC)
        leaves = mono_dec_leaves(u, N, a + b);
      else
        leaves = (uint64_t)N + a + b >= inc_limit(u, stop, thr);
      const uint64_t mask = __ballot(lane >= l0 && leaves);
      if (mask == 0) {
        const uint32_t tot = mono_apply(MonoFn{readlane_u32(incl.a0, 63), readlane_u32(incl.a1, 63)}, N);
        s = mono_value(u, DEC ? N - tot : N + tot);
        break;
      }
      const int lc = (int)__builtin_ctzll(mask);
      float r = mono_value(u, nl);
      uint32_t ev = kNone;
#pragma unroll
      for (int k = 0; k < E; k++) {
        r = DEC ? r - v[k] : r + v[k];
        if (ev == kNone && i0 + k < len && stop_at(stop, r, thr)) {
          ev = i0 + k;
          *val = r;
        }
        if (ev == kNone) s = r;  // the lane's value after its last term (no event)
      }
      const uint32_t evc = readlane_u32(ev, lc);
      if (evc != kNone) {
        *val = readlane_f32(*val, lc);
        return evc;
      }
      s = readlane_f32(s, lc);
      if (lc == 63) break;
      l0 = lc + 1;
    }
  }
  *val = s;
  return len;
}

// Increment pairs of every run at its three candidate binades. The f64 sum of
// the runs before it gives the chain's value at the run's start to far better
// than the f32 chain's own drift (at most n * 2^-24 relative for n terms, 0.9%
// at n = 151936), so the run starts in binade u - 1, u or u + 1 of that
// estimate; cu = u - 1. 4 waves per block, 4 runs per wave, one term per lane.
// s0 and len come from the arguments, or, for the draw (from_state), from
// the state: s0 = u_rand * kept_sum, len = cutoff.
template <bool DEC>
__global__ void __launch_bounds__(kEwThreads)
    k_run_pairs(const float* y, uint32_t len, float s0, int from_state, float u_rand, const SdState* st,
                const double* rs, uint32_t* rp) {
  __shared__ double red[kEwThreads / 64];
  if (from_state) {
    len = st->cutoff;
    s0 = u_rand * st->kept_sum;
  }
  const uint32_t n_runs = (len + kRun - 1) / kRun;
  const uint32_t t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint32_t r_first = blockIdx.x * kRunsPerBlock;
  if (r_first >= n_runs) return;  // uniform over the block
  double acc = 0.0;
  for (uint32_t r = t; r < r_first; r += kEwThreads) acc += rs[r];
  acc = wave_sum_f64(acc);
  if (lane == 0) red[w] = acc;
  __syncthreads();
  double pre = red[0] + red[1] + red[2] + red[3];
  const uint32_t r_wave = r_first + w * 4;
  for (uint32_t r = r_first; r < r_wave && r < n_runs; r++) pre += rs[r];
  for (uint32_t q = 0; q < 4; q++) {
    const uint32_t r = r_wave + q;
    if (r >= n_runs) break;
    const double est = DEC ? (double)s0 - pre : (double)s0 + pre;
    const float fe = (float)est;
    int ug = -149;
    if (fe > 0.0f && fe == fe && fe < __int_as_float(0x7f800000)) {
      uint32_t nn;
      mono_state(fe, &ug, &nn);
    }
    const int cu = max(-149, ug - 1);
    const uint32_t i = r * kRun + lane;
    const float term = i < len ? y[i] : 0.0f;
#pragma unroll
    for (int c = 0; c < 3; c++) {
      const MonoFn f = wave_total_fn(mono_elem(term, cu + c));
      if (lane == 0) {
        rp[pair_at(r, 1 + 2 * c)] = f.a0;
        rp[pair_at(r, 2 + 2 * c)] = f.a1;
      }
    }
    if (lane == 0) rp[pair_at(r, 0)] = (uint32_t)cu;
    pre += rs[r];
  }
}

// The walk over a long chain, 128 runs (8192 terms) per chunk. Waves 1-3
// stream chunks into an LDS ring by DMA (global_load_lds, 16 bytes per lane:
// the chunk's terms and its pairs, 36 KB) while wave 0 walks the chunk before
// them: each pass composes every lane's two runs' pairs at the current binade,
// scans them, and replays the first run that may leave the binade, reach the
// stop condition or miss the binade among its candidates, from its exact
// start (wave_chain over its 64 terms). `out` says what the result is:
// OUT_SUM: the softmax sum; OUT_TOPP: the top-p cutoff and kept sum
// (sampler.rs:135-146); OUT_DRAW: the drawn token (148-162).
constexpr int kWalkThreads = 256;
constexpr int kWalkAhead = 3;                    // chunks in flight while one is walked
constexpr int kWalkSlots = kWalkAhead + 1;
constexpr uint32_t kChunkRuns = 128;             // two per lane
constexpr uint32_t kChunkTerms = kChunkRuns * kRun;  // 8192
constexpr int kChunkPieces = (kChunkTerms * 4 + kPairRows * kChunkRuns * 4) / 1024;  // 36 copies of 1 KB
constexpr int kPiecesPerLoader = kChunkPieces / 3;                                   // 12 per loader wave
constexpr int kTermPieces = kChunkTerms * 4 / 1024;                                  // 32

struct WalkSlot {
  float terms[kChunkTerms];
  uint32_t pairs[2][kPairRows][64];  // the two pair blocks of the chunk's runs
};

// Loader wave w (1..3): its kPiecesPerLoader 1 KB pieces of chunk c into
// `slot`. Pieces of a chunk past the data copy the first piece instead (the
// copy is never read), so every loader issues the same count per chunk; the
// arrays are padded so a piece that starts inside the data stays inside the
// allocation.
__device__ __forceinline__ void walk_issue(const float* y, uint32_t len, const uint32_t* rp, uint32_t n_pair_blocks,
                                           uint32_t c, WalkSlot* slot) {
  const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int q = 0; q < kPiecesPerLoader; q++) {
    const uint32_t k = (w - 1) * kPiecesPerLoader + q;
    const char* src;
    if (k < (uint32_t)kTermPieces) {
      const uint64_t i = (uint64_t)c * kChunkTerms + k * 256 + lane * 4;
      src = (const char*)(y + (i < len ? i : 0));
    } else {
      const uint32_t blk = 2 * c + (k - kTermPieces) / 2;  // pair block (64 runs, 2 KB)
      const uint64_t i = (uint64_t)blk * (kPairRows * 64) + ((k - kTermPieces) & 1) * 256 + lane * 4;
      src = (const char*)(rp + (blk < n_pair_blocks ? i : 0));
    }
    __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)src, (RLH_LDS void*)((char*)slot + k * 1024), 16, 0,
                                     0);
  }
}

template <bool DEC>
__global__ void __launch_bounds__(kWalkThreads)
    k_run_walk(const float* y, uint32_t len, float s0, int from_state, float u_rand, const uint32_t* rp, int stop,
               float thr, int out, const uint32_t* ids, SdState* st) {
  __shared__ WalkSlot ring[kWalkSlots];
  __shared__ uint32_t done;
  const int t = (int)threadIdx.x, lane = t & 63, w = t >> 6;
  if (st->flags & F_NAN) {
    if (out == OUT_SUM && t == 0) st->sum = __int_as_float(0x7fc00000);
    return;
  }
  if (from_state) {
    len = st->cutoff;
    const float sum = st->kept_sum;
    if (sum <= 0.0f) {  // sampler.rs:152-154
      if (t == 0) {
        st->token = ids[0];
        st->rng_used = 0;
      }
      return;
    }
    s0 = u_rand * sum;  // sampler.rs:155
  }
  if (len == 0) {
    if (t == 0 && out == OUT_SUM) st->sum = s0;
    return;
  }
  const uint32_t n_runs = (len + kRun - 1) / kRun;
  const uint32_t n_pair_blocks = (n_runs + 63) / 64;
  const uint32_t n_chunks = (n_runs + kChunkRuns - 1) / kChunkRuns;
  if (t == 0) done = 0;
  if (w > 0) {
#pragma unroll
    for (int d = 0; d < kWalkAhead; d++) walk_issue(y, len, rp, n_pair_blocks, (uint32_t)d, &ring[d]);
  }
  float s = s0, val = s0;
  uint32_t idx = len;
  for (uint32_t c = 0; c < n_chunks; c++) {
    if (w > 0) wait_vmcnt<(kWalkAhead - 1) * kPiecesPerLoader>();  // this wave's pieces of chunk c have landed
    lds_barrier();  // every loader's
    if (w > 0) {
      // the slot of chunk c - 1, free since the barrier that ended it
      walk_issue(y, len, rp, n_pair_blocks, c + kWalkAhead, &ring[(c + kWalkAhead) % kWalkSlots]);
    } else {
      const WalkSlot& sl = ring[c % kWalkSlots];
      const uint32_t cb = c * kChunkRuns;
      // lane l owns runs cb + 2l and cb + 2l + 1
      int cu[2];
      MonoFn p[2][3];
      bool valid[2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const uint32_t li = (2 * (uint32_t)lane + h) & 63, blk = (2 * (uint32_t)lane + h) >> 6;
        valid[h] = cb + 2 * (uint32_t)lane + h < n_runs;
        cu[h] = (int)sl.pairs[blk][0][li];
#pragma unroll
        for (int k = 0; k < 3; k++) p[h][k] = MonoFn{sl.pairs[blk][1 + 2 * k][li], sl.pairs[blk][2 + 2 * k][li]};
      }
      uint32_t r0 = cb;  // first run not yet walked
      for (;;) {
        int u;
        uint32_t N;
        chain_state<DEC>(s, &u, &N);
        // a run whose candidates miss the current binade is treated as one
        // that may leave it: the estimate puts it past a crossing, and if it
        // is the first such run it is replayed from its exact start
        MonoFn fr[2];
        bool miss[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
          fr[h] = mono_identity();
          miss[h] = false;
          if (valid[h] && cb + 2 * (uint32_t)lane + h >= r0) {
            const int d = u - cu[h];
            if (d == 0)
              fr[h] = p[h][0];
            else if (d == 1)
              fr[h] = p[h][1];
            else if (d == 2)
              fr[h] = p[h][2];
            else
              miss[h] = true;
          }
        }
        const MonoFn f = mono_then(fr[0], fr[1]);
        const MonoFn incl = wave_scan_fn(f);
        const uint32_t a = mono_apply(wave_excl_fn(incl), N);
        const uint32_t nl = DEC ? N - a : N + a;
        // the lane's first run that may leave, 2 when neither
        const uint32_t b0 = mono_apply(fr[0], nl);
        const uint32_t n1 = DEC ? nl - b0 : nl + b0;
        const uint32_t b1 = mono_apply(fr[1], n1);
        bool l0v, l1v;
        if (DEC) {
          l0v = mono_dec_leaves(u, N, a + b0);
          l1v = mono_dec_leaves(u, N, a + b0 + b1);
        } else {
          const uint64_t lim = inc_limit(u, stop, thr);
          l0v = (uint64_t)N + a + b0 >= lim;
          l1v = (uint64_t)N + a + b0 + b1 >= lim;
        }
        const int first = (l0v || miss[0]) ? 0 : ((l1v || miss[1]) ? 1 : 2);
        const uint64_t mask = __ballot(first < 2);
        if (mask == 0) {
          const uint32_t tot = mono_apply(MonoFn{readlane_u32(incl.a0, 63), readlane_u32(incl.a1, 63)}, N);
          s = mono_value(u, DEC ? N - tot : N + tot);
          break;
        }
        const int lc = (int)__builtin_ctzll(mask);
        const int hc = (int)readlane_u32((uint32_t)first, lc);
        const uint32_t run = cb + 2 * (uint32_t)lc + (uint32_t)hc;
        const uint32_t rlen = min(kRun, len - run * kRun);
        const float start = mono_value(u, readlane_u32(hc ? n1 : nl, lc));
        const float* tr = sl.terms + (2 * lc + hc) * kRun;
        float v;
        const uint32_t j = wave_chain<DEC, 1>([=](uint32_t i) { return tr[i]; }, rlen, start, stop, thr, &v);
        if (j < rlen) {
          idx = run * kRun + j;
          val = v;
          break;
        }
        s = v;
        r0 = run + 1;
        if (r0 >= cb + kChunkRuns || r0 >= n_runs) break;
      }
      if (lane == 0 && idx != len) done = 1;
    }
    lds_barrier();  // wave 0 is done with the slot and `done` is visible
    if (done) break;
  }
  wait_vmcnt<0>();  // no copy into this block's LDS outlives it
  if (t != 0) return;
  if (idx == len) val = s;
  if (out == OUT_SUM) {
    st->sum = val;
  } else if (out == OUT_TOPP) {
    st->cutoff = idx < len ? idx + 1 : len;
    st->kept_sum = val;
  } else {
    st->token = idx < len ? ids[idx] : ids[len - 1];
    st->rng_used = 1;
  }
}

// p = e * (1/sum) when sum > 0; the histogram of p's bits 29..22 and the f64
// mass of each bin.
__global__ void __launch_bounds__(kEwThreads)
    k_sd_norm(float* x, uint32_t n, const SdState* st, uint32_t* hist, double* mass, int do_hist) {
  __shared__ uint32_t h[256];
  __shared__ double hm[256];
  const uint32_t t = threadIdx.x, lo = blockIdx.x * kEwBlock;
  const float sum = st->sum;
  const bool scale = sum > 0.0f;
  const float inv = scale ? 1.0f / sum : 1.0f;
  do_hist = do_hist && scale;
  if (do_hist) {
    h[t] = 0;
    hm[t] = 0.0;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t k = 0; k < kEwPer; k++) {
    const uint32_t i = lo + k * kEwThreads + t;
    if (i < n) {
      float p = x[i];
      if (scale) {
        p = p * inv;
        x[i] = p;
      }
      if (do_hist) {
        const uint32_t d = min(__float_as_uint(p) >> 22, 255u);
        atomicAdd(&h[d], 1u);
        atomicAdd(&hm[d], (double)p);
      }
    }
  }
  if (!do_hist) return;
  __syncthreads();
  if (h[t]) {
    atomicAdd(&hist[t], h[t]);
    atomicAdd(&mass[t], hm[t]);
  }
}

// The threshold digit and the candidates at or above it.
//   top-k (k >= 1): the largest digit d with count(digit >= d) >= k;
//   top-p only:     the largest d whose prefix mass reaches top_p with a
//                   margin above the f32 running sum's drift over 4096 terms
//                   (2.5e-4 relative), so the cutoff lies inside the prefix;
//                   failing that, the longest prefix of at most cap values.
// More than cap candidates (or none): F_OVERFLOW, the radix sort takes over.
__global__ void __launch_bounds__(kEwThreads)
    k_sd_candidates(const float* p, uint32_t n, const uint32_t* hist, const double* mass, uint32_t k, float top_p,
                    uint32_t cap, SdState* st, uint64_t* cand) {
  __shared__ uint32_t wc[kEwThreads / 64];
  __shared__ double wm[kEwThreads / 64];
  __shared__ uint32_t sel[2];  // [0]: candidates at the threshold, [1]: this block's base
  __shared__ uint32_t blk;
  const uint32_t t = threadIdx.x, lo = blockIdx.x * kEwBlock, lane = t & 63, w = t >> 6;
  if (st->flags & F_NAN) return;
  // thread t holds bin 255 - t: an inclusive scan over t gives the count and
  // mass of all bins >= 255 - t
  uint32_t c = hist[255 - t];
  double msum = mass[255 - t];
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t c2 = __shfl_up(c, off);
    const double m2 = __shfl_up(msum, off);
    if ((int)lane >= off) {
      c += c2;
      msum += m2;
    }
  }
  if (lane == 63) {
    wc[w] = c;
    wm[w] = msum;
  }
  if (t == 0) blk = 0;
  __syncthreads();
  for (uint32_t i = 0; i < w; i++) {
    c += wc[i];
    msum += wm[i];
  }
  // counts and masses of the suffixes fall as the bin rises, so each
  // threshold is one less than the number of bins meeting its condition
  uint32_t dstar;
  if (k >= 1) {
    dstar = (uint32_t)__syncthreads_count(c >= k) - 1u;
  } else {
    const uint32_t reach = (uint32_t)__syncthreads_count(msum >= (double)top_p * (1.0 + kTopPMargin));
    dstar = reach ? reach - 1u : (uint32_t)__syncthreads_count(c > cap);
  }
  if (dstar < 256 && t == 255 - dstar) sel[0] = c;
  __syncthreads();
  const uint32_t m = dstar < 256 ? sel[0] : 0u;
  if (m == 0 || m > cap) {
    if (blockIdx.x == 0 && t == 0) atomicOr(&st->flags, F_OVERFLOW);
    return;
  }
  uint64_t key[kEwPer];
  uint32_t mine = 0;
#pragma unroll
  for (uint32_t kk = 0; kk < kEwPer; kk++) {
    const uint32_t i = lo + kk * kEwThreads + t;
    key[kk] = 0;
    if (i < n) {
      const uint32_t b = __float_as_uint(p[i]);
      if (min(b >> 22, 255u) >= dstar) {
        key[kk] = ((uint64_t)b << 32) | (uint64_t)(~i);
        mine++;
      }
    }
  }
  const uint32_t off = mine ? atomicAdd(&blk, mine) : 0u;
  __syncthreads();
  if (t == 0) sel[1] = blk ? atomicAdd(&st->n_cand, blk) : 0u;
  __syncthreads();
  uint32_t at = sel[1] + off;
#pragma unroll
  for (uint32_t kk = 0; kk < kEwPer; kk++)
    if (key[kk] && at < cap) cand[at++] = key[kk];
}

// Bitonic sort of P (a power of two, 2..64) keys held one per lane,
// descending.
__device__ __forceinline__ uint64_t wave_bitonic_desc(uint64_t key, int lane, uint32_t P) {
  for (uint32_t size = 2; size <= P; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t other = __shfl_xor(key, (int)stride);
      const bool desc = (lane & size) == 0;
      const bool lower = (lane & stride) == 0;
      // the lower lane of a pair keeps the larger key in a descending block
      const bool keep_max = lower == desc;
      key = keep_max ? (key > other ? key : other) : (key < other ? key : other);
    }
  }
  return key;
}

// Sorts the candidates (p descending, id ascending), then top-p and the draw
// over the kept list with wave 0. 256 threads.
__global__ void __launch_bounds__(kEwThreads)
    k_sd_pick_candidates(const uint64_t* cand, uint32_t n, uint32_t k, float top_p, int apply_p, float u_rand,
                         SdState* st) {
  __shared__ uint64_t keys[kCandMax];
  if (st->flags & (F_NAN | F_OVERFLOW)) return;
  const uint32_t t = threadIdx.x;
  const int lane = (int)(t & 63);
  const uint32_t m = min(st->n_cand, kCandMax);
  uint32_t P = 2;
  while (P < m) P <<= 1;
  if (P <= 64) {
    if (t >= 64) return;
    uint64_t key = (uint32_t)lane < m ? cand[lane] : 0ull;
    key = wave_bitonic_desc(key, lane, P);
    keys[lane] = key;
  } else {
    for (uint32_t i = t; i < P; i += kEwThreads) keys[i] = i < m ? cand[i] : 0ull;
    __syncthreads();
    for (uint32_t size = 2; size <= P; size <<= 1) {
      for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
        for (uint32_t q = t; q < P / 2; q += kEwThreads) {
          const uint32_t i = 2 * stride * (q / stride) + (q % stride), j = i + stride;
          const bool desc = (i & size) == 0;
          const uint64_t a = keys[i], b = keys[j];
          if ((a < b) == desc) {
            keys[i] = b;
            keys[j] = a;
          }
        }
        __syncthreads();
      }
    }
    if (t >= 64) return;
  }
  // wave 0 from here on (keys[] written by this wave, or before the last barrier)
  const bool topk = k >= 1 && k < n;
  const uint32_t L = topk ? k : m;
  const bool complete = topk || m == n;
  auto y = [&](uint32_t j) { return __uint_as_float((uint32_t)(keys[j] >> 32)); };
  float sum;
  uint32_t cutoff = L;
  if (apply_p) {  // sampler.rs:135-146
    float v;
    const uint32_t j = wave_chain<false, 4>(y, L, 0.0f, STOP_GE, top_p, &v);
    if (j < L) {
      cutoff = j + 1;
    } else if (!complete) {
      if (lane == 0) atomicOr(&st->flags, F_SHORT);
      return;
    }
    sum = v;
  } else {
    wave_chain<false, 4>(y, L, 0.0f, STOP_NONE, 0.0f, &sum);
  }
  uint32_t tok;
  uint32_t used = 0;
  if (sum <= 0.0f) {  // sampler.rs:152-154
    tok = ~(uint32_t)keys[0];
  } else {
    used = 1;
    const float r0 = u_rand * sum;  // sampler.rs:155
    float v;
    const uint32_t j = wave_chain<true, 4>(y, cutoff, r0, STOP_LE0, 0.0f, &v);
    tok = ~(uint32_t)keys[j < cutoff ? j : cutoff - 1];
  }
  if (lane == 0) {
    st->token = tok;
    st->rng_used = used;
    st->cutoff = cutoff;
    st->kept_sum = sum;
  }
}

__global__ void k_sd_iota(uint32_t* ids, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) ids[i] = i;
}

}  // namespace

}  // namespace rlh

using namespace rlh;

struct rlh_dsampler {
  int device = 0;
  uint64_t cap = 0;          // largest n
  uint32_t nb_cap = 0;       // blocks of the elementwise kernels at cap
  uint32_t cand_cap = kCandMax;
  float* x = nullptr;        // scaled logits -> exponentials -> probabilities
  uint32_t* keys2 = nullptr; // sorted probabilities (bits)
  uint32_t* ids = nullptr;   // 0..cap-1
  uint32_t* ids2 = nullptr;  // ids in sorted order
  uint64_t* cand = nullptr;  // [kCandMax]
  float* part = nullptr;     // block maxima / argmax partial values
  uint32_t* part_i = nullptr;
  uint32_t* hist = nullptr;  // [256]
  double* mass = nullptr;    // [256]
  double* rs = nullptr;      // run sums [cap / 64]
  uint32_t* rp = nullptr;    // run pairs, 2 KB per chunk of 64 runs
  SdState* st = nullptr;
  SdState* host = nullptr;   // pinned
  uint32_t* tok = nullptr;   // device argmax result
  uint32_t* pen = nullptr;
  uint32_t* pen_host = nullptr;  // pinned staging
  uint64_t pen_cap = 0;
  void* sort_tmp = nullptr;
  size_t sort_bytes = 0;
  uint32_t last_path = 0;
};

namespace {

constexpr uint32_t kArgmaxParts = 256;

#define SDCHK(expr)                                                                                  \
  do {                                                                                               \
    hipError_t e_ = (expr);                                                                          \
    if (e_ != hipSuccess) return set_error(RLH_EDEVICE, (std::string(#expr) + ": " + hipGetErrorString(e_)).c_str()); \
  } while (0)

void ds_free(rlh_dsampler* ds) {
  void* ptrs[] = {ds->x, ds->keys2, ds->ids, ds->ids2, ds->cand, ds->part, ds->part_i, ds->hist, ds->mass, ds->rs,
                  ds->rp, ds->st, ds->tok, ds->pen, ds->sort_tmp};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  if (ds->host) (void)hipHostFree(ds->host);
  if (ds->pen_host) (void)hipHostFree(ds->pen_host);
  delete ds;
}

int check_device(const rlh_dsampler* ds) {
  int dev = -1;
  SDCHK(hipGetDevice(&dev));
  if (dev != ds->device) return set_error(RLH_EINVAL, "device sampler used on another device than it was made on");
  return RLH_OK;
}

// Distinct ids < n of the penalty window, sorted (sampler.rs:87-95).
void penalty_ids(const rlh_sampling_params& p, const uint32_t* recent, uint64_t n_recent, uint64_t n,
                 std::vector<uint32_t>* out) {
  out->clear();
  if (p.repetition_penalty == 1.0f) return;
  const uint64_t start = p.repeat_last_n == 0 || n_recent <= p.repeat_last_n ? 0 : n_recent - p.repeat_last_n;
  for (uint64_t k = start; k < n_recent; k++)
    if (recent[k] < n) out->push_back(recent[k]);
  std::sort(out->begin(), out->end());
  out->erase(std::unique(out->begin(), out->end()), out->end());
}

int upload_penalty(rlh_dsampler* ds, const std::vector<uint32_t>& ids, hipStream_t s) {
  if (ids.empty()) return RLH_OK;
  if (ids.size() > ds->pen_cap) {
    SDCHK(hipStreamSynchronize(s));
    if (ds->pen) (void)hipFree(ds->pen);
    if (ds->pen_host) (void)hipHostFree(ds->pen_host);
    ds->pen = nullptr;
    ds->pen_host = nullptr;
    ds->pen_cap = 0;
    const uint64_t cap = std::max<uint64_t>(ids.size(), 1024);
    if (hipMalloc((void**)&ds->pen, cap * 4) != hipSuccess || hipHostMalloc((void**)&ds->pen_host, cap * 4) != hipSuccess)
      return set_error(RLH_ENOMEM, "penalty list allocation");
    ds->pen_cap = cap;
  }
  // the previous call synchronized before returning, so the staging buffer
  // is free again
  std::copy(ids.begin(), ids.end(), ds->pen_host);
  SDCHK(hipMemcpyAsync(ds->pen, ds->pen_host, ids.size() * 4, hipMemcpyHostToDevice, s));
  return RLH_OK;
}

uint32_t ew_blocks(uint64_t n) { return (uint32_t)((n + kEwBlock - 1) / kEwBlock); }
uint32_t run_blocks(uint64_t len) {
  const uint64_t runs = (len + kRun - 1) / kRun;
  return (uint32_t)std::max<uint64_t>(1, (runs + kRunsPerBlock - 1) / kRunsPerBlock);
}

// Launches scale (+ penalty) for n values of `in` into ds->x.
int launch_scale(rlh_dsampler* ds, const float* in, uint64_t n, float inv_t, bool scale, float rp, uint32_t n_pen,
                 hipStream_t s) {
  hipLaunchKernelGGL(k_sd_scale, dim3(ew_blocks(n)), dim3(kEwThreads), 0, s, in, ds->x, (uint32_t)n, inv_t,
                     scale ? 1 : 0, rp, ds->pen, n_pen, ds->part, ds->st, ds->hist, ds->mass);
  SDCHK(hipGetLastError());
  return RLH_OK;
}

// exp, sum, normalize on ds->x (after launch_scale).
int launch_softmax_tail(rlh_dsampler* ds, uint64_t n, bool hist, hipStream_t s) {
  const uint32_t nb = ew_blocks(n);
  hipLaunchKernelGGL(k_sd_exp, dim3(nb), dim3(kEwThreads), 0, s, ds->x, (uint32_t)n, ds->part, nb, ds->st, ds->rs);
  hipLaunchKernelGGL(k_run_pairs<false>, dim3(run_blocks(n)), dim3(kEwThreads), 0, s, ds->x, (uint32_t)n, 0.0f, 0,
                     0.0f, ds->st, ds->rs, ds->rp);
  hipLaunchKernelGGL(k_run_walk<false>, dim3(1), dim3(kWalkThreads), 0, s, ds->x, (uint32_t)n, 0.0f, 0, 0.0f, ds->rp,
                     (int)STOP_NONE, 0.0f, (int)OUT_SUM, ds->ids, ds->st);
  hipLaunchKernelGGL(k_sd_norm, dim3(nb), dim3(kEwThreads), 0, s, ds->x, (uint32_t)n, ds->st, ds->hist, ds->mass,
                     hist ? 1 : 0);
  SDCHK(hipGetLastError());
  return RLH_OK;
}

int launch_full_sort_pick(rlh_dsampler* ds, uint64_t n, uint32_t k, float top_p, int apply_p, float u,
                          hipStream_t s) {
  size_t bytes = ds->sort_bytes;
  SDCHK(rocprim::radix_sort_pairs_desc(ds->sort_tmp, bytes, reinterpret_cast<const uint32_t*>(ds->x), ds->keys2,
                                       ds->ids, ds->ids2, (uint32_t)n, 0u, 30u, s));
  const uint32_t L = (k >= 1 && k < n) ? k : (uint32_t)n;
  const float* y = reinterpret_cast<const float*>(ds->keys2);
  hipLaunchKernelGGL(k_run_sums, dim3(ew_blocks(L)), dim3(kEwThreads), 0, s, y, L, ds->rs);
  hipLaunchKernelGGL(k_run_pairs<false>, dim3(run_blocks(L)), dim3(kEwThreads), 0, s, y, L, 0.0f, 0, 0.0f, ds->st,
                     ds->rs, ds->rp);
  hipLaunchKernelGGL(k_run_walk<false>, dim3(1), dim3(kWalkThreads), 0, s, y, L, 0.0f, 0, 0.0f, ds->rp,
                     apply_p ? (int)STOP_GE : (int)STOP_NONE, top_p, (int)OUT_TOPP, ds->ids2, ds->st);
  hipLaunchKernelGGL(k_run_pairs<true>, dim3(run_blocks(L)), dim3(kEwThreads), 0, s, y, L, 0.0f, 1, u, ds->st,
                     ds->rs, ds->rp);
  hipLaunchKernelGGL(k_run_walk<true>, dim3(1), dim3(kWalkThreads), 0, s, y, L, 0.0f, 1, u, ds->rp, (int)STOP_LE0, 0.0f,
                     (int)OUT_DRAW, ds->ids2, ds->st);
  SDCHK(hipGetLastError());
  return RLH_OK;
}

int read_state(rlh_dsampler* ds, hipStream_t s) {
  SDCHK(hipMemcpyAsync(ds->host, ds->st, sizeof(SdState), hipMemcpyDeviceToHost, s));
  SDCHK(hipStreamSynchronize(s));
  return RLH_OK;
}

}  // namespace

namespace rlh {

int dsampler_sample(rlh_dsampler* ds, const float* logits, uint64_t n, const rlh_sampling_params& p,
                    const uint32_t* recent, uint64_t n_recent, uint64_t* rng_state, uint32_t* token, hipStream_t s) {
  int rc = check_device(ds);
  if (rc) return rc;
  if (n > ds->cap) return set_error(RLH_EINVAL, "n above the device sampler's capacity");
  ds->last_path = 0;
  if (n == 0) {  // sampler.rs:58-60
    *token = 0;
    return RLH_OK;
  }
  const bool greedy = p.temperature <= 0.0f;
  if (greedy && p.repetition_penalty == 1.0f) {  // sampler.rs:62-70
    launch_argmax(s, logits, (uint32_t)n, ds->part, ds->part_i, kArgmaxParts, ds->tok, nullptr, nullptr, nullptr);
    SDCHK(hipGetLastError());
    SDCHK(hipMemcpyAsync(&ds->host->token, ds->tok, 4, hipMemcpyDeviceToHost, s));
    SDCHK(hipMemcpyAsync(&ds->host->sum, logits, 4, hipMemcpyDeviceToHost, s));
    SDCHK(hipStreamSynchronize(s));
    // the loop starts at index 0, so a NaN there is never beaten
    *token = ds->host->sum != ds->host->sum ? 0u : ds->host->token;
    ds->last_path = RLH_DSAMPLER_PATH_GREEDY;
    return RLH_OK;
  }
  std::vector<uint32_t> pen;
  penalty_ids(p, recent, n_recent, n, &pen);
  if ((rc = upload_penalty(ds, pen, s))) return rc;
  if (greedy) {  // sampler.rs:104-112: the first maximum of the penalized logits
    if ((rc = launch_scale(ds, logits, n, 1.0f, false, p.repetition_penalty, (uint32_t)pen.size(), s))) return rc;
    launch_argmax(s, ds->x, (uint32_t)n, ds->part, ds->part_i, kArgmaxParts, ds->tok, nullptr, nullptr, nullptr);
    SDCHK(hipGetLastError());
    SDCHK(hipMemcpyAsync(&ds->host->token, ds->tok, 4, hipMemcpyDeviceToHost, s));
    SDCHK(hipMemcpyAsync(&ds->host->sum, ds->x, 4, hipMemcpyDeviceToHost, s));
    SDCHK(hipStreamSynchronize(s));
    *token = ds->host->sum != ds->host->sum ? 0u : ds->host->token;
    ds->last_path = RLH_DSAMPLER_PATH_GREEDY;
    return RLH_OK;
  }
  if (n == 1) {  // one token: every branch returns it after one draw
    (void)sampler_next_f32(rng_state);
    *token = 0;
    return RLH_OK;
  }
  const float inv_t = 1.0f / p.temperature;
  const uint32_t k = (p.top_k == 0 || p.top_k > n) ? 0u : p.top_k;  // 0: all
  const int apply_p = p.top_p > 0.0f && p.top_p < 1.0f ? 1 : 0;
  const bool cand = ds->cand_cap > 0 && ((k >= 1 && k < n && k <= ds->cand_cap) || (k == 0 && apply_p));
  uint64_t rng = *rng_state;
  const float u = sampler_next_f32(&rng);
  if ((rc = launch_scale(ds, logits, n, inv_t, true, p.repetition_penalty, (uint32_t)pen.size(), s))) return rc;
  if ((rc = launch_softmax_tail(ds, n, cand, s))) return rc;
  if (cand) {
    const uint32_t nb = ew_blocks(n);
    hipLaunchKernelGGL(k_sd_candidates, dim3(nb), dim3(kEwThreads), 0, s, ds->x, (uint32_t)n, ds->hist, ds->mass, k,
                       p.top_p, ds->cand_cap, ds->st, ds->cand);
    hipLaunchKernelGGL(k_sd_pick_candidates, dim3(1), dim3(kEwThreads), 0, s, ds->cand, (uint32_t)n, k, p.top_p,
                       apply_p, u, ds->st);
    SDCHK(hipGetLastError());
    ds->last_path = RLH_DSAMPLER_PATH_CANDIDATES;
  } else {
    if ((rc = launch_full_sort_pick(ds, n, k, p.top_p, apply_p, u, s))) return rc;
    ds->last_path = RLH_DSAMPLER_PATH_SORT;
  }
  if ((rc = read_state(ds, s))) return rc;
  if (ds->host->flags & F_NAN)
    return set_error(RLH_EINVAL, "logits hold NaN or infinity after penalty and temperature (the reference's "
                                 "sort cannot order them)");
  if (cand && (ds->host->flags & (F_OVERFLOW | F_SHORT))) {
    if ((rc = launch_full_sort_pick(ds, n, k, p.top_p, apply_p, u, s))) return rc;
    if ((rc = read_state(ds, s))) return rc;
    ds->last_path = RLH_DSAMPLER_PATH_SORT | RLH_DSAMPLER_PATH_FALLBACK;
  }
  if (ds->host->rng_used) *rng_state = rng;
  *token = ds->host->token;
  return RLH_OK;
}

int dsampler_softmax(rlh_dsampler* ds, float* x, uint64_t n, hipStream_t s) {
  int rc = check_device(ds);
  if (rc) return rc;
  if (n > ds->cap) return set_error(RLH_EINVAL, "n above the device sampler's capacity");
  if (n == 0) return RLH_OK;
  if ((rc = launch_scale(ds, x, n, 1.0f, false, 1.0f, 0, s))) return rc;
  if ((rc = launch_softmax_tail(ds, n, false, s))) return rc;
  SDCHK(hipMemcpyAsync(x, ds->x, n * 4, hipMemcpyDeviceToDevice, s));
  return RLH_OK;
}

}  // namespace rlh

extern "C" {

int rlh_dsampler_create(uint64_t max_n, rlh_dsampler** out) {
  if (!out) return set_error(RLH_EINVAL, "null argument");
  *out = nullptr;
  if (max_n == 0 || max_n > 0xffffffffull - kEwBlock) return set_error(RLH_EINVAL, "max_n out of range");
  rlh_dsampler* ds = new rlh_dsampler();
  if (hipGetDevice(&ds->device) != hipSuccess) {
    delete ds;
    return set_error(RLH_EDEVICE, "hipGetDevice");
  }
  ds->cap = max_n;
  ds->nb_cap = ew_blocks(max_n);
  const uint32_t nparts = std::max(ds->nb_cap, kArgmaxParts);
  const uint64_t runs = (uint64_t)ds->nb_cap * (kEwBlock / kRun);  // run slots of whole blocks
  const uint64_t chunks = (runs + 63) / 64;  // pair blocks of 64 runs
  // the chain inputs (x, keys2) get 16 bytes of padding: the walk copies
  // 16-byte pieces that may start at any of the last three values
  bool ok = hipMalloc((void**)&ds->x, max_n * 4 + 16) == hipSuccess &&
            hipMalloc((void**)&ds->keys2, max_n * 4 + 16) == hipSuccess &&
            hipMalloc((void**)&ds->ids, max_n * 4) == hipSuccess && hipMalloc((void**)&ds->ids2, max_n * 4) == hipSuccess &&
            hipMalloc((void**)&ds->cand, kCandMax * 8) == hipSuccess &&
            hipMalloc((void**)&ds->part, (size_t)nparts * 4) == hipSuccess &&
            hipMalloc((void**)&ds->part_i, (size_t)nparts * 4) == hipSuccess &&
            hipMalloc((void**)&ds->hist, 256 * 4) == hipSuccess && hipMalloc((void**)&ds->mass, 256 * 8) == hipSuccess &&
            hipMalloc((void**)&ds->rs, runs * 8) == hipSuccess && hipMalloc((void**)&ds->rp, chunks * kPairRows * 64 * 4) == hipSuccess &&
            hipMalloc((void**)&ds->st, sizeof(SdState)) == hipSuccess && hipMalloc((void**)&ds->tok, 4) == hipSuccess &&
            hipHostMalloc((void**)&ds->host, sizeof(SdState)) == hipSuccess;
  if (ok) {
    size_t bytes = 0;
    ok = rocprim::radix_sort_pairs_desc(nullptr, bytes, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                        (const uint32_t*)nullptr, (uint32_t*)nullptr, (uint32_t)max_n, 0u, 30u) ==
             hipSuccess &&
         hipMalloc(&ds->sort_tmp, std::max<size_t>(bytes, 16)) == hipSuccess;
    ds->sort_bytes = bytes;
  }
  if (!ok) {
    ds_free(ds);
    return set_error(RLH_ENOMEM, "device sampler allocation");
  }
  hipLaunchKernelGGL(k_sd_iota, dim3((uint32_t)((max_n + 255) / 256)), dim3(256), 0, 0, ds->ids, (uint32_t)max_n);
  if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    ds_free(ds);
    return set_error(RLH_EDEVICE, "device sampler init");
  }
  *out = ds;
  return RLH_OK;
}

void rlh_dsampler_destroy(rlh_dsampler* ds) {
  if (!ds) return;
  (void)hipDeviceSynchronize();
  ds_free(ds);
}

int rlh_dsampler_sample(rlh_dsampler* ds, const float* logits, uint64_t n, const rlh_sampling_params* p,
                        const uint32_t* recent, uint64_t n_recent, uint64_t* rng_state, uint32_t* token,
                        void* stream) {
  if (!ds || !p || !rng_state || !token || (n && !logits) || (n_recent && !recent))
    return set_error(RLH_EINVAL, "null argument");
  return dsampler_sample(ds, logits, n, *p, recent, n_recent, rng_state, token, (hipStream_t)stream);
}

int rlh_dsampler_softmax(rlh_dsampler* ds, float* x, uint64_t n, void* stream) {
  if (!ds || (n && !x)) return set_error(RLH_EINVAL, "null argument");
  return dsampler_softmax(ds, x, n, (hipStream_t)stream);
}

int rlh_dsampler_set_candidate_cap(rlh_dsampler* ds, uint32_t cap) {
  if (!ds) return set_error(RLH_EINVAL, "null argument");
  if (cap > kCandMax) return set_error(RLH_EINVAL, "candidate cap above 4096");
  ds->cand_cap = cap;
  return RLH_OK;
}

uint32_t rlh_dsampler_last_path(const rlh_dsampler* ds) { return ds ? ds->last_path : 0u; }

}  // extern "C"
