// sampler.cpp — host restatement of the reference's token sampler
// (src/sampler.rs:29-163) and of the generation loop around it
// (src/model.rs:741-776), for callers that sample with temperature, top-k,
// top-p and a repetition penalty.
//
// The sampler is host code in the reference as well: it runs once per token
// on 151936 logits, next to a decode step of milliseconds. Arithmetic is
// f32 in the reference's order (softmax_inplace, ops.rs:398-419, with the
// platform expf), compiled without FMA contraction.
//
// Top-k keeps the k largest probabilities and orders them by descending
// probability. The reference selects them with select_nth_unstable_by and
// then sorts stably, so the order of exactly equal probabilities follows the
// internals of Rust's selection; here equal probabilities are ordered by
// token id (lower first). The two agree whenever the kept probabilities are
// distinct.
#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../../include/rlh.h"
#include "sampler.h"

#define RLH_EXPF_QUAL inline
#include "expf_glibc.h"

namespace rlh {

namespace {

// Sampler::next_u64 (sampler.rs:40-48): xorshift64*.
uint64_t next_u64(uint64_t* state) {
  uint64_t x = *state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  *state = x;
  return x * 0x2545F4914F6CDD1DULL;
}

// Sampler::next_f32 (sampler.rs:51-54): uniform in [0, 1) from 24 bits.
float next_f32(uint64_t* state) { return (float)(next_u64(state) >> 40) / (float)(1u << 24); }

// Index of the first maximum under strict '>' (sampler.rs:62-70, 104-112).
uint32_t first_max(const float* v, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; i++)
    if (v[i] > v[best]) best = i;
  return (uint32_t)best;
}

// expf of glibc on x86-64 with FMA (the variant f32::exp reaches there), the
// method of expf_glibc.h four lanes per AVX2 step; lanes with |x| >= 88 or
// NaN take the library call. tests/test_host_expf.py checks this path and
// expf_glibc_t (the kernels' expf) against the library on every float.
const uint64_t kExp2T[32] = RLH_EXP2_TABLE_INIT;

// x[i] = expf(x[i] - mx) for i < n.
__attribute__((target("avx2,fma"))) void exp_shift_avx2(float* x, size_t n, float mx) {
  const __m256d inv_ln2n = _mm256_set1_pd(RLH_EXPF_INV_LN2_N);
  const __m256d shift = _mm256_set1_pd(RLH_EXPF_SHIFT);
  const __m256d c0 = _mm256_set1_pd(RLH_EXPF_C0);
  const __m256d c1 = _mm256_set1_pd(RLH_EXPF_C1);
  const __m256d c2 = _mm256_set1_pd(RLH_EXPF_C2);
  const __m256d one = _mm256_set1_pd(1.0);
  const __m128 vmx = _mm_set1_ps(mx);
  const __m128i lim = _mm_set1_epi32(0x42b);
  size_t i = 0;
  for (; i + 4 <= n; i += 4) {
    const __m128 xs = _mm_sub_ps(_mm_loadu_ps(x + i), vmx);
    const __m128i top = _mm_and_si128(_mm_srli_epi32(_mm_castps_si128(xs), 20), _mm_set1_epi32(0x7ff));
    if (_mm_movemask_epi8(_mm_cmpgt_epi32(lim, top)) != 0xffff) {  // a lane with |x| >= 88 or NaN
      float v[4];
      _mm_storeu_ps(v, xs);
      for (int k = 0; k < 4; k++) x[i + k] = expf(v[k]);
      continue;
    }
    const __m256d xd = _mm256_cvtps_pd(xs);
    __m256d kd = _mm256_fmadd_pd(inv_ln2n, xd, shift);
    const __m256i ki = _mm256_castpd_si256(kd);
    kd = _mm256_sub_pd(kd, shift);
    const __m256d r = _mm256_fmsub_pd(inv_ln2n, xd, kd);
    const __m256i idx = _mm256_and_si256(ki, _mm256_set1_epi64x(31));
    const __m256i t = _mm256_add_epi64(_mm256_i64gather_epi64((const long long*)kExp2T, idx, 8),
                                       _mm256_slli_epi64(ki, 47));
    const __m256d sc = _mm256_castsi256_pd(t);
    const __m256d z = _mm256_fmadd_pd(c0, r, c1);
    const __m256d r2 = _mm256_mul_pd(r, r);
    __m256d y = _mm256_fmadd_pd(c2, r, one);
    y = _mm256_fmadd_pd(z, r2, y);
    y = _mm256_mul_pd(y, sc);
    _mm_storeu_ps(x + i, _mm256_cvtpd_ps(y));
  }
  for (; i < n; i++) x[i] = expf(x[i] - mx);
}

// x[i] *= f (each product rounded once, as the scalar loop).
__attribute__((target("avx2,fma"))) void scale_avx2(float* x, size_t n, float f) {
  const __m256 vf = _mm256_set1_ps(f);
  size_t i = 0;
  for (; i + 8 <= n; i += 8) _mm256_storeu_ps(x + i, _mm256_mul_ps(_mm256_loadu_ps(x + i), vf));
  for (; i < n; i++) x[i] *= f;
}

// The reference's max (ops.rs:402-407): x[0], then every later v > max. A
// NaN in x[0] stays; later NaNs never compare greater and are skipped, as
// max_ps(v, acc) skips a NaN v. Equal zeros of either sign give the same
// exponentials, so which one is kept does not matter.
__attribute__((target("avx2,fma"))) float max_ref_avx2(const float* x, size_t n) {
  if (x[0] != x[0]) return x[0];
  __m256 acc = _mm256_set1_ps(x[0]);
  size_t i = 1;
  for (; i + 8 <= n; i += 8) acc = _mm256_max_ps(_mm256_loadu_ps(x + i), acc);
  float v[8];
  _mm256_storeu_ps(v, acc);
  float mx = v[0];
  for (int k = 1; k < 8; k++) mx = v[k] > mx ? v[k] : mx;
  for (; i < n; i++)
    if (x[i] > mx) mx = x[i];
  return mx;
}

// First index at or after i whose value is >= thr (n when none): the top-k
// scan skips eight values per compare while none can enter the list.
__attribute__((target("avx2,fma"))) size_t next_candidate_avx2(const float* x, size_t i, size_t n, float thr) {
  const __m256 vt = _mm256_set1_ps(thr);
  for (; i + 8 <= n; i += 8)
    if (_mm256_movemask_ps(_mm256_cmp_ps(_mm256_loadu_ps(x + i), vt, _CMP_GE_OQ))) break;
  for (; i < n; i++)
    if (x[i] >= thr) return i;
  return n;
}

bool have_avx2_fma() {
  static const bool ok = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  return ok;
}

// ops::softmax_inplace (ops.rs:398-419): the exponentials first (they are
// independent), then the sum in index order as the reference adds them.
void softmax_ref(float* x, size_t n) {
  if (n == 0) return;
  const bool vec = have_avx2_fma();
  float mx = x[0];
  if (vec) {
    mx = max_ref_avx2(x, n);
    exp_shift_avx2(x, n, mx);
  } else {
    for (size_t i = 1; i < n; i++)
      if (x[i] > mx) mx = x[i];
    for (size_t i = 0; i < n; i++) x[i] = expf(x[i] - mx);
  }
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) sum += x[i];
  if (sum > 0.0f) {
    const float inv = 1.0f / sum;
    if (vec)
      scale_avx2(x, n, inv);
    else
      for (size_t i = 0; i < n; i++) x[i] *= inv;
  }
}

}  // namespace

void softmax_inplace(float* x, size_t n) { softmax_ref(x, n); }

float sampler_next_f32(uint64_t* state) { return next_f32(state); }

uint32_t sample_logits(const float* logits, size_t n, const rlh_sampling_params& p, const uint32_t* recent,
                       size_t n_recent, uint64_t* state) {
  if (n == 0) return 0;
  if (p.temperature <= 0.0f && p.repetition_penalty == 1.0f) return first_max(logits, n);
  thread_local std::vector<float> probs;  // reused from call to call
  probs.assign(logits, logits + n);
  // repetition penalty over the distinct tokens of the last repeat_last_n
  // (all when 0), each at most once (sampler.rs:82-102)
  if (p.repetition_penalty != 1.0f) {
    const size_t start = p.repeat_last_n == 0 || n_recent <= p.repeat_last_n ? 0 : n_recent - p.repeat_last_n;
    std::vector<uint32_t> seen;
    seen.reserve(n_recent - start);
    for (size_t k = start; k < n_recent; k++) {
      const uint32_t t = recent[k];
      if (t >= n || std::find(seen.begin(), seen.end(), t) != seen.end()) continue;
      seen.push_back(t);
      if (probs[t] > 0.0f)
        probs[t] /= p.repetition_penalty;
      else
        probs[t] *= p.repetition_penalty;
    }
  }
  if (p.temperature <= 0.0f) return first_max(probs.data(), n);
  const float inv_t = 1.0f / p.temperature;  // sampler.rs:115-118
  if (have_avx2_fma())
    scale_avx2(probs.data(), n, inv_t);
  else
    for (float& v : probs) v *= inv_t;
  softmax_ref(probs.data(), n);
  // top-k (sampler.rs:122-132), as a bounded selection: descending
  // probability, equal probabilities by token id
  const size_t k = (p.top_k == 0 || p.top_k > n) ? n : p.top_k;
  auto before = [&](uint32_t a, uint32_t b) { return probs[a] > probs[b] || (probs[a] == probs[b] && a < b); };
  thread_local std::vector<uint32_t> idx;
  if (k < n) {
    // one pass keeping the k best in order; a later index never precedes an
    // equal probability already kept, so the list equals a sort's first k
    // (values below the last kept one are skipped eight at a time)
    idx.assign(1, 0u);
    const bool vec = have_avx2_fma();
    for (size_t i = 1; i < n; i++) {
      if (idx.size() == k) {
        if (vec) {
          i = next_candidate_avx2(probs.data(), i, n, probs[idx.back()]);
          if (i >= n) break;
        }
        if (!before((uint32_t)i, idx.back())) continue;
      }
      auto at = std::upper_bound(idx.begin(), idx.end(), (uint32_t)i, before);
      if (idx.size() == k) idx.pop_back();
      idx.insert(at, (uint32_t)i);
    }
  } else {
    idx.resize(n);
    for (size_t i = 0; i < n; i++) idx[i] = (uint32_t)i;
    std::sort(idx.begin(), idx.end(), before);
  }
  // top-p on the sorted list (sampler.rs:135-146)
  size_t cutoff = idx.size();
  if (p.top_p > 0.0f && p.top_p < 1.0f) {
    float cum = 0.0f;
    for (size_t pos = 0; pos < idx.size(); pos++) {
      cum += probs[idx[pos]];
      if (cum >= p.top_p) {
        cutoff = pos + 1;
        break;
      }
    }
  }
  idx.resize(cutoff);
  // draw (sampler.rs:148-162)
  float sum = 0.0f;
  for (uint32_t i : idx) sum += probs[i];
  if (sum <= 0.0f) return idx[0];
  float r = next_f32(state) * sum;
  for (uint32_t i : idx) {
    r -= probs[i];
    if (r <= 0.0f) return i;
  }
  return idx.back();
}

}  // namespace rlh

extern "C" {

uint64_t rlh_sampler_init(uint64_t seed) { return seed | 1; }  // Sampler::new (sampler.rs:33-37)

int rlh_softmax(float* x, uint64_t n) {
  if (n && !x) return rlh::set_error(RLH_EINVAL, "null argument");
  rlh::softmax_inplace(x, (size_t)n);
  return RLH_OK;
}

int rlh_sample(const float* logits, uint64_t n, const rlh_sampling_params* p, const uint32_t* recent,
               uint64_t n_recent, uint64_t* rng_state, uint32_t* token) {
  if (!p || !rng_state || !token || (n && !logits) || (n_recent && !recent)) return rlh::set_error(RLH_EINVAL,
                                                                                                  "null argument");
  *token = rlh::sample_logits(logits, (size_t)n, *p, recent, (size_t)n_recent, rng_state);
  return RLH_OK;
}

}  // extern "C"
