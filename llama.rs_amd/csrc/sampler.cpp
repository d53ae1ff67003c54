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
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../../include/rlh.h"
#include "sampler.h"

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

// ops::softmax_inplace (ops.rs:398-419).
void softmax_ref(float* x, size_t n) {
  if (n == 0) return;
  float mx = x[0];
  for (size_t i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  if (sum > 0.0f) {
    const float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
  }
}

}  // namespace

uint32_t sample_logits(const float* logits, size_t n, const rlh_sampling_params& p, const uint32_t* recent,
                       size_t n_recent, uint64_t* state) {
  if (n == 0) return 0;
  if (p.temperature <= 0.0f && p.repetition_penalty == 1.0f) return first_max(logits, n);
  std::vector<float> probs(logits, logits + n);
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
  for (float& v : probs) v *= inv_t;
  softmax_ref(probs.data(), n);
  // top-k (sampler.rs:122-132), as a bounded selection: descending
  // probability, equal probabilities by token id
  const size_t k = (p.top_k == 0 || p.top_k > n) ? n : p.top_k;
  auto before = [&](uint32_t a, uint32_t b) { return probs[a] > probs[b] || (probs[a] == probs[b] && a < b); };
  std::vector<uint32_t> idx(n);
  for (size_t i = 0; i < n; i++) idx[i] = (uint32_t)i;
  if (k < n) {
    std::partial_sort(idx.begin(), idx.begin() + k, idx.end(), before);
    idx.resize(k);
  } else {
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

int rlh_sample(const float* logits, uint64_t n, const rlh_sampling_params* p, const uint32_t* recent,
               uint64_t n_recent, uint64_t* rng_state, uint32_t* token) {
  if (!p || !rng_state || !token || (n && !logits) || (n_recent && !recent)) return rlh::set_error(RLH_EINVAL,
                                                                                                  "null argument");
  *token = rlh::sample_logits(logits, (size_t)n, *p, recent, (size_t)n_recent, rng_state);
  return RLH_OK;
}

}  // extern "C"
