// sampler.h — host sampler (sampler.rs:56-163) shared by the C entries.
#pragma once
#include <cstddef>
#include <cstdint>

#include "../../include/rlh.h"

namespace rlh {

// ops::softmax_inplace (ops.rs:398-419) as the sampler runs it.
void softmax_inplace(float* x, size_t n);
// Sampler::sample on host logits; advances the xorshift64* state.
uint32_t sample_logits(const float* logits, size_t n, const rlh_sampling_params& p, const uint32_t* recent,
                       size_t n_recent, uint64_t* state);
// Sampler::next_f32 (sampler.rs:51-54): advances the xorshift64* state and
// returns the uniform draw in [0, 1).
float sampler_next_f32(uint64_t* state);
// Records the thread's last error message (rlh_last_error) and returns code.
int set_error(int code, const char* msg);

}  // namespace rlh
