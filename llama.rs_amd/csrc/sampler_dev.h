// sampler_dev.h — the device sampler (sampler_dev.hip) for the engine's
// sampled decode loop.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rlh.h"

namespace rlh {

// Sampler::sample (sampler.rs:56-163) on device logits[n]; the token and the
// xorshift64* state advance as the host restatement's.
int dsampler_sample(rlh_dsampler* ds, const float* logits, uint64_t n, const rlh_sampling_params& p,
                    const uint32_t* recent, uint64_t n_recent, uint64_t* rng_state, uint32_t* token, hipStream_t s);
// ops::softmax_inplace (ops.rs:398-419) on device x[n].
int dsampler_softmax(rlh_dsampler* ds, float* x, uint64_t n, hipStream_t s);

}  // namespace rlh
