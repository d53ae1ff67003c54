// kernels.h — host-side launch wrappers of the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlh_format.h"

namespace rlh {

using Q8Buf = Q8Mut;

// Largest hidden size the single-block row kernels (rmsnorm) stage in LDS.
constexpr int kMaxEmbd = 7168;

bool matvec_supported(uint32_t ty);

void launch_embed(hipStream_t st, const DevMat& w, const uint32_t* tok, uint32_t n_tok, float* x);
void launch_rmsnorm_q8(hipStream_t st, const float* x, const float* w, uint32_t n, uint32_t n_tok, float eps,
                       const Q8Buf& out, float* xb);
void launch_quantize_q8(hipStream_t st, const float* x, uint32_t n, const Q8Buf& out);
void launch_block_dots(hipStream_t st, const DevMat& w, const int8_t* a, int32_t* out, uint32_t per_row);
void launch_dequant(hipStream_t st, const DevMat& w, float* out);
void launch_qk_norm_rope_kv(hipStream_t st, float* q, float* k, const float* v, const float* bq, const float* bk,
                            const float* bv, const float* qn, const float* kn, const float* rope_cs,
                            const uint32_t* pos0, float* kcache, float* vcache, int H, int KVH, uint32_t n_tok,
                            float eps);
void launch_swiglu_q8(hipStream_t st, const float* g, const float* u, uint32_t n_total, const Q8Buf& out,
                      float* h_out);
// Final reduction of per-block (max, lowest index) candidates; with `step`
// set it also advances the greedy loop state (pos += 1, hist[++step] = tok).
void launch_argmax_final(hipStream_t st, const float* pv, const uint32_t* pi, uint32_t nparts, uint32_t* tok_out,
                         uint32_t* pos, uint32_t* step, uint32_t* hist);
void launch_argmax(hipStream_t st, const float* x, uint32_t n, float* pv, uint32_t* pi, uint32_t nparts,
                   uint32_t* tok_out, uint32_t* pos, uint32_t* step, uint32_t* hist);

}  // namespace rlh
