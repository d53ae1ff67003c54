// gemm.h — batched prefill products Y = X W^T on int8 MFMA (ops.rs:150-313,
// integer semantics of RUST_LLAMA_BATCH_INT=1).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "matvec.h"
#include "rlh_format.h"

namespace rlh {

struct GemmArgs {
  DevMat w;        // rows x cols, tiled layout (rlh_format.h)
  Q8Ptr x;         // n Q8 activation rows: qs[n][cols], d/s[n][cols/32], s16[n][cols/16]
  uint32_t n;      // tokens
  float* y;        // y[t * rows + r] = total (nullable)
  float* resid;    // resid[t * rows + r] += total (nullable)
  uint32_t n_tt;   // token tiles (ceil(n / 64))
  uint32_t n_rt;   // row tiles of both segments
  // an optional second segment of the same type and columns (the q and k
  // products of a layer in one launch): row tiles from n_rt1 on belong to
  // w2 and write y2 (no residual)
  DevMat w2;
  float* y2;
  uint32_t n_rt1;  // row tiles of w (n_rt when there is no second segment)
};

bool gemm_supported(uint32_t ty);
// Y[n][rows] (token-major) for the n activation rows; cols % 256 == 0.
void launch_gemm(hipStream_t st, const DevMat& w, const Q8Mut& x, uint32_t n, float* y, float* resid);
// Two products of one activation in one launch: Y[n][w.rows] and
// Y2[n][w2.rows], w and w2 of the same supported type and columns.
bool gemm_pair_supported(const DevMat& w, const DevMat& w2);
void launch_gemm_pair(hipStream_t st, const DevMat& w, const DevMat& w2, const Q8Mut& x, uint32_t n, float* y,
                      float* y2);
// Weight types without an integer batch path (Q5_K): matmul_batch's f32
// route on the f32 activations x[n][cols]; the tokens from n4 on (the last
// n % 4 of the whole batch) take the single-token dot order.
bool gemm_f32_supported(uint32_t ty);
void launch_gemm_f32(hipStream_t st, const DevMat& w, const float* x, uint32_t n, uint32_t n4, float* y,
                     float* resid);

}  // namespace rlh
