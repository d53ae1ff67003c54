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
  uint32_t n_rt;   // row tiles (ceil(rows / 64))
};

bool gemm_supported(uint32_t ty);
// Y[n][rows] (token-major) for the n activation rows; cols % 256 == 0.
void launch_gemm(hipStream_t st, const DevMat& w, const Q8Mut& x, uint32_t n, float* y, float* resid);

}  // namespace rlh
