// attention.h — launch arguments of the exact GQA attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlh_format.h"

namespace rlh {

struct AttnArgs {
  const float* q;  // [n_tok][H*128]  raw projections (decode) or normed+roped (prefill)
  const float* k;  // [n_tok][KVH*128] raw (decode only)
  const float* v;  // [n_tok][KVH*128] raw (decode only)
  const float* bq;
  const float* bk;
  const float* bv;
  const float* qn;       // attn_q_norm (nullable)
  const float* kn;       // attn_k_norm (nullable)
  const float* rope_cs;  // [n_ctx][128] (cos, sin) pairs
  const uint32_t* pos0;  // device: position of token 0
  float* kcache;         // layer base [max_ctx][KVH*128]
  float* vcache;
  float* scores;         // [n_tok][H][t_stride]
  uint32_t t_stride;
  uint32_t t_max;  // bound on positions attended in this launch (grid / LDS sizing)
  uint32_t vtile;  // V positions per LDS tile (attn_vtile)
  int H, KVH;
  float eps, scale;
  float* out;    // [n_tok][H*128]
  Q8Mut out_q8;  // Q8 blocks of out
};

uint32_t attn_vtile(uint32_t t_max);
size_t attn_out_lds(uint32_t t_max, uint32_t vtile);
// fused = decode: QK-norm + RoPE + K/V write inside the scores kernel.
void launch_attn_scores(hipStream_t st, const AttnArgs& a, uint32_t n_tok, bool fused);
void launch_attn_out(hipStream_t st, const AttnArgs& a, uint32_t n_tok);
bool attn_set_max_lds(size_t bytes);

}  // namespace rlh
