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
  float* scores;         // [n_tok][H][t_stride]: scores, then softmax probabilities in place
  uint32_t t_stride;
  uint32_t t_max;        // bound on positions attended in this launch (grid / LDS sizing)
  uint32_t max_ctx;      // rows of the cache (K/V tiles never read past it)
  uint32_t n_tok;
  int H, KVH;
  float eps, scale;
  float* out;    // [n_tok][H*128]
  Q8Mut out_q8;  // Q8 blocks of out
  uint32_t* err; // device error word (nullable): an expired bounded wait sets kErrAttnExp
  // test knob of the decode softmax's exact parallel sum (0 in use): shifts
  // the walk's predicted binades so that runs replay (block_softmax_sum)
  int walk_shift;
};

// Query heads per KV head the kernels accept (1..8).
constexpr int kAttnMaxGroup = 8;
// Positions a softmax row may hold (dynamic LDS of one row).
constexpr uint32_t kAttnMaxCtx = 32768;

// Scores s_j = dot(q_h, K_j) * scale for every token and head. fused =
// decode (one token): QK-norm + RoPE of q and k and the K/V write at pos are
// done here as well.
void launch_attn_scores(hipStream_t st, const AttnArgs& a, bool fused);
// softmax_inplace of every score row (probabilities overwrite the scores).
void launch_attn_softmax(hipStream_t st, const AttnArgs& a);
// Decode (one token) after the scores: softmax and the ordered V
// accumulation. f32_out: out in f32 only (the caller quantizes it) by the
// kernel that keeps its V slices in LDS when attn_dec_v_lds is nonzero,
// else by launch_attn_softmax + a PV kernel streaming V and p through LDS
// rings (any context). Otherwise the kernels that also write the Q8 blocks
// out_q8.
void launch_attn_decode(hipStream_t st, const AttnArgs& a, bool f32_out);
// LDS of the resident-V decode kernel (0 when it does not apply: more than 4
// query heads per KV head or too many positions).
size_t attn_dec_v_lds(uint32_t t_max, uint32_t group);
// LDS of the fused decode kernel for t_max positions and `group` query heads
// per KV head (0 when the rows do not fit).
size_t attn_dec_fused_lds(uint32_t t_max, uint32_t group);
// Ordered V accumulation of the probabilities; writes out and its Q8 blocks.
// decode = one token (d-sliced blocks), else token tiles sharing V chunks.
void launch_attn_pv(hipStream_t st, const AttnArgs& a, bool decode);
// Raises the softmax kernel's dynamic LDS limit to cover max_ctx positions.
bool attn_init(uint32_t max_ctx);

}  // namespace rlh
