// matvec.h — launch descriptors of the decode matvec (ops.rs:67-141).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlh_format.h"

namespace rlh {

struct Q8Ptr {
  const int8_t* qs;
  const float* d;
  const int32_t* s;
  const int32_t* s16;
};

// One matrix (or a gate/up pair) of a launch. Every segment of a launch
// multiplies the same Q8 activation row (cols wide).
struct MvSeg {
  DevMat w;            // rows summed into y / resid (gate in PAIR mode)
  DevMat w2;           // PAIR mode: up
  float* y;            // single: y[r] = total (nullable); PAIR: h[r] = silu(g)*u (nullable)
  float* resid;        // single: resid[r] = resid[r] + total (nullable)
  Q8Mut hq;            // PAIR: Q8 blocks of h (the next matvec's activation)
  uint32_t blk_begin;  // first block of this segment
  uint32_t pair;
};

// Greedy argmax candidates of the logits launch: every block leaves its
// (max, lowest index) in pv/pi[block]; launch_argmax_final reduces them
// (main.rs:453-463 semantics).
struct MvArgmax {
  float* pv;
  uint32_t* pi;
};

struct MvLaunch {
  MvSeg seg[3];
  uint32_t nseg;
  uint32_t cols;
  uint32_t rows_per_blk;  // R: rows of one block (all segments)
  Q8Ptr act;              // Q8 activation row in HBM, staged into LDS by each block
  // norm input (nx set): the activation is quantize_q8(rmsnorm(nx, nw)) of
  // the f32 row nx (simd.rs:282-326, 116-203), computed by every block in
  // its prologue while its first weights are in flight; act is unused
  const float* nx;
  const float* nw;
  float eps;
  // f32 activation row, needed by Q5_K segments (the reference multiplies
  // Q5_K weights with the unquantized activation, quant.rs:528-539): staged
  // from xf in Q8 launches, written by the norm prologue otherwise
  const float* xf;
  uint32_t need_xf;
  uint32_t need_q8;  // 0: every segment multiplies the f32 row (Q5_K, Q4_1, Q5_0, Q5_1), no Q8 staging
  uint32_t xf_off;  // byte offset of the f32 row in LDS
  uint32_t region_off;    // byte offset of the term tiles in LDS
  uint32_t tile_stride;   // floats per term-tile row
  // ring plans (long rows, one row tile per block): the term region holds
  // `ring` rounds of the producer waves' tiles, which wave 0 chains as they
  // complete; 0 = every row's terms stay in LDS until the end
  uint32_t ring;
  uint32_t has_argmax;
  MvArgmax am;
  // device error word (nullable): a bounded intra-block wait that expires
  // sets its bit (kErrMvRing / kErrMvSplit) here
  uint32_t* err;
};

// Host-side plan: segments are appended, then launched once.
struct MvPlan {
  MvLaunch L{};
  uint32_t blocks = 0;
  uint32_t lds = 0;
  uint32_t waves = 0;  // waves per block
  uint32_t max_terms = 0;
  uint32_t slot_stride = 0;  // float plans: floats per row of chain results
  uint32_t float_stage = 0;  // float plans: LDS bytes of the row stage buffers
  uint32_t rows = 0;   // rows over all segments
  bool norm = false;   // activation from the norm prologue
  bool quant = false;  // ... without the norm (quantize_q8 of the f32 row only)
};

// Terms (float summands of the reference's per-row chain) per 256-value
// super-block: one per 64 values for Q4_K, per 16 for Q6_K, per 32 for
// Q8_0/Q4_0/Q4_1/Q5_0/Q5_1, one per super-block for Q5_K (its f32 block
// dot); none for float weights, whose rows are whole chains.
__host__ __device__ inline uint32_t mv_terms_per_sb(uint32_t ty) {
  if (ty == RLH_TYPE_F16 || ty == RLH_TYPE_F32 || ty == RLH_TYPE_BF16) return 0u;  // whole-row chains
  return ty == RLH_TYPE_Q6_K ? 16u : (ty == RLH_TYPE_Q4_K ? 4u : (ty == RLH_TYPE_Q5_K ? 1u : 8u));
}

// Plan construction: act is the Q8 activation row (cols values, cols a
// multiple of 256). Every segment must have `cols` columns; PAIR plans hold
// exactly one segment. mv_plan_finish fixes the block shape (returns false
// when no shape fits the LDS).
void mv_plan_init(MvPlan& p, uint32_t cols, const Q8Mut& act);
// Same, with the activation computed in the kernel from the f32 row x and
// the rmsnorm weight w (cols <= kMvMaxNormCols).
void mv_plan_init_norm(MvPlan& p, uint32_t cols, const float* x, const float* w, float eps);
constexpr uint32_t kMvMaxNormCols = 7168;
// Same, with the activation quantize_q8(x) of the f32 row x computed in the
// kernel (no norm; cols <= kMvMaxQuantCols).
void mv_plan_init_quant(MvPlan& p, uint32_t cols, const float* x);
constexpr uint32_t kMvMaxQuantCols = 12288;
// The f32 form of a Q8 launch's activation (used when a segment is Q5_K).
void mv_plan_set_f32(MvPlan& p, const float* xf);
void mv_plan_add(MvPlan& p, const DevMat& w, float* y, float* resid);
void mv_plan_add_pair(MvPlan& p, const DevMat& gate, const DevMat& up, const Q8Mut& hq, float* h);
void mv_plan_argmax(MvPlan& p, const MvArgmax& am);
bool mv_plan_finish(MvPlan& p);
// err: the device error word the launch's bounded waits report to
// (nullable). ev_start / ev_stop (optional, not under graph capture): events
// that take the kernel's own start and end times (hipExtLaunchKernel), for
// probes.
void mv_launch(hipStream_t st, const MvPlan& p, uint32_t* err, hipEvent_t ev_start = nullptr,
               hipEvent_t ev_stop = nullptr);
// Blocks of a single-matrix plan over `rows` rows of `cols` columns (the
// argmax partial buffers of the logits launch hold one entry per block).
uint32_t mv_blocks_for(uint32_t ty, uint32_t rows, uint32_t cols);
bool mv_set_max_lds(size_t bytes);

}  // namespace rlh
