// matvec.h — launch descriptors of the multi-segment decode matvec.
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

// One matrix (or a gate/up pair) of a launch.
struct MvSeg {
  DevMat w;          // rows summed into y / resid (gate in PAIR mode)
  DevMat w2;         // PAIR mode: up
  Q8Ptr act;         // Q8 activation row (cols of w)
  float* y;          // single: y[r] = total (nullable); PAIR: h[r] (nullable)
  float* resid;      // single: resid[r] = resid[r] + total (nullable)
  Q8Mut hq;          // PAIR: Q8 blocks of h = silu(gate) * up
  uint32_t wg_begin;     // first block index of this segment
  uint32_t rows_per_wg;  // R = 4 * NS * P (NS of the launch; 32 in PAIR mode)
  uint32_t pair;
};

struct MvLaunch {
  MvSeg seg[3];
  uint32_t nseg;
};

// Rows packed per wave instruction for a row of `units` units.
inline uint32_t mv_pack(uint32_t units) { return units <= 16 ? 4u : (units <= 32 ? 2u : 1u); }
inline uint32_t mv_units(uint32_t ty, uint32_t cols) {
  return (ty == RLH_TYPE_Q8_0 || ty == RLH_TYPE_Q4_0) ? cols / 32 : cols / 64;
}
inline uint32_t mv_terms_per_unit(uint32_t ty) { return ty == RLH_TYPE_Q6_K ? 4u : 1u; }

// ns: row slots per lane (1, 2, 4 or 8), shared by all segments of L.
void launch_mv(hipStream_t st, const MvLaunch& L, uint32_t total_wgs, uint32_t lds_bytes, uint32_t ns);
bool mv_set_max_lds(size_t bytes);

}  // namespace rlh
