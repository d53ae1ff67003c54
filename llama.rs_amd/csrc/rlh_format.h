// rlh_format.h — device layout of the weight matrices (shared host/device).
//
// The bytes are the ggml block bytes of the reference (src/quant.rs:10-106);
// only their placement in HBM differs. Quantized matrices (Q4_K, Q6_K, Q8_0,
// Q4_0, Q5_K, Q4_1, Q5_0, Q5_1) are cut into items, one per 256 values of a
// row:
//   Q4_K  item = the 144-byte super-block as is;
//   Q5_K  item = the 176-byte super-block as is (d, dmin, scales[12], qh[32], qs[128]);
//   Q6_K  item = the 210-byte super-block as is (ql[128], qh[64], scales[16], d);
//   Q8_0  item = 8 consecutive blocks: their 8 x 32 quants, then their 8 f16 d;
//   Q4_0  item = 8 consecutive blocks: their 8 x 16 quant bytes, then 8 f16 d;
//   Q4_1  item = 8 blocks: 8 x 16 quant bytes, then 8 (f16 d, f16 m) pairs (160 B);
//   Q5_0  item = 8 blocks: 8 x 16 quant bytes, 8 u32 qh, 8 f16 d (176 B);
//   Q5_1  item = 8 blocks: 8 x 16 quant bytes, 8 u32 qh, 8 (d, m) pairs (192 B).
// Items are grouped in tiles of TR rows x TJ items (TR * TJ = 64); lane
// l = (j % TJ) * TR + (r % TR) of a wave owns item (r, j). Inside a tile the
// k-th 16-byte chunk of lane l's item sits at k * 1024 + l * 16, so one
// 16-byte load per lane reads 1 KB of contiguous memory (fully coalesced)
// while every lane still receives a whole item; the last ib % 16 bytes of
// an item (Q6_K's f16 d) follow at CH * 1024 + l * (ib % 16). Tiles are
// stored row-tile major. TJ is the largest of 4, 2, 1 dividing the items per
// row, so no column padding is needed; rows are padded with zero items to a
// multiple of TR.
//   F32/F16/BF16 (norm vectors, optional f32 weights): rows as is.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/rlh.h"

namespace rlh {

struct DevMat {
  uint32_t ty;
  uint32_t rows;
  uint32_t cols;
  uint32_t row_bytes;  // ggml bytes per row (rlh_row_bytes)
  const uint8_t* a;    // tiles (quantized types) or rows (float types)
  uint32_t tr, tj;     // tile shape: rows x items
  uint32_t ntj;        // tiles per row-tile (items per row / tj)
  uint32_t ib;         // item bytes
};

__host__ __device__ inline bool is_tiled(uint32_t ty) {
  return ty == RLH_TYPE_Q4_K || ty == RLH_TYPE_Q6_K || ty == RLH_TYPE_Q8_0 || ty == RLH_TYPE_Q4_0 ||
         ty == RLH_TYPE_Q5_K || ty == RLH_TYPE_Q4_1 || ty == RLH_TYPE_Q5_0 || ty == RLH_TYPE_Q5_1;
}
__host__ __device__ inline uint32_t item_bytes(uint32_t ty) {
  switch (ty) {
    case RLH_TYPE_Q6_K: return 210u;
    case RLH_TYPE_Q8_0: return 272u;
    case RLH_TYPE_Q5_K: return 176u;
    case RLH_TYPE_Q4_1: return 160u;
    case RLH_TYPE_Q5_0: return 176u;
    case RLH_TYPE_Q5_1: return 192u;
    default: return 144u;  // Q4_K, Q4_0
  }
}
// Items per row must be a multiple of the tile width.
__host__ __device__ inline uint32_t tile_width(uint32_t items_per_row) {
  return items_per_row % 4 == 0 ? 4u : (items_per_row % 2 == 0 ? 2u : 1u);
}
// Byte offset of byte o of item (row, j) from the matrix base.
__host__ __device__ inline size_t item_offset(const DevMat& w, uint32_t row, uint32_t j, uint32_t o) {
  const uint32_t rt = row / w.tr, jt = j / w.tj, l = (j % w.tj) * w.tr + row % w.tr;
  const size_t base = ((size_t)rt * w.ntj + jt) * 64 * w.ib;
  const uint32_t ch = w.ib / 16;
  if (o < ch * 16) return base + (size_t)(o / 16) * 1024 + l * 16 + o % 16;
  return base + (size_t)ch * 1024 + l * (w.ib - ch * 16) + (o - ch * 16);
}

// Q8 activation rows in device memory (Q8Row, simd.rs:88-101), token-major:
// qs[n][cols], d[n][cols/32], s[n][cols/32], s16[n][cols/16].
struct Q8Mut {
  int8_t* qs;
  float* d;
  int32_t* s;
  int32_t* s16;
};

}  // namespace rlh
