// rlh_format.h — device layouts of the weight matrices (shared host/device).
//
// The bytes are the ggml block bytes of the reference (src/quant.rs:10-106);
// only their placement in HBM differs where a block is not 16-byte aligned:
//   Q4_K  144-byte super-blocks, kept as is (144 = 9*16, so every block and
//         its 128 quant bytes at offset 16 are 16-byte aligned).
//         a = blocks, row r at r*row_bytes.
//   Q6_K  210-byte super-blocks are only 2-byte aligned, so the four fields
//         are split into planes, each indexed by super-block s = r*nsb + bi:
//         a = ql[s][128], b = qh[s][64], c = scales[s][16], d = d[s] (f16).
//   Q8_0  34-byte blocks: a = qs[b][32], b = d[b] (f16), b = r*nb + block.
//   Q4_0  18-byte blocks: a = qs[b][16], b = d[b] (f16).
//   F32/F16/BF16: rows as is.
// Total bytes per matrix equal the ggml bytes (planes add no padding beyond
// 256-byte alignment of each plane start).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "../../include/rlh.h"

namespace rlh {

struct DevMat {
  uint32_t ty;
  uint32_t rows;
  uint32_t cols;
  uint32_t row_bytes;  // ggml bytes per row (rlh_row_bytes)
  const uint8_t* a;
  const uint8_t* b;
  const uint8_t* c;
  const uint8_t* d;
};

// Q8 activation rows in device memory (Q8Row, simd.rs:88-101), token-major:
// qs[n][cols], d[n][cols/32], s[n][cols/32], s16[n][cols/16].
struct Q8Mut {
  int8_t* qs;
  float* d;
  int32_t* s;
  int32_t* s16;
};

}  // namespace rlh
