// gemm.hip — batched prefill products on int8 MFMA (ops.rs:150-313 with
// RUST_LLAMA_BATCH_INT=1: quantize_q8 of every token, then dot_qk_q8_row per
// (row, token), simd.rs:898-910).
//
// Exactness: for every (token, row) the output is the reference's f32 chain
// `total += term` over the row's terms in index order; each term is formed
// with the reference's expression (simd.rs:581 Q4_K, 663 Q6_K, 863 Q4_0,
// 891 Q8_0). The integer block dots inside the terms come from
// v_mfma_i32_16x16x32_i8 and are exact:
//   Q4_K  unsigned nibbles (0..15) x Q8 bytes, one MFMA per 32-value block;
//   Q6_K  q = u - 32 as signed bytes, so the MFMA gives sum(q a) = ss - 32 sa
//         exactly, which is what (ss as f32 - 32.0 * sa as f32) evaluates to
//         (both are integers below 2^24); one MFMA per 16-value half, the
//         other half of the operand zeroed;
//   Q8_0  signed bytes; Q4_0 nibble - 8, i.e. i0 + i1 - 8 * sum exactly.
// The per-element float epilogue runs on the VALU and dominates the cost.
//
// Tiling: a block owns 64 tokens x 64 rows; 4 waves of 32 x 32, each 2 x 2
// MFMA tiles of 16 x 16. Per super-block (256 values) the block stages the
// 64 tokens' Q8 bytes and block scales into LDS (double buffered, copied
// through registers); every lane loads the weight bytes of its row straight
// from the tiled layout, one super-block ahead. Block b runs on XCD b % 8; the blocks
// of one XCD walk the token tiles of a row tile first, so each weight tile
// is fetched into that XCD's L2 once and reused by all token tiles.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm.h"
#include "rlh_device.h"

namespace rlh {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef RLH_LDS uint8_t lbyte;

constexpr uint32_t kTile = 64;                          // tokens and rows per block
constexpr uint32_t kXStride = 272;                      // LDS bytes per token per super-block (16-byte pad)
constexpr uint32_t kXBytes = kTile * kXStride;          // 17408
constexpr uint32_t kDBytes = kTile * 8 * 4;             // da of 8 blocks per token, block-major [8][64]
constexpr uint32_t kRBytes = kTile * 4 * 16;            // Q4_K row scales: [4 groups][64 rows] float4
constexpr uint32_t kStageBytes = kXBytes + 2 * kDBytes + kRBytes;  // + sums as f32 (Q4_K), + row scales

__device__ __forceinline__ uint64_t g8(const uint8_t* p) { return *(const RLH_GLOBAL uint64_t*)p; }
__device__ __forceinline__ u32x4_t g16(const uint8_t* p) { return *(const RLH_GLOBAL u32x4_t*)p; }
__device__ __forceinline__ long l8(const lbyte* p) { return *(const RLH_LDS long*)p; }

__device__ __forceinline__ v4i mfma(long a, uint64_t b) {
  const v4i z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, (long)b, z, 0, 0, 0);
}

// Bytes of item (row, j) in the tiled layout: byte o < 16 * (ib / 16) lies
// at base + (o / 16) * 1024 + o % 16; the ib % 16 tail bytes at `tail`.
struct ItemPtr {
  const uint8_t* base;
  const uint8_t* tail;
};
__device__ __forceinline__ ItemPtr item_ptr(const DevMat& w, uint32_t row, uint32_t j) {
  const uint32_t rt = row / w.tr, jt = j / w.tj, l = (j % w.tj) * w.tr + row % w.tr;
  const uint8_t* tb = w.a + ((size_t)rt * w.ntj + jt) * 64 * w.ib;
  const uint32_t ch = w.ib / 16;
  return ItemPtr{tb + l * 16, tb + ch * 1024 + l * (w.ib - ch * 16)};
}
__device__ __forceinline__ const uint8_t* at(const ItemPtr& p, uint32_t o) { return p.base + (o >> 4) * 1024 + (o & 15); }

// Lane coordinates inside the block: lane = 16 q + i16; wave = 2 rw + tw.
struct Lane {
  uint32_t q, i16, tw, rw;
};

// View of a staged super-block. The token scales and sums are block-major
// ([block][token], so the four tokens a lane owns are one 16-byte read) for
// Q4_K, Q8_0 and Q4_0, token-major ([token][block]) for Q6_K.
struct StageView {
  const lbyte* xs;            // [64][kXStride] Q8 bytes
  const RLH_LDS float* d;     // block scales
  const RLH_LDS float* s;     // Q4_K: block sums, as f32 (exact: |sum| <= 4064), block-major
  const RLH_LDS f32x4_t* rs;  // Q4_K, [4][64]: {d*sc, dmin*m} of sub-blocks 2g, 2g+1 of each row
};

__device__ __forceinline__ StageView view(const lbyte* buf) {
  return StageView{buf, (const RLH_LDS float*)(buf + kXBytes), (const RLH_LDS float*)(buf + kXBytes + kDBytes),
                   (const RLH_LDS f32x4_t*)(buf + kXBytes + 2 * kDBytes)};
}

// The lane's four tokens' values of block kb (scales or sums).
__device__ __forceinline__ f32x4_t tok4(const RLH_LDS float* t, const Lane& ln, uint32_t tr, uint32_t kb) {
  return *(const RLH_LDS f32x4_t*)(t + kb * kTile + 32 * ln.tw + 16 * tr + 4 * ln.q);
}

// A operands of block kb (0..7 inside the super-block) for token tile tr.
__device__ __forceinline__ long a_frag(const StageView& v, const Lane& ln, uint32_t tr, uint32_t kb) {
  const uint32_t tok = 32 * ln.tw + 16 * tr + ln.i16;
  return l8(v.xs + tok * kXStride + kb * 32 + 8 * ln.q);
}

// The per-type loops below are not unrolled (unrolling them makes the
// compiler keep every iteration's MFMA results and operands live at once);
// instead of indexing a register array with the loop counter (which would
// move the array to scratch memory), each iteration uses element 0 and the
// arrays are rotated by one at its end.
template <int N>
__device__ __forceinline__ void rotate(uint64_t (&a)[N]) {
#pragma unroll
  for (int i = 0; i + 1 < N; i++) a[i] = a[i + 1];
}

// ---- per-type weight fragments and term evaluation --------------------------
template <uint32_t TY>
struct GT;

// Q4_K: lane k-range 8q..8q+7 of block 2g is the low nibbles of item bytes
// 16 + 32g + 8q .. +8, of block 2g+1 their high nibbles. The row scales
// d*sc and dmin*m (get_scale_min_k4, quant.rs:176-185) are staged once per
// super-block for the block's 64 rows (stage_store), not decoded per lane.
template <>
struct GT<RLH_TYPE_Q4_K> {
  static constexpr bool kNeedS = true;  // block sums and row scales staged
  static constexpr bool kBlockMajor = true;
  struct W {
    uint64_t qs[4];
  };
  __device__ __forceinline__ static void load(W& r, const DevMat& w, uint32_t row, uint32_t j, uint32_t q) {
    const ItemPtr p = item_ptr(w, row, j);
#pragma unroll
    for (int g = 0; g < 4; g++) r.qs[g] = g8(at(p, 16 + 32 * g + 8 * q));
  }
  __device__ __forceinline__ static void compute(const W (&w)[2], const StageView& v, const Lane& ln,
                                                 float (&acc)[2][2][4]) {
    const uint64_t m4 = 0x0F0F0F0F0F0F0F0Full;
#pragma unroll 2
    for (int g = 0; g < 4; g++) {
      long alo[2], ahi[2];
#pragma unroll
      for (int tr = 0; tr < 2; tr++) {
        alo[tr] = a_frag(v, ln, tr, 2 * g);
        ahi[tr] = a_frag(v, ln, tr, 2 * g + 1);
      }
      f32x4_t rsc[2];  // {d1, mm1, d2, mm2} of the lane's rows
      uint64_t blo[2], bhi[2];
#pragma unroll
      for (int tc = 0; tc < 2; tc++) {
        const uint64_t qg = g == 0 ? w[tc].qs[0] : (g == 1 ? w[tc].qs[1] : (g == 2 ? w[tc].qs[2] : w[tc].qs[3]));
        blo[tc] = qg & m4;
        bhi[tc] = (qg >> 4) & m4;
        rsc[tc] = v.rs[g * kTile + 32 * ln.rw + 16 * tc + ln.i16];
      }
#pragma unroll
      for (int tr = 0; tr < 2; tr++) {
        const f32x4_t da = tok4(v.d, ln, tr, 2 * g), db = tok4(v.d, ln, tr, 2 * g + 1);
        const f32x4_t sa = tok4(v.s, ln, tr, 2 * g), sb = tok4(v.s, ln, tr, 2 * g + 1);
#pragma unroll
        for (int tc = 0; tc < 2; tc++) {
          const v4i c1 = mfma(alo[tr], blo[tc]);
          const v4i c2 = mfma(ahi[tr], bhi[tc]);
          const float d1 = rsc[tc].x, mm1 = rsc[tc].y, d2 = rsc[tc].z, mm2 = rsc[tc].w;
#pragma unroll
          for (int e = 0; e < 4; e++)  // simd.rs:581
            acc[tr][tc][e] = acc[tr][tc][e] + (da[e] * (d1 * (float)c1[e] - mm1 * sa[e]) +
                                               db[e] * (d2 * (float)c2[e] - mm2 * sb[e]));
        }
      }
    }
  }
};

// Q6_K: block c of half h covers item bytes ql[64h + 32(c&1) + p] (nibble
// c >> 1) and qh[128 + 32h + p] (bits 2c, 2c+1), p = position 0..31; the
// lane's positions 8q..8q+7 all belong to sub-half s = q >> 1.
template <>
struct GT<RLH_TYPE_Q6_K> {
  static constexpr bool kNeedS = false;
  static constexpr bool kBlockMajor = false;  // four blocks of one token per read
  struct W {
    uint64_t ql[2][2], qh[2];
    u32x4_t sc;
    uint32_t d;
  };
  __device__ __forceinline__ static void load(W& r, const DevMat& w, uint32_t row, uint32_t j, uint32_t q) {
    const ItemPtr p = item_ptr(w, row, j);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      r.ql[h][0] = g8(at(p, 64 * h + 8 * q));
      r.ql[h][1] = g8(at(p, 64 * h + 32 + 8 * q));
      r.qh[h] = g8(at(p, 128 + 32 * h + 8 * q));
    }
    r.sc = g16(at(p, 192));
    r.d = ld_g2(p.tail);
  }
  __device__ __forceinline__ static void compute(const W (&w)[2], const StageView& v, const Lane& ln,
                                                 float (&acc)[2][2][4]) {
    const uint64_t m4 = 0x0F0F0F0F0F0F0F0Full, m2 = 0x0303030303030303ull;
    const uint64_t hi = 0x8080808080808080ull, k32 = 0x2020202020202020ull;
    const bool sub1 = ln.q >= 2;
    uint64_t hq[2][4], hh[2][2];  // per row tile: ql pieces of half 0 then 1, qh of half 0 then 1
    uint32_t hs[2][4];            // scale words of half 0 then 1
#pragma unroll
    for (int tc = 0; tc < 2; tc++) {
      hq[tc][0] = w[tc].ql[0][0];
      hq[tc][1] = w[tc].ql[0][1];
      hq[tc][2] = w[tc].ql[1][0];
      hq[tc][3] = w[tc].ql[1][1];
      hh[tc][0] = w[tc].qh[0];
      hh[tc][1] = w[tc].qh[1];
      hs[tc][0] = w[tc].sc.x;
      hs[tc][1] = w[tc].sc.y;
      hs[tc][2] = w[tc].sc.z;
      hs[tc][3] = w[tc].sc.w;
    }
#pragma unroll 1
    for (int h = 0; h < 2; h++) {
      // signed weights q = u - 32 of the half's 4 blocks, per row tile
      uint64_t bq[2][4];
      float dsc[2][2][4];
#pragma unroll
      for (int tc = 0; tc < 2; tc++) {
        const float d = f16_to_f32(w[tc].d);
        const uint32_t swlo = hs[tc][0], swhi = hs[tc][1];  // the half's 8 scales
        const uint64_t ql0 = hq[tc][0], ql1 = hq[tc][1], qh = hh[tc][0];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const uint64_t nib = (((c & 1) ? ql1 : ql0) >> (4 * (c >> 1))) & m4;
          const uint64_t u = nib | (((qh >> (2 * c)) & m2) << 4);
          bq[tc][c] = ((u | hi) - k32) ^ hi;
#pragma unroll
          for (int s = 0; s < 2; s++) {
            const uint32_t bi = s + 2 * c;  // scales[sub + 2c] of the half (simd.rs:626-629)
            dsc[tc][s][c] = d * (float)(int8_t)(((bi < 4 ? swlo : swhi) >> (8 * (bi & 3))) & 0xff);
          }
        }
      }
      long a[2][4];
      f32x4_t da[2][4];  // [tr][e] -> da of blocks 4h..4h+3 (token-major staging)
#pragma unroll
      for (int tr = 0; tr < 2; tr++) {
#pragma unroll
        for (int c = 0; c < 4; c++) a[tr][c] = a_frag(v, ln, tr, 4 * h + c);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t tok = 32 * ln.tw + 16 * tr + 4 * ln.q + e;
          da[tr][e] = *(const RLH_LDS f32x4_t*)(v.d + tok * 8 + 4 * h);
        }
      }
      // terms in the order s = 0 (c = 0..3), then s = 1 (simd.rs:630-665);
      // the four products of a (s, c) step are issued before their
      // combines, so no combine waits on the product just issued
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const bool keep = (s == 1) == sub1;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          v4i ci[2][2];
#pragma unroll
          for (int tr = 0; tr < 2; tr++)
#pragma unroll
            for (int tc = 0; tc < 2; tc++) ci[tr][tc] = mfma(a[tr][c], keep ? bq[tc][c] : 0ull);
#pragma unroll
          for (int tr = 0; tr < 2; tr++) {
#pragma unroll
            for (int tc = 0; tc < 2; tc++) {
#pragma unroll
              for (int e = 0; e < 4; e++)  // simd.rs:663
                acc[tr][tc][e] = acc[tr][tc][e] + dsc[tc][s][c] * (float)ci[tr][tc][e] * da[tr][e][c];
            }
          }
        }
      }
#pragma unroll
      for (int tc = 0; tc < 2; tc++) {  // half 1 moves into place
        hq[tc][0] = hq[tc][2];
        hq[tc][1] = hq[tc][3];
        hh[tc][0] = hh[tc][1];
        hs[tc][0] = hs[tc][2];
        hs[tc][1] = hs[tc][3];
      }
    }
  }
};

// Q8_0: item = 8 blocks; lane bytes 32k + 8q .. +8 of block k, then the 8
// f16 scales at item bytes 256..271.
template <>
struct GT<RLH_TYPE_Q8_0> {
  static constexpr bool kNeedS = false;
  static constexpr bool kBlockMajor = true;
  struct W {
    uint64_t qs[8];
    u32x4_t dv;
  };
  __device__ __forceinline__ static void load(W& r, const DevMat& w, uint32_t row, uint32_t j, uint32_t q) {
    const ItemPtr p = item_ptr(w, row, j);
#pragma unroll
    for (int k = 0; k < 8; k++) r.qs[k] = g8(at(p, 32 * k + 8 * q));
    r.dv = g16(at(p, 256));
  }
  __device__ __forceinline__ static void compute(const W (&wr)[2], const StageView& v, const Lane& ln,
                                                 float (&acc)[2][2][4]) {
    uint64_t qs[2][8];
    uint32_t dw[2][4];
#pragma unroll
    for (int tc = 0; tc < 2; tc++) {
#pragma unroll
      for (int k = 0; k < 8; k++) qs[tc][k] = wr[tc].qs[k];
      dw[tc][0] = wr[tc].dv.x;
      dw[tc][1] = wr[tc].dv.y;
      dw[tc][2] = wr[tc].dv.z;
      dw[tc][3] = wr[tc].dv.w;
    }
#pragma unroll 2
    for (int k = 0; k < 8; k++) {
      float dk[2];
#pragma unroll
      for (int tc = 0; tc < 2; tc++) dk[tc] = f16_to_f32((dw[tc][0] >> (16 * (k & 1))) & 0xffff);
#pragma unroll
      for (int tr = 0; tr < 2; tr++) {
        const long a = a_frag(v, ln, tr, k);
        const f32x4_t da = tok4(v.d, ln, tr, k);
#pragma unroll
        for (int tc = 0; tc < 2; tc++) {
          const v4i ci = mfma(a, qs[tc][0]);
#pragma unroll
          for (int e = 0; e < 4; e++)  // simd.rs:891
            acc[tr][tc][e] = acc[tr][tc][e] + dk[tc] * (float)ci[e] * da[e];
        }
      }
#pragma unroll
      for (int tc = 0; tc < 2; tc++) {
        rotate(qs[tc]);
        if (k & 1) {  // next pair of f16 scales
          dw[tc][0] = dw[tc][1];
          dw[tc][1] = dw[tc][2];
          dw[tc][2] = dw[tc][3];
        }
      }
    }
  }
};

// Q4_0: item = 8 blocks of 16 bytes; positions 0..15 are the low nibbles,
// 16..31 the high nibbles, so lane q reads bytes 16k + 8(q & 1) .. +8 and
// takes nibble q >> 1; weights are nibble - 8.
template <>
struct GT<RLH_TYPE_Q4_0> {
  static constexpr bool kNeedS = false;
  static constexpr bool kBlockMajor = true;
  struct W {
    uint64_t qs[8];
    u32x4_t dv;
  };
  __device__ __forceinline__ static void load(W& r, const DevMat& w, uint32_t row, uint32_t j, uint32_t q) {
    const ItemPtr p = item_ptr(w, row, j);
#pragma unroll
    for (int k = 0; k < 8; k++) r.qs[k] = g8(at(p, 16 * k + 8 * (q & 1)));
    r.dv = g16(at(p, 128));
  }
  __device__ __forceinline__ static void compute(const W (&wr)[2], const StageView& v, const Lane& ln,
                                                 float (&acc)[2][2][4]) {
    const uint64_t m4 = 0x0F0F0F0F0F0F0F0Full, hi = 0x8080808080808080ull, k8 = 0x0808080808080808ull;
    uint64_t qs[2][8];
    uint32_t dw[2][4];
#pragma unroll
    for (int tc = 0; tc < 2; tc++) {
#pragma unroll
      for (int k = 0; k < 8; k++) qs[tc][k] = wr[tc].qs[k];
      dw[tc][0] = wr[tc].dv.x;
      dw[tc][1] = wr[tc].dv.y;
      dw[tc][2] = wr[tc].dv.z;
      dw[tc][3] = wr[tc].dv.w;
    }
#pragma unroll 2
    for (int k = 0; k < 8; k++) {
      float dk[2];
      uint64_t b[2];
#pragma unroll
      for (int tc = 0; tc < 2; tc++) {
        dk[tc] = f16_to_f32((dw[tc][0] >> (16 * (k & 1))) & 0xffff);
        const uint64_t nib = (qs[tc][0] >> (4 * (ln.q >> 1))) & m4;
        b[tc] = ((nib | hi) - k8) ^ hi;
      }
#pragma unroll
      for (int tr = 0; tr < 2; tr++) {
        const long a = a_frag(v, ln, tr, k);
        const f32x4_t da = tok4(v.d, ln, tr, k);
#pragma unroll
        for (int tc = 0; tc < 2; tc++) {
          const v4i ci = mfma(a, b[tc]);
#pragma unroll
          for (int e = 0; e < 4; e++)  // simd.rs:863
            acc[tr][tc][e] = acc[tr][tc][e] + dk[tc] * (float)ci[e] * da[e];
        }
      }
#pragma unroll
      for (int tc = 0; tc < 2; tc++) {
        rotate(qs[tc]);
        if (k & 1) {
          dw[tc][0] = dw[tc][1];
          dw[tc][1] = dw[tc][2];
          dw[tc][2] = dw[tc][3];
        }
      }
    }
  }
};

// Stages super-block j of the block's 64 tokens: Q8 bytes into the padded
// [64][272] layout (17 slots of 16 bytes per token, the 17th unused), the 8
// block scales of every token, and for Q4_K the 8 block sums (as f32) and the
// 64 rows' scale headers turned into {d*sc, dmin*m} pairs. Scales and sums
// are stored block-major ([block][token]) for the types that read them four
// tokens at a time (Q4_K, Q8_0, Q4_0), token-major for Q6_K (four blocks of
// one token at a time). The copy goes through registers: stage_load issues
// the global loads at the top of a super-block step and stage_store writes
// them to LDS at its end, so their latency hides behind the step's products.
// (Copies straight into LDS, global_load_lds, measured ~0.5 us per
// instruction per wave here: the step's copies took as long as its
// products.) Jobs of thread t, wave w = t / 64 (every role is whole waves,
// so the branches are uniform): jobs 0-3 Q8 slots t + 256k; job 4 Q8 slots
// 1024-1087 (wave 0), the scales (waves 1-2: 128 slots of 16 bytes, token
// (t - 64) / 2, blocks 4 ((t - 64) & 1) .. +3), the sums of tokens 0-31
// (wave 3, Q4_K); job 5 (Q4_K) the sums of tokens 32-63 (wave 0) and the
// row headers (wave 1). Slots past the valid tokens or the 17th slot of a
// token load a clamped, valid address and are not stored.
constexpr uint32_t kStageJobs = 6;

struct StageRegs {
  u32x4_t v[kStageJobs];
  const uint8_t* src[kStageJobs];  // job k's source for the current super-block (not the header job)
  uint32_t keep;                   // bit k: job k is stored
  uint32_t sub4, sub5;             // jobs 4/5: scale or sum slot (token * 2 + half), or the header row
};

__device__ __forceinline__ uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Sources of super-block 0; super-block j + 1 is 256 bytes further for Q8
// bytes and 32 bytes for scales and sums; the header job addresses item
// (row, j) itself.
__device__ __forceinline__ void stage_init(StageRegs& r, const GemmArgs& a, uint32_t t0, bool q4k) {
  const uint32_t cols = a.w.cols, nb = cols / 32, t = threadIdx.x, w = wave_id();
  r.keep = 0;
  auto q8_job = [&](uint32_t k, uint32_t p) {
    const uint32_t tok = p / 17, ch = p - tok * 17;
    r.keep |= (ch < 16 && t0 + tok < a.n) ? 1u << k : 0u;
    r.src[k] = (const uint8_t*)a.x.qs + (size_t)min(t0 + tok, a.n - 1) * cols + 16 * min(ch, 15u);
  };
  auto small_job = [&](uint32_t k, const void* base, uint32_t slot) {
    const uint32_t tok = slot >> 1;
    r.keep |= t0 + tok < a.n ? 1u << k : 0u;
    r.src[k] = (const uint8_t*)base + ((size_t)min(t0 + tok, a.n - 1) * nb + 4 * (slot & 1)) * 4;
  };
#pragma unroll
  for (uint32_t k = 0; k < 4; k++) q8_job(k, t + 256 * k);
  r.sub4 = r.sub5 = 0;
  r.src[4] = r.src[5] = (const uint8_t*)a.x.d;
  if (w == 0) {
    q8_job(4, t + 1024);
  } else if (w <= 2) {
    r.sub4 = t - 64;
    small_job(4, a.x.d, r.sub4);
  } else if (q4k) {
    r.sub4 = t - 192;
    small_job(4, a.x.s, r.sub4);
  }
  if (q4k && w == 0) {
    r.sub5 = t + 64;
    small_job(5, a.x.s, r.sub5);
  } else if (q4k && w == 1) {
    r.sub5 = t - 64;
    r.keep |= 1u << 5;
  }
}

// q8_dma: the Q8 byte jobs (0..3, and job 4 of wave 0) go by DMA
// (stage_dma_q8) and are skipped here.
__device__ __forceinline__ void stage_load(StageRegs& r, const GemmArgs& a, uint32_t row0, uint32_t j, bool q4k,
                                           bool q8_dma = false) {
  const uint32_t w = wave_id();
#pragma unroll
  for (uint32_t k = 0; k < 5; k++) {
    if (q8_dma && (k < 4 || w == 0)) continue;
    r.v[k] = *(const RLH_GLOBAL u32x4_t*)r.src[k];
    r.src[k] += (k < 4 || w == 0) ? 256 : 32;
  }
  if (q4k && w == 0) {
    r.v[5] = *(const RLH_GLOBAL u32x4_t*)r.src[5];
    r.src[5] += 32;
  } else if (q4k && w == 1) {  // the row's d, dmin and 12 scale bytes (item bytes 0..15)
    r.v[5] = *(const RLH_GLOBAL u32x4_t*)item_ptr(a.w, min(row0 + r.sub5, a.w.rows - 1), j).base;
  }
}

// Q6_K stages super-block j by DMA straight into `buf` (global_load_lds, 16
// bytes per lane; no staging registers): the 64 tokens' Q8 bytes (1088
// pieces of 16 bytes, token p / 17, piece p % 17; the pad piece repeats
// piece 15 and tokens past n repeat the last one, neither is read for a
// kept output) and the token-major block scales (128 slots of 16 bytes).
// Every wave issues its copies; the caller waits for them (vmcnt) and then
// the block barrier.
__device__ __forceinline__ void stage_dma_q8(const GemmArgs& a, uint32_t t0, uint32_t j, lbyte* buf) {
  const uint32_t cols = a.w.cols, lane = threadIdx.x & 63, w = wave_id();
  auto q8_piece = [&](uint32_t p0) {  // pieces p0 .. p0 + 63, p0 a multiple of 64
    const uint32_t p = p0 + lane, tok = p / 17, ch = p - tok * 17;
    const int8_t* src = a.x.qs + (size_t)min(t0 + tok, a.n - 1) * cols + 256 * j + 16 * min(ch, 15u);
    __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)src, (RLH_LDS void*)(buf + p0 * 16), 16, 0, 0);
  };
#pragma unroll
  for (uint32_t k = 0; k < 4; k++) q8_piece(64 * w + 256 * k);
  if (w == 0) q8_piece(1024);
}
__device__ __forceinline__ void stage_dma(const GemmArgs& a, uint32_t t0, uint32_t j, lbyte* buf) {
  const uint32_t nb = a.w.cols / 32, lane = threadIdx.x & 63, w = wave_id();
  stage_dma_q8(a, t0, j, buf);
  if (w == 1 || w == 2) {  // scale slots (token slot >> 1, blocks 4 (slot & 1) .. +3)
    const uint32_t slot = 64 * (w - 1) + lane, tok = slot >> 1;
    const float* src = a.x.d + (size_t)min(t0 + tok, a.n - 1) * nb + 8 * j + 4 * (slot & 1);
    __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)src,
                                     (RLH_LDS void*)(buf + kXBytes + 4 * 64 * (w - 1) * 4), 16, 0, 0);
  }
}

// A scale or sum slot (token slot >> 1, blocks 4 (slot & 1) .. +3) into LDS.
__device__ __forceinline__ void store_small(lbyte* buf, bool sum, bool block_major, uint32_t slot, const u32x4_t& v) {
  RLH_LDS float* base = (RLH_LDS float*)(buf + kXBytes + (sum ? kDBytes : 0u));
  const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
  if (block_major) {
    RLH_LDS float* t = base + 4 * (slot & 1) * kTile + (slot >> 1);
#pragma unroll
    for (int i = 0; i < 4; i++) t[i * kTile] = sum ? (float)(int32_t)w4[i] : __uint_as_float(w4[i]);
  } else {
    *(RLH_LDS u32x4_t*)(base + 4 * slot) = v;
  }
}

template <bool kBlockMajor>
__device__ __forceinline__ void stage_store(const StageRegs& r, lbyte* buf, bool q4k, bool q8_dma = false) {
  const uint32_t t = threadIdx.x, w = wave_id();
  if (!q8_dma) {
#pragma unroll
    for (uint32_t k = 0; k < 4; k++)
      if (r.keep >> k & 1u) *(RLH_LDS u32x4_t*)(buf + (t + 256 * k) * 16) = r.v[k];
  }
  if (r.keep >> 4 & 1u) {
    if (w == 0) {
      if (!q8_dma) *(RLH_LDS u32x4_t*)(buf + (t + 1024) * 16) = r.v[4];
    } else {
      store_small(buf, w == 3, kBlockMajor, r.sub4, r.v[4]);
    }
  }
  if (q4k && (r.keep >> 5 & 1u)) {
    if (w == 0) {
      store_small(buf, true, kBlockMajor, r.sub5, r.v[5]);
    } else {
      // get_scale_min_k4 (quant.rs:176-185) of the 8 sub-blocks; the pairs
      // d*sc, dmin*m of sub-blocks 2g, 2g+1 (exact in f32: an f16 times a
      // 6-bit integer)
      const u32x4_t v = r.v[5];
      RLH_LDS f32x4_t* rs = (RLH_LDS f32x4_t*)(buf + kXBytes + 2 * kDBytes);
      const float dd = f16_to_f32(v.x & 0xffff), dmin = f16_to_f32(v.x >> 16);
      const uint32_t s0 = v.y, s1 = v.z, s2 = v.w;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        uint32_t sc[2], m[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const uint32_t sh = 16 * (g & 1) + 8 * h;
          if (g < 2) {
            sc[h] = (s0 >> sh) & 63;
            m[h] = (s1 >> sh) & 63;
          } else {
            sc[h] = ((s2 >> sh) & 0xF) | (((s0 >> sh) >> 6 & 3) << 4);
            m[h] = ((s2 >> sh) >> 4 & 0xF) | (((s1 >> sh) >> 6 & 3) << 4);
          }
        }
        rs[g * kTile + r.sub5] = f32x4_t{dd * (float)sc[0], dmin * (float)m[0], dd * (float)sc[1], dmin * (float)m[1]};
      }
    }
  }
}

// Q4_K fits 166 VGPRs when asked for three waves per SIMD (no scratch), so a
// CU holds three of its blocks (3 x 51 KB of LDS); the other types keep the
// allocator's choice.
template <uint32_t TY>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TY == RLH_TYPE_Q4_K ? 3 : 1)))
k_gemm(GemmArgs a0) {
  using G = GT<TY>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_generic[];
  lbyte* lds = (lbyte*)lds_generic;
  // XCD-aware tile order (see file header)
  const uint32_t b = blockIdx.x, xcd = b & 7, k = b >> 3;
  const uint32_t tt = k % a0.n_tt, rtg = (k / a0.n_tt) * 8 + xcd;
  if (rtg >= a0.n_rt) return;  // whole block, before any barrier
  // the block's segment (uniform: from the block index)
  GemmArgs a = a0;
  uint32_t rt = rtg;
  if (rtg >= a0.n_rt1) {
    a.w = a0.w2;
    a.y = a0.y2;
    a.resid = nullptr;
    rt = rtg - a0.n_rt1;
  }
  const uint32_t t0 = tt * kTile, r0 = rt * kTile;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Lane ln{lane >> 4, lane & 15, wave & 1, wave >> 1};
  const uint32_t rows = a.w.rows, nsb = a.w.cols >> 8;
  uint32_t rowc[2];
#pragma unroll
  for (int tc = 0; tc < 2; tc++) {
    const uint32_t r = r0 + 32 * ln.rw + 16 * tc + ln.i16;
    rowc[tc] = r < rows ? r : rows - 1;  // loads stay inside the matrix
  }
  float acc[2][2][4];
#pragma unroll
  for (int tr = 0; tr < 2; tr++)
#pragma unroll
    for (int tc = 0; tc < 2; tc++)
#pragma unroll
      for (int e = 0; e < 4; e++) acc[tr][tc][e] = 0.0f;

  typename G::W wc[2], wn[2];
  if constexpr (TY == RLH_TYPE_Q6_K) {
    // stages by DMA (stage_dma): the copies of super-block j + 1 are issued
    // with its weight loads and waited for before the loop's barrier
#pragma unroll
    for (int tc = 0; tc < 2; tc++) G::load(wc[tc], a.w, rowc[tc], 0, ln.q);
    stage_dma(a, t0, 0, lds);
    wait_vmcnt<0>();
    __syncthreads();
    for (uint32_t j = 0; j < nsb; j++) {
      const bool more = j + 1 < nsb;
      if (more) {
        stage_dma(a, t0, j + 1, lds + ((j + 1) & 1) * kStageBytes);  // freed by the last barrier
#pragma unroll
        for (int tc = 0; tc < 2; tc++) G::load(wn[tc], a.w, rowc[tc], j + 1, ln.q);
      }
      G::compute(wc, view(lds + (j & 1) * kStageBytes), ln, acc);
      if (more) {
#pragma unroll
        for (int tc = 0; tc < 2; tc++) wc[tc] = wn[tc];
      }
      wait_vmcnt<0>();  // this wave's copies (and weights) of super-block j + 1 have landed
      __syncthreads();  // ... every wave's; the current buffer is free
    }
  } else {
  // the Q8 bytes by DMA (stage_dma_q8), the block scales, sums and row
  // scales through registers (they are converted or transposed on the way)
  StageRegs sr;
#pragma unroll
  for (int tc = 0; tc < 2; tc++) G::load(wc[tc], a.w, rowc[tc], 0, ln.q);
  stage_init(sr, a, t0, G::kNeedS);
  stage_dma_q8(a, t0, 0, lds);
  stage_load(sr, a, r0, 0, G::kNeedS, true);
  stage_store<G::kBlockMajor>(sr, lds, G::kNeedS, true);
  wait_vmcnt<0>();
  __syncthreads();
  for (uint32_t j = 0; j < nsb; j++) {
    const bool more = j + 1 < nsb;
    if (more) {
      stage_dma_q8(a, t0, j + 1, lds + ((j + 1) & 1) * kStageBytes);  // freed by the last barrier
      stage_load(sr, a, r0, j + 1, G::kNeedS, true);
#pragma unroll
      for (int tc = 0; tc < 2; tc++) G::load(wn[tc], a.w, rowc[tc], j + 1, ln.q);
    }
    G::compute(wc, view(lds + (j & 1) * kStageBytes), ln, acc);
    if (more) {
#pragma unroll
      for (int tc = 0; tc < 2; tc++) wc[tc] = wn[tc];
      stage_store<G::kBlockMajor>(sr, lds + ((j + 1) & 1) * kStageBytes, G::kNeedS, true);
    }
    wait_vmcnt<0>();  // this wave's copies of super-block j + 1 have landed
    __syncthreads();  // ... every wave's; the current buffer is free
  }
  }
#pragma unroll
  for (int tr = 0; tr < 2; tr++)
#pragma unroll
    for (int tc = 0; tc < 2; tc++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t tok = t0 + 32 * ln.tw + 16 * tr + 4 * ln.q + e;
        const uint32_t row = r0 + 32 * ln.rw + 16 * tc + ln.i16;
        if (tok < a.n && row < rows) {
          const size_t idx = (size_t)tok * rows + row;
          if (a.resid) {
            RLH_GLOBAL float* x = (RLH_GLOBAL float*)a.resid;
            x[idx] = x[idx] + acc[tr][tc][e];  // xs += xb (model.rs:548-552, 569-573)
          }
          if (a.y) ((RLH_GLOBAL float*)a.y)[idx] = acc[tr][tc][e];
        }
      }
}

// ---------------------------------------------------------------------------
// Prefill products for the types with no integer batch path in the reference
// (Q5_K, Q4_1, Q5_0, Q5_1, F16, BF16): matmul_batch's f32 route (ops.rs:237-312)
// dequantizes rows (quant.rs:191-385) and runs dot_multi_rows::<3, 4>
// (simd.rs:779-836) on the f32 activations. Every output of a token group of
// 4 is one 8-lane FMA chain over the row (lane l takes elements 8i + l in
// order) reduced by the AVX2 tree; the last n % 4 tokens take dot_f32_avx2
// (32 chains over 32-value chunks, (a0+a1)+(a2+a3), tree). ys starts at zero
// and gets `+= value`. F32 weights take matmul_batch's F32 fast path
// (ops.rs:165-174): dot(row, x) for every token, stored as is.
// Block: 16 rows x 16 tokens, one thread per (row, token) running its
// chains; each 256-value super-block of the 16 rows is dequantized into LDS
// once and the 16 tokens' activations staged beside it.
// ---------------------------------------------------------------------------
constexpr uint32_t kFR = 16, kFT = 16, kFS = 260;  // rows, tokens, LDS floats per 256 values

struct GemmF32Args {
  DevMat w;
  const float* x;  // [n][cols] f32
  uint32_t n;
  float* y;
  float* resid;
  uint32_t n4;     // tokens handled in groups of 4 (n - n % 4)
};

__device__ __forceinline__ float tree8(const float* A) {
  return ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
}

// Values 16 * dp .. 16 * dp + 15 of super-block j (256 values) of row r,
// dequantized exactly (quant.rs:191-385). The loads come first, the
// conversion second, so that callers can place a barrier between them.
template <uint32_t TY>
struct Dq16 {
  u32x4_t v[4];  // raw bytes
  uint32_t aux0, aux1;
  __device__ __forceinline__ void load(const DevMat& w, uint32_t r, uint32_t j, uint32_t dp) {
    if constexpr (TY == RLH_TYPE_Q5_K) {
      const uint32_t dsub = dp / 2, dl = 16 * (dp % 2);
      v[0] = *(const RLH_GLOBAL u32x4_t*)(w.a + item_offset(w, r, j, 0));
      v[1] = *(const RLH_GLOBAL u32x4_t*)(w.a + item_offset(w, r, j, 48 + 32 * (dsub / 2) + dl));
      v[2] = *(const RLH_GLOBAL u32x4_t*)(w.a + item_offset(w, r, j, 16 + dl));
    } else if constexpr (TY == RLH_TYPE_Q4_1 || TY == RLH_TYPE_Q5_0 || TY == RLH_TYPE_Q5_1) {
      const uint32_t k = dp / 2;  // the 32-value block
      v[0] = *(const RLH_GLOBAL u32x4_t*)(w.a + item_offset(w, r, j, 16 * k));
      const uint32_t sc0 = TY == RLH_TYPE_Q4_1 ? 128 : 160;
      if constexpr (TY != RLH_TYPE_Q4_1) aux1 = *(const RLH_GLOBAL uint32_t*)(w.a + item_offset(w, r, j, 128 + 4 * k));
      if constexpr (TY == RLH_TYPE_Q5_0)
        aux0 = *(const RLH_GLOBAL uint16_t*)(w.a + item_offset(w, r, j, sc0 + 2 * k));
      else
        aux0 = *(const RLH_GLOBAL uint32_t*)(w.a + item_offset(w, r, j, sc0 + 4 * k));
    } else if constexpr (TY == RLH_TYPE_F16 || TY == RLH_TYPE_BF16) {
      const uint8_t* p = w.a + (size_t)r * w.row_bytes + 2 * (256 * (size_t)j + 16 * dp);
      v[0] = *(const RLH_GLOBAL u32x4_t*)p;
      v[1] = *(const RLH_GLOBAL u32x4_t*)(p + 16);
    } else {  // F32
      const uint8_t* p = w.a + (size_t)r * w.row_bytes + 4 * (256 * (size_t)j + 16 * dp);
#pragma unroll
      for (int q = 0; q < 4; q++) v[q] = *(const RLH_GLOBAL u32x4_t*)(p + 16 * q);
    }
  }
  __device__ __forceinline__ void values(uint32_t dp, f32x4_t* o) const {
    if constexpr (TY == RLH_TYPE_Q5_K) {
      const uint32_t dsub = dp / 2;
      const u32x4_t hdr = v[0], qv = v[1], hv = v[2];
      const float d = f16_to_f32(hdr.x & 0xffff), dmin = f16_to_f32(hdr.x >> 16);
      uint8_t sb[12];
      const uint32_t sw[3] = {hdr.y, hdr.z, hdr.w};
#pragma unroll
      for (int k = 0; k < 12; k++) sb[k] = (uint8_t)(sw[k / 4] >> (8 * (k % 4)));
      uint32_t sc, m;
      scale_min_k4((int)dsub, sb, sc, m);
      const float d1 = d * (float)sc, mm1 = dmin * (float)m;
      const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w}, hw[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t u = ((qw[q] >> (4 * (dsub & 1))) & 0x0F0F0F0Fu) | (((hw[q] >> dsub) & 0x01010101u) << 4);
        o[q].x = d1 * (float)(u & 0xff) - mm1;
        o[q].y = d1 * (float)((u >> 8) & 0xff) - mm1;
        o[q].z = d1 * (float)((u >> 16) & 0xff) - mm1;
        o[q].w = d1 * (float)(u >> 24) - mm1;
      }
    } else if constexpr (TY == RLH_TYPE_Q4_1 || TY == RLH_TYPE_Q5_0 || TY == RLH_TYPE_Q5_1) {
      const uint32_t half = dp % 2;  // values 16 * half .. + 15 of the block
      const uint32_t qw[4] = {v[0].x, v[0].y, v[0].z, v[0].w};
      float d, m = 0.0f;
      if constexpr (TY == RLH_TYPE_Q5_0) {
        d = f16_to_f32(aux0 & 0xffff);
      } else {
        d = f16_to_f32(aux0 & 0xffff);
        m = f16_to_f32(aux0 >> 16);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float e[4];
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const uint32_t i = 4 * q + b;  // byte i of the block's quants
          uint32_t x = (qw[q] >> (8 * b + 4 * half)) & 0xF;
          if constexpr (TY != RLH_TYPE_Q4_1) x |= ((aux1 >> (i + 16 * half)) & 1u) << 4;
          if constexpr (TY == RLH_TYPE_Q5_0)
            e[b] = (float)((int)x - 16) * d;
          else
            e[b] = (float)x * d + m;
        }
        o[q] = f32x4_t{e[0], e[1], e[2], e[3]};
      }
    } else if constexpr (TY == RLH_TYPE_F16 || TY == RLH_TYPE_BF16) {
      const uint32_t hw[8] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w};
      auto cv = [](uint32_t h) {
        return TY == RLH_TYPE_F16 ? f16_to_f32(h) : __uint_as_float(h << 16);  // quant.rs:115-157, bf16_to_f32
      };
#pragma unroll
      for (int q = 0; q < 4; q++)
        o[q] = f32x4_t{cv(hw[2 * q] & 0xffff), cv(hw[2 * q] >> 16), cv(hw[2 * q + 1] & 0xffff),
                       cv(hw[2 * q + 1] >> 16)};
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++)
        o[q] = f32x4_t{__uint_as_float(v[q].x), __uint_as_float(v[q].y), __uint_as_float(v[q].z),
                       __uint_as_float(v[q].w)};
    }
  }
};

template <uint32_t TY>
__global__ void __launch_bounds__(256) k_gemm_f32(GemmF32Args a) {
  __shared__ __attribute__((aligned(16))) float ws_g[kFR * kFS];
  __shared__ __attribute__((aligned(16))) float xs_g[kFT * kFS];
  typedef RLH_LDS float lfloat;
  typedef RLH_LDS f32x4_t lf32x4;
  lfloat* ws = (lfloat*)ws_g;
  lfloat* xs = (lfloat*)xs_g;
  const uint32_t tid = threadIdx.x, r0 = blockIdx.x * kFR, t0 = blockIdx.y * kFT;
  const uint32_t rl = tid / kFT, tl = tid % kFT, row = r0 + rl, tok = t0 + tl;
  const uint32_t nsb = a.w.cols / 256;
  const bool tail = tok >= a.n4;
  // dequant duty: row r0 + tid / 16, values 16 * (tid % 16) .. + 15 of the super-block
  const uint32_t dr = tid / 16, dp = tid % 16;
  const uint32_t drow = min(r0 + dr, a.w.rows - 1);
  float c8[8], c32[4][8];
#pragma unroll
  for (int l = 0; l < 8; l++) {
    c8[l] = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; m++) c32[m][l] = 0.0f;
  }
  for (uint32_t j = 0; j < nsb; j++) {
    Dq16<TY> dq;
    dq.load(a.w, drow, j, dp);
    f32x4_t xv[4];
    const uint32_t xt = min(t0 + tid / 16, a.n - 1);
#pragma unroll
    for (int q = 0; q < 4; q++)  // token t0 + tid / 16, values 16 * (tid % 16) + 4q
      xv[q] = *(const RLH_GLOBAL f32x4_t*)(a.x + (size_t)xt * a.w.cols + 256 * j + 16 * (tid % 16) + 4 * q);
    f32x4_t wv[4];
    dq.values(dp, wv);
    __syncthreads();  // the previous super-block's tiles are consumed
#pragma unroll
    for (int q = 0; q < 4; q++) {
      *(lf32x4*)(ws + dr * kFS + 16 * dp + 4 * q) = wv[q];
      *(lf32x4*)(xs + (tid / 16) * kFS + 16 * (tid % 16) + 4 * q) = xv[q];
    }
    __syncthreads();
    const lf32x4* w4 = (const lf32x4*)(ws + rl * kFS);
    const lf32x4* x4 = (const lf32x4*)(xs + tl * kFS);
    if (!tail) {  // dot_multi_rows: lane l of the 8-wide chain takes 8i + l
#pragma unroll 8
      for (int i = 0; i < 32; i++) {
        const f32x4_t wa = w4[2 * i], wb = w4[2 * i + 1], xa = x4[2 * i], xb = x4[2 * i + 1];
        c8[0] = __builtin_fmaf(wa.x, xa.x, c8[0]);
        c8[1] = __builtin_fmaf(wa.y, xa.y, c8[1]);
        c8[2] = __builtin_fmaf(wa.z, xa.z, c8[2]);
        c8[3] = __builtin_fmaf(wa.w, xa.w, c8[3]);
        c8[4] = __builtin_fmaf(wb.x, xb.x, c8[4]);
        c8[5] = __builtin_fmaf(wb.y, xb.y, c8[5]);
        c8[6] = __builtin_fmaf(wb.z, xb.z, c8[6]);
        c8[7] = __builtin_fmaf(wb.w, xb.w, c8[7]);
      }
    } else {  // dot_f32_avx2: chain (m, l) takes 32c + 8m + l
#pragma unroll 2
      for (int c = 0; c < 8; c++) {
#pragma unroll
        for (int mq = 0; mq < 4; mq++) {
          const f32x4_t wa = w4[8 * c + 2 * mq], wb = w4[8 * c + 2 * mq + 1];
          const f32x4_t xa = x4[8 * c + 2 * mq], xb = x4[8 * c + 2 * mq + 1];
          c32[mq][0] = __builtin_fmaf(wa.x, xa.x, c32[mq][0]);
          c32[mq][1] = __builtin_fmaf(wa.y, xa.y, c32[mq][1]);
          c32[mq][2] = __builtin_fmaf(wa.z, xa.z, c32[mq][2]);
          c32[mq][3] = __builtin_fmaf(wa.w, xa.w, c32[mq][3]);
          c32[mq][4] = __builtin_fmaf(wb.x, xb.x, c32[mq][4]);
          c32[mq][5] = __builtin_fmaf(wb.y, xb.y, c32[mq][5]);
          c32[mq][6] = __builtin_fmaf(wb.z, xb.z, c32[mq][6]);
          c32[mq][7] = __builtin_fmaf(wb.w, xb.w, c32[mq][7]);
        }
      }
    }
  }
  if (row >= a.w.rows || tok >= a.n) return;
  float v;
  if (!tail) {
    v = 0.0f + (tree8(c8) + 0.0f);  // out += hsum(acc) + tail (no tail: cols % 8 == 0)
  } else {
    float A[8];
#pragma unroll
    for (int l = 0; l < 8; l++) A[l] = (c32[0][l] + c32[1][l]) + (c32[2][l] + c32[3][l]);
    // F32 weights store dot(row, x) (ops.rs:169-173); the others add it to
    // the zeroed output (ops.rs:236 ys.fill, then +=)
    v = TY == RLH_TYPE_F32 ? tree8(A) : 0.0f + tree8(A);
  }
  const size_t idx = (size_t)tok * a.w.rows + row;
  if (a.resid) {
    RLH_GLOBAL float* x = (RLH_GLOBAL float*)a.resid;
    x[idx] = x[idx] + v;
  }
  if (a.y) ((RLH_GLOBAL float*)a.y)[idx] = v;
}

}  // namespace

bool gemm_supported(uint32_t ty) {
  return ty == RLH_TYPE_Q4_K || ty == RLH_TYPE_Q6_K || ty == RLH_TYPE_Q8_0 || ty == RLH_TYPE_Q4_0;
}

bool gemm_f32_supported(uint32_t ty) {
  return ty == RLH_TYPE_Q5_K || ty == RLH_TYPE_Q4_1 || ty == RLH_TYPE_Q5_0 || ty == RLH_TYPE_Q5_1 ||
         ty == RLH_TYPE_F16 || ty == RLH_TYPE_BF16 || ty == RLH_TYPE_F32;
}

void launch_gemm_f32(hipStream_t st, const DevMat& w, const float* x, uint32_t n, uint32_t n4, float* y,
                     float* resid) {
  GemmF32Args a{};
  a.w = w;
  a.x = x;
  a.n = n;
  a.n4 = n4;
  a.y = y;
  a.resid = resid;
  if (w.ty == RLH_TYPE_F32) a.n4 = 0;  // every token takes dot_f32_avx2 (ops.rs:165-174)
  const dim3 grid((w.rows + kFR - 1) / kFR, (n + kFT - 1) / kFT);
  switch (w.ty) {
    case RLH_TYPE_Q5_K: hipLaunchKernelGGL(k_gemm_f32<RLH_TYPE_Q5_K>, grid, dim3(256), 0, st, a); break;
    case RLH_TYPE_Q4_1: hipLaunchKernelGGL(k_gemm_f32<RLH_TYPE_Q4_1>, grid, dim3(256), 0, st, a); break;
    case RLH_TYPE_Q5_0: hipLaunchKernelGGL(k_gemm_f32<RLH_TYPE_Q5_0>, grid, dim3(256), 0, st, a); break;
    case RLH_TYPE_Q5_1: hipLaunchKernelGGL(k_gemm_f32<RLH_TYPE_Q5_1>, grid, dim3(256), 0, st, a); break;
    case RLH_TYPE_F16: hipLaunchKernelGGL(k_gemm_f32<RLH_TYPE_F16>, grid, dim3(256), 0, st, a); break;
    case RLH_TYPE_BF16: hipLaunchKernelGGL(k_gemm_f32<RLH_TYPE_BF16>, grid, dim3(256), 0, st, a); break;
    case RLH_TYPE_F32: hipLaunchKernelGGL(k_gemm_f32<RLH_TYPE_F32>, grid, dim3(256), 0, st, a); break;
    default: break;
  }
}

static void launch_gemm_args(hipStream_t st, uint32_t ty, const GemmArgs& a) {
  const uint32_t blocks = a.n_tt * ((a.n_rt + 7) / 8) * 8;
  const size_t lds = 2 * kStageBytes;
  switch (ty) {
    case RLH_TYPE_Q4_K: hipLaunchKernelGGL(k_gemm<RLH_TYPE_Q4_K>, dim3(blocks), dim3(256), lds, st, a); break;
    case RLH_TYPE_Q6_K: hipLaunchKernelGGL(k_gemm<RLH_TYPE_Q6_K>, dim3(blocks), dim3(256), lds, st, a); break;
    case RLH_TYPE_Q8_0: hipLaunchKernelGGL(k_gemm<RLH_TYPE_Q8_0>, dim3(blocks), dim3(256), lds, st, a); break;
    case RLH_TYPE_Q4_0: hipLaunchKernelGGL(k_gemm<RLH_TYPE_Q4_0>, dim3(blocks), dim3(256), lds, st, a); break;
    default: break;
  }
}

bool gemm_pair_supported(const DevMat& w, const DevMat& w2) {
  return gemm_supported(w.ty) && w2.ty == w.ty && w2.cols == w.cols;
}

void launch_gemm_pair(hipStream_t st, const DevMat& w, const DevMat& w2, const Q8Mut& x, uint32_t n, float* y,
                      float* y2) {
  GemmArgs a{};
  a.w = w;
  a.w2 = w2;
  a.x = Q8Ptr{x.qs, x.d, x.s, x.s16};
  a.n = n;
  a.y = y;
  a.y2 = y2;
  a.n_tt = (n + kTile - 1) / kTile;
  a.n_rt1 = (w.rows + kTile - 1) / kTile;
  a.n_rt = a.n_rt1 + (w2.rows + kTile - 1) / kTile;
  launch_gemm_args(st, w.ty, a);
}

void launch_gemm(hipStream_t st, const DevMat& w, const Q8Mut& x, uint32_t n, float* y, float* resid) {
  GemmArgs a{};
  a.w = w;
  a.x = Q8Ptr{x.qs, x.d, x.s, x.s16};
  a.n = n;
  a.y = y;
  a.resid = resid;
  a.n_tt = (n + kTile - 1) / kTile;
  a.n_rt = (w.rows + kTile - 1) / kTile;
  a.n_rt1 = a.n_rt;
  launch_gemm_args(st, w.ty, a);
}

}  // namespace rlh
