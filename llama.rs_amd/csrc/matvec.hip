// matvec.hip — decode matvec (ops.rs:67-141, integer path) for gfx950.
//
// Exactness: every row's f32 total is the sequential sum, in the reference's
// index order, of the per-group terms of dot_q4k_q8_avx2 (simd.rs:581),
// dot_q6k_q8_avx2 (simd.rs:663), dot_q80_q8_avx2 (simd.rs:891) or
// dot_q40_q8_avx2 (simd.rs:863), each term evaluated with the reference's
// expression and rounding.
//
// Structure (HBM-bound, one pass over the weights):
//  * A block owns R rows (whole row-tiles of the tiled weight layout, see
//    rlh_format.h); wave w takes the block's tiles w, w + waves, ... A lane
//    owns one item (a 256-value super-block of one row) of the tile and
//    loads it with 16-byte loads that are contiguous across the wave, so
//    every load instruction reads 1 KB of HBM while the scale unpacking and
//    address arithmetic are paid once per 256 weights.
//  * The activation is a Q8 row in HBM (Q8Row, simd.rs:88-101), staged into
//    LDS with global_load_lds issued ahead of the first weights.
//    Q8 super-blocks are stored in LDS with a 16-byte pad so that lanes on
//    different super-blocks hit different banks.
//  * Every item writes its terms into the block's LDS tile [row][term]; after
//    one barrier, lane r of wave 0 adds row r's terms in order (the
//    reference's `total +=` chain) and runs the epilogue.
//  * PAIR mode multiplies the same rows of ffn_gate and ffn_up and writes
//    h = silu(gate) * up (ops.rs:393-395, model.rs:722-724) with its Q8
//    blocks. Single mode can add into the residual (model.rs:714-716,
//    726-728) or leave each block's greedy-argmax candidate of the logits.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include <algorithm>
#include <cstdlib>

#include "kernels.h"
#include "matvec.h"
#include "rlh_device.h"

namespace rlh {

namespace {

typedef RLH_LDS float lfloat;
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef RLH_LDS f32x4_t lf32x4;
typedef RLH_LDS u32x4_t lu32x4;

constexpr uint32_t kSbStride = 272;  // LDS bytes per 256 Q8 values (16-byte pad)

// Q8 activation row in LDS (Q8Row, simd.rs:88-101).
struct LAct {
  RLH_LDS int8_t* qs;  // padded: value i at (i / 256) * kSbStride + i % 256
  RLH_LDS float* d;
  RLH_LDS int32_t* s;
  RLH_LDS float* s16x32;  // 32.0f * (float)sums16 (the Q6_K correction, exact in f32)
  RLH_LDS float* xf;      // f32 row, padded: value i at (i / 256) * kXfStride + i % 256
};

constexpr uint32_t kXfStride = 260;  // LDS floats per 256 f32 activation values (16-byte pad)

__device__ __forceinline__ const RLH_LDS int8_t* qblk(const LAct& a, uint32_t b) {
  return a.qs + (b >> 3) * kSbStride + (b & 7) * 32;
}
__device__ __forceinline__ u32x4_t lds_u4(const RLH_LDS int8_t* p) { return *(const lu32x4*)p; }
// Weight loads: every weight is read once per token, so the loads carry the
// non-temporal hint (nt); measured faster than ordinary loads on every shape.
__device__ __forceinline__ u32x4_t gl_u4(const void* p) {
  return __builtin_nontemporal_load((const RLH_GLOBAL u32x4_t*)p);
}

__device__ __forceinline__ int dot16(u32x4_t w, u32x4_t a, int acc) {
  acc = sdot4(w.x, a.x, acc);
  acc = sdot4(w.y, a.y, acc);
  acc = sdot4(w.z, a.z, acc);
  return sdot4(w.w, a.w, acc);
}

// Makes a tile's weight registers opaque at the start of its terms: the
// unpacking (nibble masks, scale shifts) depends only on the weights, and
// without this the compiler may move it next to the loads of the tile, where
// it waits for the data that was meant to stream in behind other work.
template <class W>
__device__ __forceinline__ void weights_ready(W& r) {
  static_assert(sizeof(W) % 16 == 0, "item registers are whole 16-byte loads");
  u32x4_t* p = reinterpret_cast<u32x4_t*>(&r);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(W) / 16); i++) asm volatile("" : "+v"(p[i]));
}

// ---- work items: one super-block of one row ---------------------------------
// An item is streamed in kParts parts (halves of its super-block, each with
// the item's small scale words again), so that a wave keeps one part in
// flight while it computes the previous one. Part h of kParts writes the
// item's terms [h * kT / kParts, (h + 1) * kT / kParts).
template <uint32_t TY>
struct MI;

template <>
struct MI<RLH_TYPE_Q4_K> {
  static constexpr uint32_t kT = 4;
  static constexpr int kParts = 2;
  static constexpr int kQ = 8 / kParts;  // 16-byte quant chunks per part
  static constexpr int kLoads = kQ + 1;  // vector-memory loads per part
  struct P {
    u32x4_t hdr, q[kQ];
  };
  __device__ __forceinline__ static void load(P& r, const uint8_t* tile, uint32_t lane, int h) {
    r.hdr = gl_u4(tile + lane * 16);
#pragma unroll
    for (int k = 0; k < kQ; k++) r.q[k] = gl_u4(tile + (h * kQ + k + 1) * 1024 + lane * 16);
  }
  // Group g: low nibbles of q[2g], q[2g+1] = sub-block 2g, high = 2g+1.
  __device__ __forceinline__ static void terms(const P& r, const LAct& act, uint32_t j, lfloat* t, int h) {
    const uint32_t m4 = 0x0F0F0F0Fu;
    const float d = f16_to_f32(r.hdr.x & 0xffff);
    const float dmin = f16_to_f32(r.hdr.x >> 16);
    const uint32_t s0 = r.hdr.y, s1 = r.hdr.z, s2 = r.hdr.w;  // the 12 scale bytes
    float out[kQ / 2];
#pragma unroll
    for (int gl = 0; gl < kQ / 2; gl++) {
      const int g = h * (kQ / 2) + gl;
      // get_scale_min_k4 (quant.rs:176-185) for sub-blocks 2g and 2g+1
      uint32_t sc1, m1, sc2, m2;
      if (g < 2) {
        const uint32_t sh1 = 16 * g, sh2 = 16 * g + 8;
        sc1 = (s0 >> sh1) & 63;
        m1 = (s1 >> sh1) & 63;
        sc2 = (s0 >> sh2) & 63;
        m2 = (s1 >> sh2) & 63;
      } else {
        const uint32_t sh1 = 16 * (g - 2), sh2 = sh1 + 8;
        sc1 = ((s2 >> sh1) & 0xF) | (((s0 >> sh1) >> 6 & 3) << 4);
        m1 = ((s2 >> sh1) >> 4 & 0xF) | (((s1 >> sh1) >> 6 & 3) << 4);
        sc2 = ((s2 >> sh2) & 0xF) | (((s0 >> sh2) >> 6 & 3) << 4);
        m2 = ((s2 >> sh2) >> 4 & 0xF) | (((s1 >> sh2) >> 6 & 3) << 4);
      }
      const uint32_t ab = j * 8 + 2 * g;
      const RLH_LDS int8_t* pa = qblk(act, ab);
      const u32x4_t a0 = lds_u4(pa), a1 = lds_u4(pa + 16), b0 = lds_u4(pa + 32), b1 = lds_u4(pa + 48);
      const u32x4_t q0 = r.q[2 * gl], q1 = r.q[2 * gl + 1];
      int i1 = dot16(q0 & m4, a0, 0);
      i1 = dot16(q1 & m4, a1, i1);
      int i2 = dot16((q0 >> 4) & m4, b0, 0);
      i2 = dot16((q1 >> 4) & m4, b1, i2);
      const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
      const float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
      const float da = act.d[ab], db = act.d[ab + 1];
      const float sa = (float)act.s[ab], sb = (float)act.s[ab + 1];
      out[gl] = da * (d1 * (float)i1 - mm1 * sa) + db * (d2 * (float)i2 - mm2 * sb);
    }
#pragma unroll
    for (int gl = 0; gl < kQ / 2; gl++) t[h * (kQ / 2) + gl] = out[gl];
  }
};

// Q6_K terms in the reference order: for half { for sub { for c } }
// (simd.rs:611-666), 16 per super-block; part h = half h.
template <>
struct MI<RLH_TYPE_Q6_K> {
  static constexpr uint32_t kT = 16;
  static constexpr int kParts = 2;
  static constexpr int kLoads = 8;
  struct P {
    u32x4_t ql[4], qh[2], sc;
    u32x4_t d;  // .x = the f16 scale (the other lanes unused)
  };
  __device__ __forceinline__ static void load(P& r, const uint8_t* tile, uint32_t lane, int h) {
#pragma unroll
    for (int k = 0; k < 4; k++) r.ql[k] = gl_u4(tile + (4 * h + k) * 1024 + lane * 16);
#pragma unroll
    for (int k = 0; k < 2; k++) r.qh[k] = gl_u4(tile + (8 + 2 * h + k) * 1024 + lane * 16);
    r.sc = gl_u4(tile + 12 * 1024 + lane * 16);
    r.d = u32x4_t{ld_g2(tile + 13 * 1024 + lane * 2), 0u, 0u, 0u};
  }
  __device__ __forceinline__ static void terms(const P& r, const LAct& act, uint32_t j, lfloat* t, int h) {
    const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x03030303u;
    const float d = f16_to_f32(r.d.x);
    const uint32_t wlo = h ? r.sc.z : r.sc.x, whi = h ? r.sc.w : r.sc.y;  // the half's 8 scale bytes
    const uint32_t ab = j * 8 + 4 * h;
    // the half's 128 activation bytes, scales and 16-value sums, read in
    // one batch so the LDS latency is paid once per half
    u32x4_t av[4][2];
    float da[4], sa[4][2];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      av[c][0] = lds_u4(qblk(act, ab + c));
      av[c][1] = lds_u4(qblk(act, ab + c) + 16);
      da[c] = act.d[ab + c];
      sa[c][0] = act.s16x32[(ab + c) * 2];
      sa[c][1] = act.s16x32[(ab + c) * 2 + 1];
    }
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const u32x4_t ql0 = r.ql[s], ql1 = r.ql[2 + s], qh = r.qh[s];
      float out[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const u32x4_t lo = (c & 1) ? ql1 : ql0;
        const u32x4_t nib = (c < 2) ? (lo & m4) : ((lo >> 4) & m4);
        const u32x4_t uu = nib | (((qh >> (2 * c)) & m2) << 4);
        const int ss = dot16(uu, av[c][s], 0);
        const uint32_t bi = s + 2 * c;  // sc[sub + 2c] (simd.rs:626-629)
        const float scf = (float)(int8_t)(((bi < 4 ? wlo : whi) >> (8 * (bi & 3))) & 0xff);
        out[c] = d * scf * ((float)ss - sa[c][s]) * da[c];
      }
      *(lf32x4*)(t + 8 * h + 4 * s) = f32x4_t{out[0], out[1], out[2], out[3]};
    }
  }
};

// Q8_0: item = 8 consecutive 32-value blocks (256 values); part h = blocks
// 4h .. 4h+3.
template <>
struct MI<RLH_TYPE_Q8_0> {
  static constexpr uint32_t kT = 8;
  static constexpr int kParts = 2;
  static constexpr int kLoads = 9;
  struct P {
    u32x4_t q[8], dv;
  };
  __device__ __forceinline__ static void load(P& r, const uint8_t* tile, uint32_t lane, int h) {
#pragma unroll
    for (int k = 0; k < 8; k++) r.q[k] = gl_u4(tile + (8 * h + k) * 1024 + lane * 16);
    r.dv = gl_u4(tile + 16 * 1024 + lane * 16);
  }
  __device__ __forceinline__ static void terms(const P& r, const LAct& act, uint32_t j, lfloat* t, int h) {
    const uint32_t dw[4] = {r.dv.x, r.dv.y, r.dv.z, r.dv.w};
    float out[4];
#pragma unroll
    for (int kl = 0; kl < 4; kl++) {
      const int k = 4 * h + kl;
      const uint32_t b = j * 8 + k;
      const RLH_LDS int8_t* pa = qblk(act, b);
      const int i = dot16(r.q[2 * kl + 1], lds_u4(pa + 16), dot16(r.q[2 * kl], lds_u4(pa), 0));
      const float dk = f16_to_f32((dw[k >> 1] >> (16 * (k & 1))) & 0xffff);
      out[kl] = dk * (float)i * act.d[b];  // simd.rs:891
    }
    *(lf32x4*)(t + 4 * h) = f32x4_t{out[0], out[1], out[2], out[3]};
  }
};

// Q4_0: item = 8 consecutive 32-value blocks; part h = blocks 4h .. 4h+3.
template <>
struct MI<RLH_TYPE_Q4_0> {
  static constexpr uint32_t kT = 8;
  static constexpr int kParts = 2;
  static constexpr int kLoads = 5;
  struct P {
    u32x4_t q[4], dv;
  };
  __device__ __forceinline__ static void load(P& r, const uint8_t* tile, uint32_t lane, int h) {
#pragma unroll
    for (int k = 0; k < 4; k++) r.q[k] = gl_u4(tile + (4 * h + k) * 1024 + lane * 16);
    r.dv = gl_u4(tile + 8 * 1024 + lane * 16);
  }
  __device__ __forceinline__ static void terms(const P& r, const LAct& act, uint32_t j, lfloat* t, int h) {
    const uint32_t m4 = 0x0F0F0F0Fu;
    const uint32_t dw[4] = {r.dv.x, r.dv.y, r.dv.z, r.dv.w};
    float out[4];
#pragma unroll
    for (int kl = 0; kl < 4; kl++) {
      const int k = 4 * h + kl;
      const uint32_t b = j * 8 + k;
      const RLH_LDS int8_t* pa = qblk(act, b);
      const int i0 = dot16(r.q[kl] & m4, lds_u4(pa), 0);
      const int i1 = dot16((r.q[kl] >> 4) & m4, lds_u4(pa + 16), 0);
      const float dk = f16_to_f32((dw[k >> 1] >> (16 * (k & 1))) & 0xffff);
      out[kl] = dk * (float)(i0 + i1 - 8 * act.s[b]) * act.d[b];  // simd.rs:863
    }
    *(lf32x4*)(t + 4 * h) = f32x4_t{out[0], out[1], out[2], out[3]};
  }
};

// Q5_K: no integer kernel in the reference; the row is
// sum over super-blocks, in order, of dot_f32_avx2(dequant(block), x_block)
// (dequant_dot_scalar's generic fallback, quant.rs:528-539, with ops::dot =
// simd.rs:328-377 for 256 values): slot (m, l) is the FMA chain over the
// eight 32-value chunks c of element 32c + 8m + l, A_l = (a0+a1)+(a2+a3),
// then the AVX2 tree. Dequant (quant.rs:313-349): d1 * (q + 16*hbit) - mm1.
// One term per super-block, one part (the chains run through all chunks).
template <>
struct MI<RLH_TYPE_Q5_K> {
  static constexpr uint32_t kT = 1;
  static constexpr int kParts = 1;
  static constexpr int kLoads = 11;
  struct P {
    u32x4_t hdr, qh[2], q[8];
  };
  __device__ __forceinline__ static void load(P& r, const uint8_t* tile, uint32_t lane, int) {
    r.hdr = gl_u4(tile + lane * 16);
    r.qh[0] = gl_u4(tile + 1024 + lane * 16);
    r.qh[1] = gl_u4(tile + 2048 + lane * 16);
#pragma unroll
    for (int k = 0; k < 8; k++) r.q[k] = gl_u4(tile + (k + 3) * 1024 + lane * 16);
  }
  __device__ __forceinline__ static void terms(const P& r, const LAct& act, uint32_t j, lfloat* t, int) {
    const float d = f16_to_f32(r.hdr.x & 0xffff);
    const float dmin = f16_to_f32(r.hdr.x >> 16);
    const uint32_t s0 = r.hdr.y, s1 = r.hdr.z, s2 = r.hdr.w;
    const lf32x4* x4 = (const lf32x4*)(act.xf + j * kXfStride);
    const uint32_t qh[8] = {r.qh[0].x, r.qh[0].y, r.qh[0].z, r.qh[0].w, r.qh[1].x, r.qh[1].y, r.qh[1].z, r.qh[1].w};
    float a[4][8];
#pragma unroll
    for (int mm = 0; mm < 4; mm++)
#pragma unroll
      for (int l = 0; l < 8; l++) a[mm][l] = 0.0f;
    // one sub-block (32 values, chunk c of dot_f32_avx2) per iteration; the
    // chains start at +0.0 as _mm256_setzero_ps does
#pragma unroll 1
    for (int c = 0; c < 8; c++) {
      const int g = c >> 1, sh4 = 4 * (c & 1), sh = 8 * (c & 3);
      const uint32_t sc_lo = (s0 >> sh) & 63, m_lo = (s1 >> sh) & 63;
      const uint32_t sc_hi = ((s2 >> sh) & 0xF) | (((s0 >> sh) >> 6 & 3) << 4);
      const uint32_t m_hi = ((s2 >> sh) >> 4 & 0xF) | (((s1 >> sh) >> 6 & 3) << 4);
      const uint32_t sc = c < 4 ? sc_lo : sc_hi, m = c < 4 ? m_lo : m_hi;
      const float d1 = d * (float)sc, mm1 = dmin * (float)m;
      const u32x4_t qa = g == 0 ? r.q[0] : (g == 1 ? r.q[2] : (g == 2 ? r.q[4] : r.q[6]));
      const u32x4_t qb = g == 0 ? r.q[1] : (g == 1 ? r.q[3] : (g == 2 ? r.q[5] : r.q[7]));
      const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
      for (int w4 = 0; w4 < 8; w4++) {  // values 4*w4 .. 4*w4+3 of the sub-block
        const uint32_t nib = (qw[w4] >> sh4) & 0x0F0F0F0Fu;
        const uint32_t hb = ((qh[w4] >> c) & 0x01010101u) << 4;
        const uint32_t v = nib | hb;  // 4 bytes of q + 16 * hbit
        const f32x4_t xv = x4[8 * c + w4];
        const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const int i = 4 * w4 + b, mi = i >> 3, l = i & 7;
          const float wv = d1 * (float)((v >> (8 * b)) & 0xff) - mm1;
          a[mi][l] = __builtin_fmaf(wv, xs[b], a[mi][l]);
        }
      }
    }
    float A[8];
#pragma unroll
    for (int l = 0; l < 8; l++) A[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    t[0] = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
  }
};

// Q4_1 / Q5_0 / Q5_1: no integer kernel in the reference; the row is
// dequant_dot_scalar's generic fallback (quant.rs:528-539): per 32-value
// block, dequant_row (quant.rs:222-272) then ops::dot, which for 32 values is
// dot_f32_avx2 (simd.rs:328-377) with one chunk: slot (m, l) = fma(w, x, +0)
// of value 8m + l, A_l = (a0+a1)+(a2+a3), the AVX2 tree. One term per block,
// added to the row total in block order; part h = blocks 4h .. 4h+3. Item
// chunks: 0-7 the blocks' quants, then qh (8-9; Q5_0/Q5_1), then d / (d, m).
template <uint32_t TY>
struct MI32f {
  static constexpr bool kHi = TY != RLH_TYPE_Q4_1;  // a fifth bit per value
  static constexpr bool kMin = TY != RLH_TYPE_Q5_0;  // q * d + m (else (q - 16) * d)
  static constexpr uint32_t kT = 8;
  static constexpr int kParts = 2;
  static constexpr int kLoads = kHi ? 6 : 5;
  struct P {
    u32x4_t q[4], sc, hi;  // hi: qh of the part's blocks (zero for Q4_1)
  };
  __device__ __forceinline__ static void load(P& r, const uint8_t* tile, uint32_t lane, int h) {
#pragma unroll
    for (int k = 0; k < 4; k++) r.q[k] = gl_u4(tile + (4 * h + k) * 1024 + lane * 16);
    if (kHi) {
      r.hi = gl_u4(tile + (8 + h) * 1024 + lane * 16);
      r.sc = gl_u4(tile + (kMin ? 10 + h : 10) * 1024 + lane * 16);
    } else {
      r.hi = u32x4_t{0u, 0u, 0u, 0u};
      r.sc = gl_u4(tile + (8 + h) * 1024 + lane * 16);
    }
  }
  __device__ __forceinline__ static void terms(const P& r, const LAct& act, uint32_t j, lfloat* t, int h) {
    const lf32x4* x4 = (const lf32x4*)(act.xf + j * kXfStride);
    const uint32_t sw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
    const uint32_t hw[4] = {r.hi.x, r.hi.y, r.hi.z, r.hi.w};
    float out[4];
#pragma unroll
    for (int kl = 0; kl < 4; kl++) {
      const int k = 4 * h + kl;
      float d, m = 0.0f;
      if (kMin) {
        d = f16_to_f32(sw[kl] & 0xffff);
        m = f16_to_f32(sw[kl] >> 16);
      } else {
        d = f16_to_f32((sw[k >> 1] >> (16 * (k & 1))) & 0xffff);
      }
      const u32x4_t qv = r.q[kl];
      const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
      float a[4][8];
#pragma unroll
      for (int c = 0; c < 8; c++) {  // values 4c .. 4c+3 of the block
        const f32x4_t xv = x4[8 * k + c];
        const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const int e = 4 * c + b;
          const uint32_t byte = (qw[(e & 15) >> 2] >> (8 * (e & 3))) & 0xff;
          uint32_t q = e < 16 ? (byte & 0xF) : (byte >> 4);
          if (kHi) q |= ((hw[kl] >> e) & 1u) << 4;
          const float wv = kMin ? (float)q * d + m : (float)((int)q - 16) * d;
          a[e >> 3][e & 7] = __builtin_fmaf(wv, xs[b], 0.0f);
        }
      }
      float A[8];
#pragma unroll
      for (int l = 0; l < 8; l++) A[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
      out[kl] = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
    }
    *(lf32x4*)(t + 4 * h) = f32x4_t{out[0], out[1], out[2], out[3]};
  }
};
template <>
struct MI<RLH_TYPE_Q4_1> : MI32f<RLH_TYPE_Q4_1> {};
template <>
struct MI<RLH_TYPE_Q5_0> : MI32f<RLH_TYPE_Q5_0> {};
template <>
struct MI<RLH_TYPE_Q5_1> : MI32f<RLH_TYPE_Q5_1> {};

// In-order sum of n terms (the per-row f32 chain).
__device__ __forceinline__ float chain(const lfloat* t, uint32_t n) { return seq_sum_lds(t, n); }

// Asynchronous copies HBM -> LDS with global_load_lds (no registers
// involved, so they overlap the weight loads already in flight). lds_dma4:
// n bytes (a multiple of 4) in 256-byte pieces, wave `wave` of `nw` taking
// pieces wave, wave + nw, ...; lanes past the end are masked off.
__device__ __forceinline__ void lds_dma4(RLH_LDS void* dst, const void* src, uint32_t n, uint32_t wave, uint32_t nw) {
  const uint32_t lane = threadIdx.x & 63;
  for (uint32_t off = wave * 256; off < n; off += nw * 256) {
    if (off + lane * 4 < n)
      __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)((const uint8_t*)src + off + lane * 4),
                                       (RLH_LDS void*)((RLH_LDS uint8_t*)dst + off), 4, 0, 0);
  }
}

// Stages the Q8 activation row (HBM, Q8Row layout) into LDS by DMA. The
// quants go to the padded layout (17 slots of 16 bytes per 256 values, the
// 17th empty): lane i of a copy fills slot s0 + i, so its source is chosen per
// slot and the pad slots are simply masked off. act_finish runs after the
// copies have landed (wait_vmcnt) and turns the 16-value sums into floats.
__device__ __forceinline__ void act_dma(const MvLaunch& L, const LAct& la) {
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const uint32_t cols = L.cols, nsb = cols >> 8, nb = cols >> 5, nslots = nsb * 17;
  if (L.need_q8) {
    for (uint32_t s0 = wave * 64; s0 < nslots; s0 += nw * 64) {
      const uint32_t p = s0 + lane, sb = p / 17, ch = p - sb * 17;
      if (p < nslots && ch < 16)
        __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)(L.act.qs + sb * 256 + ch * 16),
                                         (RLH_LDS void*)(la.qs + s0 * 16), 16, 0, 0);
    }
    lds_dma4(la.d, L.act.d, nb * 4, wave, nw);
    lds_dma4(la.s, L.act.s, nb * 4, wave, nw);
    lds_dma4(la.s16x32, L.act.s16, nb * 8, wave, nw);
  }
  if (L.need_xf)  // the f32 row, one 256-value super-block per wave instruction
    for (uint32_t sb = wave; sb < nsb; sb += nw)
      __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)(L.xf + sb * 256 + lane * 4),
                                       (RLH_LDS void*)(la.xf + sb * kXfStride), 16, 0, 0);
}

__device__ __forceinline__ void act_finish(const MvLaunch& L, const LAct& la) {
  const uint32_t nb = L.need_q8 ? L.cols >> 5 : 0u;
  lds_barrier();
  for (uint32_t i = threadIdx.x; i < 2 * nb; i += blockDim.x) {
    const int v = ((RLH_LDS int32_t*)la.s16x32)[i];
    la.s16x32[i] = 32.0f * (float)v;
  }
  lds_barrier();
}

// Norm input: every block computes quantize_q8(rmsnorm(x, w)) itself
// (k_rmsnorm_q8's arithmetic), or quantize_q8(x) when there is no norm
// weight (nw null: the attention output entering attn_output). norm_dma
// copies the row and the norm weights into LDS (xs, ws: the term tiles, free
// until the terms are written); norm_finish, after the copies have landed,
// runs the 32 FMA chains of the sum of squares in wave 0, then each group of
// 8 threads quantizes one 32-value block straight into the LDS activation.
__device__ __forceinline__ void norm_dma(const MvLaunch& L, lfloat* xs, lfloat* ws) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const uint32_t nbytes = L.cols * 4;  // a multiple of 1024
  for (uint32_t off = wave * 1024; off < nbytes; off += nw * 1024) {
    __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)((const uint8_t*)L.nx + off + lane * 16),
                                     (RLH_LDS void*)((RLH_LDS uint8_t*)xs + off), 16, 0, 0);
    if (L.nw)
      __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)((const uint8_t*)L.nw + off + lane * 16),
                                       (RLH_LDS void*)((RLH_LDS uint8_t*)ws + off), 16, 0, 0);
  }
}

__device__ __forceinline__ void norm_finish(const MvLaunch& L, const LAct& la, const lfloat* xs, const lfloat* ws,
                                            lfloat* misc) {
  const uint32_t tid = threadIdx.x, NT = blockDim.x, n4 = L.cols / 4;
  const bool nrm = L.nw != nullptr;
  lds_barrier();
  if (nrm && tid < 64) {
    const float ss = rms_sumsq_lds(xs, (int)L.cols);
    if (tid == 0) misc[0] = 1.0f / sqrtf(ss / (float)L.cols + L.eps);
  }
  lds_barrier();
  const float s = nrm ? misc[0] : 1.0f;
  const lf32x4* x4 = (const lf32x4*)xs;
  const lf32x4* w4 = (const lf32x4*)ws;
  // n4 and NT are multiples of 8: whole 8-lane groups stay active together
  for (uint32_t i = tid; i < n4; i += NT) {
    const f32x4_t xr = x4[i], wr = nrm ? w4[i] : f32x4_t{1.0f, 1.0f, 1.0f, 1.0f};
    // without a norm weight (x * 1) * 1 == x exactly: the plain quantize_q8
    const float v0 = (xr.x * s) * wr.x, v1 = (xr.y * s) * wr.y;
    const float v2 = (xr.z * s) * wr.z, v3 = (xr.w * s) * wr.w;
    if (L.need_xf) *(lf32x4*)(la.xf + (i >> 6) * kXfStride + 4 * (i & 63)) = f32x4_t{v0, v1, v2, v3};
    const Q8Blk8x4 r = q8_block8x4(v0, v1, v2, v3);
    const uint32_t blk = i / 8, l = i & 7;
    *(RLH_LDS uint32_t*)(la.qs + (blk >> 3) * kSbStride + (blk & 7) * 32 + 4 * l) = r.packed;
    if (l == 0) {
      la.d[blk] = r.d;
      la.s[blk] = r.tot;
      la.s16x32[2 * blk] = 32.0f * (float)r.s;
    } else if (l == 4) {
      la.s16x32[2 * blk + 1] = 32.0f * (float)r.s;
    }
  }
  lds_barrier();
}

__device__ __forceinline__ void argmax_merge(float& bv, uint32_t& bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__device__ __forceinline__ void wave_argmax(float& bv, uint32_t& bi) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m);
    const uint32_t oi = __shfl_xor(bi, m);
    argmax_merge(bv, bi, ov, oi);
  }
}

// Float weights (F16, F32, BF16: rows as stored, no tiles). The reference's
// row products are chains over the whole row: F16 (simd.rs:401-419) eight
// FMA chains, lane l taking values 8i + l, then the AVX2 tree; F32 weights
// (ops.rs:77-83, dot_f32_avx2 simd.rs:328-377) 32 FMA chains, chain (m, l)
// taking 32c + 8m + l, then (a0+a1)+(a2+a3) and the tree; BF16
// (quant.rs:427-433) one chain acc += w * x in index order.
// A block owns R rows (16, 32 in PAIR mode, 64 beside tiled segments). The
// rows stream through LDS in stages of 32 KB per matrix (16 KB in PAIR mode;
// a stage holds 1/R of it from each row), double buffered: every thread
// loads its 16-byte pieces of the next stage into registers while the chains
// run over the current one, and stores them after it. F16 and F32 chains are (matrix,
// row, slot) triples spread over the block's threads, carried in registers
// across stages; BF16 chains (one per row) read eight values per LDS read.
// Lane r of wave m then reduces row r's slots; the epilogue is the tiled
// path's.
__host__ __device__ constexpr uint32_t mv_float_slots(uint32_t ty) {
  return ty == RLH_TYPE_F32 ? 32u : (ty == RLH_TYPE_F16 ? 8u : 1u);
}
// bytes per matrix per stage: 32 KB (16 KB in PAIR mode, two matrices)
__host__ __device__ constexpr uint32_t mv_float_stage(uint32_t nm) { return nm == 2 ? 16384u : 32768u; }
__host__ __device__ constexpr uint32_t mv_float_stage_bytes(uint32_t nm, uint32_t R) {
  return nm * 2u * R * (mv_float_stage(nm) / R + 16);  // rows padded by 16 bytes
}

template <uint32_t TY, int NM>
__device__ __forceinline__ void mv_block_float(const MvLaunch& L, const MvSeg& g, uint32_t blk, lfloat* lds,
                                               lfloat* misc, lu64* exp_tab) {
  constexpr uint32_t S = mv_float_slots(TY);
  constexpr uint32_t ES = TY == RLH_TYPE_F32 ? 4u : 2u;
  constexpr uint32_t kPer = (NM * 64u * S + 511u) / 512u;  // chains per thread at most (R <= 64)
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t R = L.rows_per_blk, cols = L.cols, nsb = cols >> 8, nb = cols >> 5;
  const uint32_t rows = g.w.rows, row0 = blk * R;
  const uint32_t nrows = rows - row0 < R ? rows - row0 : R;
  const uint32_t stride = L.tile_stride;
  constexpr uint32_t kJ = mv_float_stage(NM) / 8192u;   // 16-byte pieces per thread per matrix
  const uint32_t RY = mv_float_stage(NM) / R, RS = RY + 16;  // row bytes per stage, LDS row stride
  const uint32_t C = RY / ES;                           // values per row per stage
  const uint32_t PR = RY / 16;                          // 16-byte pieces per row per stage
  const uint32_t bufb = NM * R * RS;                    // bytes of one stage buffer
  LAct la;
  la.qs = (RLH_LDS int8_t*)lds;
  la.d = (RLH_LDS float*)((RLH_LDS int8_t*)lds + nsb * kSbStride);
  la.s = (RLH_LDS int32_t*)(la.d + nb);
  la.s16x32 = (RLH_LDS float*)(la.s + nb);
  la.xf = (RLH_LDS float*)((RLH_LDS int8_t*)lds + L.xf_off);
  lfloat* region = (lfloat*)((RLH_LDS int8_t*)lds + L.region_off);
  // stage buffers after the chain results (the norm prologue's row copies
  // overlap them; the first stage is stored after the prologue)
  RLH_LDS uint8_t* stg = (RLH_LDS uint8_t*)(region + NM * R * stride);
  float rsd = 0.0f;
  if (NM == 1 && g.resid && wave == 0) rsd = ld_gf(g.resid + row0 + min(lane, nrows - 1));
  lfloat* xs = region;
  lfloat* ws = region + cols;
  if (NM == 2 && wave == 0) exp_tab_dma(exp_tab);
  if (L.nx) norm_dma(L, xs, ws);
  else act_dma(L, la);
  __builtin_amdgcn_sched_barrier(0);  // the copies stay ahead of the weight loads
  // piece k of this thread: P = tid + 512 (k % kJ) of matrix k / kJ: row
  // P / PR (clamped to the valid rows), 16 bytes at 16 (P % PR) of the stage
  constexpr int NP = (int)kJ * NM;
  const uint8_t* src[NP];
  uint32_t dof[NP];
#pragma unroll
  for (int k = 0; k < NP; k++) {
    const uint32_t P = tid + 512u * (k % kJ), r = P / PR, c = P - r * PR;
    src[k] = (k / kJ ? g.w2.a : g.w.a) + (size_t)(row0 + min(r, nrows - 1)) * g.w.row_bytes + 16 * c;
    dof[k] = (k / kJ) * R * RS + r * RS + 16 * c;
  }
  u32x4_t pc[NP];
#pragma unroll
  for (int k = 0; k < NP; k++) pc[k] = *(const RLH_GLOBAL u32x4_t*)src[k];
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt<NP>();  // this wave's copies have landed (the weight loads may not)
  if (L.nx) norm_finish(L, la, xs, ws, misc);
  else act_finish(L, la);
#pragma unroll
  for (int k = 0; k < NP; k++) *(RLH_LDS u32x4_t*)(stg + dof[k]) = pc[k];
  float a[kPer];
#pragma unroll
  for (uint32_t i = 0; i < kPer; i++) a[i] = 0.0f;
  const uint32_t nst = cols / C, nchain = NM * R * S;
  for (uint32_t st = 0; st < nst; st++) {
    lds_barrier();  // stage st is in its buffer; the other buffer is free
    const bool more = st + 1 < nst;
    if (more) {
#pragma unroll
      for (int k = 0; k < NP; k++) pc[k] = *(const RLH_GLOBAL u32x4_t*)(src[k] + (size_t)RY * (st + 1));
    }
    const RLH_LDS uint8_t* buf = stg + (st & 1) * bufb;
    const uint32_t e0 = st * C;  // first value of the stage
    if constexpr (TY == RLH_TYPE_BF16) {
      if (tid < nchain) {  // chain = (matrix tid / R, row tid % R): eight values per read
        const RLH_LDS uint8_t* wr = buf + tid * RS;
        float acc = a[0];
#pragma unroll 2
        for (uint32_t k = 0; k < C / 8; k++) {
          const uint32_t e = e0 + 8 * k;  // eight values inside one 256-value super-block
          const lfloat* xr = la.xf + (e >> 8) * kXfStride + (e & 255);
          const u32x4_t w8 = *(const lu32x4*)(wr + 16 * k);
          const f32x4_t xa = *(const lf32x4*)xr, xb = *(const lf32x4*)(xr + 4);
          const uint32_t wv[4] = {w8.x, w8.y, w8.z, w8.w};
          const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const float w = __uint_as_float(i & 1 ? wv[i / 2] & 0xffff0000u : wv[i / 2] << 16);
            acc = acc + w * xv[i];  // acc += w * x: the product rounded, then the add
          }
        }
        a[0] = acc;
      }
    } else {
#pragma unroll
      for (uint32_t i = 0; i < kPer; i++) {
        const uint32_t q = tid + 512u * i;  // chain (matrix q / (R S), row (q / S) % R, slot q % S)
        if (q < nchain) {
          const RLH_LDS uint8_t* wr = buf + (q / S) * RS;  // (matrix, row) rows are consecutive
          const uint32_t s = q % S;
          float acc = a[i];
#pragma unroll 4
          for (uint32_t k = 0; k < C / S; k++) {
            const uint32_t el = k * S + s, e = e0 + el;
            const float x = la.xf[(e >> 8) * kXfStride + (e & 255)];
            float w;
            if constexpr (TY == RLH_TYPE_F32)
              w = *(const lfloat*)(wr + 4 * el);
            else
              w = f16_to_f32(*(const RLH_LDS uint16_t*)(wr + 2 * el));
            acc = __builtin_fmaf(w, x, acc);
          }
          a[i] = acc;
        }
      }
    }
    if (more) {
      RLH_LDS uint8_t* nbuf = stg + ((st + 1) & 1) * bufb;  // freed by this step's barrier
#pragma unroll
      for (int k = 0; k < NP; k++) *(RLH_LDS u32x4_t*)(nbuf + dof[k]) = pc[k];
    }
  }
  // chain results into the tile [matrix][row][slot]
  if constexpr (TY == RLH_TYPE_BF16) {
    if (tid < nchain) region[tid * stride] = a[0];
  } else {
#pragma unroll
    for (uint32_t i = 0; i < kPer; i++) {
      const uint32_t q = tid + 512u * i;
      if (q < nchain) region[(q / S) * stride + q % S] = a[i];
    }
  }
  __syncthreads();
  float acc = 0.0f;
  if (wave < (uint32_t)NM) {
    const lfloat* sl = region + (wave * R + (lane < nrows ? lane : 0)) * stride;
    if constexpr (TY == RLH_TYPE_BF16) {
      acc = sl[0];
    } else {
      float A[8];
#pragma unroll
      for (int l = 0; l < 8; l++) A[l] = TY == RLH_TYPE_F32 ? (sl[l] + sl[8 + l]) + (sl[16 + l] + sl[24 + l]) : sl[l];
      acc = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
    }
  }
  if (NM == 2) {
    if (wave == 1) misc[4 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    const float x = acc, up = misc[4 + lane];
    const float h = (x / (1.0f + expf_glibc_t(-x, exp_tab))) * up;  // ops.rs:393-395
    if (lane < nrows && g.y) ((RLH_GLOBAL float*)g.y)[row0 + lane] = h;
    q8_quant_wave2(h, g.hq, row0 / 32, nrows > 0, nrows > 32);
    return;
  }
  const bool mine = wave == 0 && lane < nrows;
  const uint32_t row = row0 + lane;
  if (mine) {
    if (g.resid) ((RLH_GLOBAL float*)g.resid)[row] = rsd + acc;
    if (g.y) ((RLH_GLOBAL float*)g.y)[row] = acc;
  }
  if (wave != 0 || !L.has_argmax) return;
  const bool cand = mine && acc == acc;
  float bv = cand ? acc : -__int_as_float(0x7f800000);
  uint32_t bi = cand ? row : 0xffffffffu;
  wave_argmax(bv, bi);
  if (lane == 0) {
    ((RLH_GLOBAL float*)L.am.pv)[blockIdx.x] = bv;
    ((RLH_GLOBAL uint32_t*)L.am.pi)[blockIdx.x] = bi;
  }
}

// The body of one block for weight type TY; NM = 2 in PAIR mode (gate and
// up share type and tiling).
template <uint32_t TY, int NM, bool RING = false>
__device__ __forceinline__ void mv_block(const MvLaunch& L, const MvSeg& g, uint32_t blk, lfloat* lds, lfloat* misc,
                                         lu64* exp_tab) {
  if constexpr (TY == RLH_TYPE_F16 || TY == RLH_TYPE_F32 || TY == RLH_TYPE_BF16) {
    mv_block_float<TY, NM>(L, g, blk, lds, misc, exp_tab);
    return;
  } else {
  using I = MI<TY>;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  const uint32_t R = L.rows_per_blk, cols = L.cols, nsb = cols >> 8, nb = cols >> 5;
  const uint32_t TR = g.w.tr, TJ = g.w.tj, ntj = g.w.ntj, RB = R / TR;
  const uint32_t rows = g.w.rows, row0 = blk * R;
  const uint32_t nrows = rows - row0 < R ? rows - row0 : R;
  const uint32_t rt0 = blk * RB, nrt = (rows + TR - 1) / TR;
  const uint32_t ntiles = (nrt - rt0 < RB ? nrt - rt0 : RB) * ntj;
  const size_t tile_bytes = (size_t)64 * g.w.ib;
  const uint32_t stride = L.tile_stride;

  LAct la;
  la.qs = (RLH_LDS int8_t*)lds;
  la.d = (RLH_LDS float*)((RLH_LDS int8_t*)lds + nsb * kSbStride);
  la.s = (RLH_LDS int32_t*)(la.d + nb);
  la.s16x32 = (RLH_LDS float*)(la.s + nb);
  la.xf = (RLH_LDS float*)((RLH_LDS int8_t*)lds + L.xf_off);
  lfloat* region = (lfloat*)((RLH_LDS int8_t*)lds + L.region_off);

  // The wave streams its work as units (tile t, matrix m, part h), one
  // unit in flight: when a unit's data has arrived the next unit's loads are
  // issued, then the arrived unit's terms are computed. More data in flight
  // per wave queues up the requests of the whole chip and every wave's data
  // lands late; measured slower. The staging copies (activation row or norm
  // inputs, silu's table) are issued first and the first unit right after
  // them, so the prologue waits for the copies alone while the weights
  // stream in. The first unit is loaded unconditionally (a wave without a
  // tile loads the last one and never uses it); weights_ready() keeps the
  // compiler from moving a unit's unpacking next to its loads, where it
  // would wait for the data.
  using P = typename I::P;
  constexpr int kP = I::kParts;
  constexpr int kH1 = kP == 2 ? 1 : 0;  // part of the odd units
  // Ring plan (NM = 1, one row tile per block): waves 1.. produce tiles in
  // rounds (producer p takes tiles p, p + np, ...; round r = the r-th tile
  // of every producer), writing round r's terms into slot r % ring of the
  // region, and wave 0 adds each completed round to the row chains in item
  // order. done[s] counts the tiles written into slot s so far (a round is
  // complete when the count reaches the tiles of all rounds of that slot up
  // to it: only the last round may be short); `consumed` counts the rounds
  // wave 0 has added, and a producer writes round r only once round
  // r - ring has been consumed. Relaxed LDS atomics after lgkmcnt(0), as in
  // the split chain below.
  const uint32_t ring = NM == 1 && RING ? L.ring : 0u;  // RING: the ring plans' own instantiation
  const uint32_t np = ring ? nwaves - 1 : nwaves;           // producer waves
  const uint32_t pw = ring ? wave - 1 : wave;               // producer index (wave 0 of a ring: none)
  const bool producer = !ring || wave != 0;
  RLH_LDS uint32_t* ring_done = (RLH_LDS uint32_t*)(misc + 4);  // [ring], then `consumed`
  RLH_LDS uint32_t* ring_consumed = ring_done + 3;
  const uint32_t my_tiles = producer && pw < ntiles ? (ntiles - 1 - pw) / np + 1 : 0;
  const uint32_t nunits = my_tiles * NM * kP;
  auto tile_off = [&](uint32_t t) { return ((size_t)(rt0 + t / ntj) * ntj + t % ntj) * tile_bytes; };
  auto issue = [&](P& r, uint32_t u, int h) {
    const uint32_t t = min(pw + (u / (NM * kP)) * np, ntiles - 1);
    const uint8_t* base = (NM == 2 && (u / kP) % NM == 1) ? g.w2.a : g.w.a;
    I::load(r, base + tile_off(t), lane, h);
  };
  auto work = [&](const P& r, uint32_t u, int h) {
    const uint32_t rr = u / (NM * kP), t = pw + rr * np, m = (u / kP) % NM;
    const uint32_t rl = (t / ntj) * TR + lane % TR, j = (t % ntj) * TJ + lane / TR;
    if (ring)  // slot rr % ring, the round's items from 0 (one row tile: t < ntj)
      I::terms(r, la, j, region + ((rr % ring) * R + rl) * stride + (pw * TJ + lane / TR) * I::kT, h);
    else
      I::terms(r, la, j, region + (m * R + rl) * stride + j * I::kT, h);
  };
  // ring: before the first part of a tile, wait until its slot is free;
  // after the last part, count the tile into its slot
  auto ring_wait = [&](uint32_t u) {
    const uint32_t rr = u / kP;
    if (u % kP != 0 || rr < ring) return;
    wait_lds_count(ring_consumed, rr - ring + 1, L.err, kErrMvRing);  // wave 0 keeps consuming
  };
  auto ring_signal = [&](uint32_t u) {
    if (u % kP != kP - 1) return;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0): the terms are in LDS
    asm volatile("" ::: "memory");
    if (lane == 0)
      __hip_atomic_fetch_add(ring_done + (u / kP) % max(ring, 1u), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  // Split chain (single matrix, two-part items, one row tile per block, a
  // long chain): the waves' tiles come in rounds (tile w + r * nwaves in
  // round r) and the last wave runs out of tiles kr rounds early. Once every
  // wave has finished its first kr tiles (a block counter in LDS), the last
  // wave adds those rounds' terms in order while the others stream the rest;
  // wave 0 continues the chain from that partial sum after the block
  // barrier. Items are ordered by tile, so the first kr rounds hold the
  // row's first kr * nwaves * TJ items.
  const uint32_t kr = ntiles > nwaves ? (ntiles - 1 - (nwaves - 1)) / nwaves + 1 : 0;
  const bool split = !ring && NM == 1 && kP == 2 && RB == 1 && ntiles % nwaves != 0 && kr > 0 && nsb * I::kT >= 256;
  RLH_LDS uint32_t* rounds_done = (RLH_LDS uint32_t*)(misc + 3);
  if (split && tid == 0) *rounds_done = 0u;  // seen by all after the prologue's barriers
  if (ring && tid == 0)
    for (int i = 0; i < 4; i++) ring_done[i] = 0u;
  // the residual of the chain lane's row, read now so that the epilogue
  // does not wait for it
  float rsd = 0.0f;
  if (NM == 1 && g.resid && wave == 0) rsd = ld_gf(g.resid + row0 + min(lane, nrows - 1));
  lfloat* xs = region;
  lfloat* ws = region + cols;
  if (NM == 2 && wave == 0) exp_tab_dma(exp_tab);
  if (L.nx) norm_dma(L, xs, ws);
  else act_dma(L, la);
  __builtin_amdgcn_sched_barrier(0);  // the copies stay ahead of the weight loads
  P ua, ub;
  if (producer) issue(ua, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  if (producer)
    wait_vmcnt<I::kLoads>();  // this wave's copies have landed (the unit's loads may not)
  else
    wait_vmcnt<0>();
  if (L.nx) norm_finish(L, la, xs, ws, misc);
  else act_finish(L, la);
  for (uint32_t u = 0; u < nunits; u += 2) {
    weights_ready(ua);
    if (u + 1 < nunits) issue(ub, u + 1, kH1);
    __builtin_amdgcn_sched_barrier(0);
    if (ring) ring_wait(u);
    work(ua, u, 0);
    if (ring) ring_signal(u);
    if (u + 1 >= nunits) break;
    weights_ready(ub);
    if (u + 2 < nunits) issue(ua, u + 2, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (ring) ring_wait(u + 1);
    work(ub, u + 1, kH1);
    if (ring) ring_signal(u + 1);
    if (split && u / 2 < kr) {  // tile u / 2 (one tile = two units) is done
      // LDS-only hand-over (a wave's LDS operations complete in order):
      // lgkmcnt(0), then a relaxed add; release/acquire atomics would also
      // wait for the unit loads in flight. The asm statements keep the
      // compiler from moving accesses across.
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0): its terms are in LDS
      asm volatile("" ::: "memory");
      if (lane == 0) __hip_atomic_fetch_add(rounds_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  float acc = 0.0f;
  if (ring) {
    if (wave != 0) return;
    // the row chains, round by round as the producers complete them
    const uint32_t nr = (ntiles + np - 1) / np;
    const lfloat* rowp = region + (lane < nrows ? lane : 0) * stride;
    for (uint32_t rr = 0; rr < nr; rr++) {
      const uint32_t s = rr % ring, tin = min(np, ntiles - rr * np), need = np * (rr / ring) + tin;
      wait_lds_count(ring_done + s, need, L.err, kErrMvRing);  // every producer reaches its tiles
      acc = seq_sum_lds(rowp + s * R * stride, tin * TJ * I::kT, acc);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0): the slot's reads are done
      asm volatile("" ::: "memory");
      if (lane == 0) __hip_atomic_fetch_add(ring_consumed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  } else {
  const uint32_t n_early = split ? kr * nwaves * TJ * I::kT : 0u;
  if (split && wave == nwaves - 1) {
    // every wave reaches kr tiles (each has at least kr), so the wait ends
    wait_lds_count(rounds_done, kr * nwaves, L.err, kErrMvSplit);
    misc[4 + lane] = chain(region + (lane < nrows ? lane : 0) * stride, n_early);
  }
  __syncthreads();

  // wave m < NM: lane r adds row r's terms of matrix m in order (after the
  // early part of a split chain); lanes past the valid rows chain a copy of
  // row 0 so that the wave stays converged
  if (wave < (uint32_t)NM)
    acc = seq_sum_lds(region + (wave * R + (lane < nrows ? lane : 0)) * stride + n_early, nsb * I::kT - n_early,
                      split ? misc[4 + lane] : 0.0f);
  }

  if (NM == 2) {
    if (wave == 1) misc[4 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    // h = silu(gate) * up for the block's rows (R is a multiple of 32 and
    // divides the rows, so the lanes form whole Q8 blocks)
    const float x = acc, up = misc[4 + lane];
    const float h = (x / (1.0f + expf_glibc_t(-x, exp_tab))) * up;  // ops.rs:393-395
    if (lane < nrows && g.y) ((RLH_GLOBAL float*)g.y)[row0 + lane] = h;
    q8_quant_wave2(h, g.hq, row0 / 32, nrows > 0, nrows > 32);  // the whole wave: nrows is 32 or 64
    return;
  }

  const bool mine = wave == 0 && lane < nrows;
  const uint32_t row = row0 + lane;
  if (mine) {
    if (g.resid) ((RLH_GLOBAL float*)g.resid)[row] = rsd + acc;
    if (g.y) ((RLH_GLOBAL float*)g.y)[row] = acc;
  }
  if (wave != 0 || !L.has_argmax) return;
  // the block's greedy candidate (max, lowest index); a second launch
  // reduces the candidates of all blocks (main.rs:453-463 semantics)
  // (a NaN row never becomes a candidate: it would stick in the merge)
  const bool cand = mine && acc == acc;
  float bv = cand ? acc : -__int_as_float(0x7f800000);
  uint32_t bi = cand ? row : 0xffffffffu;
  wave_argmax(bv, bi);
  if (lane == 0) {
    ((RLH_GLOBAL float*)L.am.pv)[blockIdx.x] = bv;
    ((RLH_GLOBAL uint32_t*)L.am.pi)[blockIdx.x] = bi;
  }
  }  // tiled types
}

// TY = the weight type of every segment, or 0 for launches that mix types
// (a switch per block); one instantiation per type keeps each kernel's
// register allocation to what its own item type needs.
template <uint32_t TY, int NM, bool RING = false>
__global__ void __launch_bounds__(512) k_mv(MvLaunch L) {
  extern __shared__ __attribute__((aligned(16))) float lds_generic[];
  __shared__ float misc_generic[4 + 64];
  __shared__ uint64_t tab_g[NM == 2 ? 32 : 1];
  lfloat* lds = (lfloat*)lds_generic;
  lfloat* misc = (lfloat*)misc_generic;
  // segment of this block, selected without indexing the argument array
  // (a dynamic index would copy the kernel argument to private memory)
  MvSeg g = L.seg[0];
  if (L.nseg > 1 && blockIdx.x >= L.seg[1].blk_begin) g = L.seg[1];
  if (L.nseg > 2 && blockIdx.x >= L.seg[2].blk_begin) g = L.seg[2];
  const uint32_t blk = blockIdx.x - g.blk_begin;
  if constexpr (TY != 0) {
    mv_block<TY, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g);
  } else {
    switch (g.w.ty) {
      case RLH_TYPE_Q4_K: mv_block<RLH_TYPE_Q4_K, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_Q6_K: mv_block<RLH_TYPE_Q6_K, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_Q8_0: mv_block<RLH_TYPE_Q8_0, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_Q4_0: mv_block<RLH_TYPE_Q4_0, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_Q5_K: mv_block<RLH_TYPE_Q5_K, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_Q4_1: mv_block<RLH_TYPE_Q4_1, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_Q5_0: mv_block<RLH_TYPE_Q5_0, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_Q5_1: mv_block<RLH_TYPE_Q5_1, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_F16: mv_block<RLH_TYPE_F16, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_F32: mv_block<RLH_TYPE_F32, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      case RLH_TYPE_BF16: mv_block<RLH_TYPE_BF16, NM, RING>(L, g, blk, lds, misc, (lu64*)tab_g); break;
      default: break;
    }
  }
}

typedef void (*MvKernel)(MvLaunch);

template <int NM, bool RING = false>
MvKernel mv_kernel(uint32_t ty) {
  switch (ty) {
    case RLH_TYPE_Q4_K: return k_mv<RLH_TYPE_Q4_K, NM, RING>;
    case RLH_TYPE_Q6_K: return k_mv<RLH_TYPE_Q6_K, NM, RING>;
    case RLH_TYPE_Q8_0: return k_mv<RLH_TYPE_Q8_0, NM, RING>;
    case RLH_TYPE_Q4_0: return k_mv<RLH_TYPE_Q4_0, NM, RING>;
    case RLH_TYPE_Q5_K: return k_mv<RLH_TYPE_Q5_K, NM, RING>;
    case RLH_TYPE_Q4_1: return k_mv<RLH_TYPE_Q4_1, NM, RING>;
    case RLH_TYPE_Q5_0: return k_mv<RLH_TYPE_Q5_0, NM, RING>;
    case RLH_TYPE_Q5_1: return k_mv<RLH_TYPE_Q5_1, NM, RING>;
    case RLH_TYPE_F16: return k_mv<RLH_TYPE_F16, NM, RING>;
    case RLH_TYPE_F32: return k_mv<RLH_TYPE_F32, NM, RING>;
    case RLH_TYPE_BF16: return k_mv<RLH_TYPE_BF16, NM, RING>;
    default: return k_mv<0, NM, RING>;
  }
}

constexpr uint32_t kMaxLds = 150u * 1024u;

// Types whose matvec multiplies the f32 activation (the reference's fused f32
// path: no integer kernel for them, ops.rs:93-140).
bool mv_needs_f32(uint32_t ty) {
  return ty == RLH_TYPE_Q5_K || ty == RLH_TYPE_Q4_1 || ty == RLH_TYPE_Q5_0 || ty == RLH_TYPE_Q5_1 ||
         ty == RLH_TYPE_F16 || ty == RLH_TYPE_F32 || ty == RLH_TYPE_BF16;
}
bool mv_is_float(uint32_t ty) { return ty == RLH_TYPE_F16 || ty == RLH_TYPE_F32 || ty == RLH_TYPE_BF16; }

// LDS of a plan with R rows per block: the padded Q8 activation row, the
// padded f32 row when a segment is Q5_K, then the term tiles (which the norm
// prologue borrows for the f32 input row and the norm weights).
uint32_t plan_act_bytes(const MvPlan& p) {
  if (!p.L.need_q8) return 0u;
  const uint32_t nsb = p.L.cols / 256, nb = p.L.cols / 32;
  return (nsb * kSbStride + nb * 16 + 15) & ~15u;
}
uint32_t plan_xf_bytes(const MvPlan& p) { return p.L.need_xf ? (p.L.cols / 256) * kXfStride * 4 : 0u; }
uint32_t plan_lds(const MvPlan& p, uint32_t R, uint32_t nm) {
  const uint32_t cols = p.L.cols, nsb = cols / 256;
  const uint32_t stride = std::max(nsb * p.max_terms + 4, p.slot_stride);
  const uint32_t tile = nm * R * stride * 4 + p.float_stage;  // float plans: stage buffers after the tile
  return plan_act_bytes(p) + plan_xf_bytes(p) + std::max(tile, p.norm ? 2 * cols * 4 : 0u);
}

// Waves of a tiled block of R rows (all eight for a quantize prologue).
uint32_t plan_waves(const MvPlan& p, uint32_t R, uint32_t tr, uint32_t ntj, uint32_t nm) {
  return p.quant ? 8u : std::max<uint32_t>(nm, std::min<uint32_t>(8, (R / tr) * ntj));
}

// Blocks the GPU holds at once (CUs x blocks per CU) for the plan's single
// kernel with `threads` per block and `lds` bytes, 0 if unknown.
uint32_t mv_resident(const MvPlan& p, uint32_t threads, uint32_t lds, bool ring = false) {
  uint32_t ty = p.L.seg[0].w.ty;
  for (uint32_t s = 1; s < p.L.nseg; s++)
    if (p.L.seg[s].w.ty != ty) ty = 0;
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const void* k = ring ? (const void*)mv_kernel<1, true>(ty) : (const void*)mv_kernel<1>(ty);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, (int)threads, lds) !=
      hipSuccess)
    return 0;
  return (uint32_t)(cus * per_cu);
}
uint32_t mv_resident_blocks(const MvPlan& p, uint32_t R, uint32_t tr, uint32_t ntj) {
  return mv_resident(p, 64 * plan_waves(p, R, tr, ntj, 1), plan_lds(p, R, 1));
}

// Ring plan rows: floats per row of one slot (np producers' tiles of tj
// items), 16-byte aligned, padded like the whole-row tiles.
uint32_t ring_stride(const MvPlan& p, uint32_t np, uint32_t tj) { return ((np * tj * p.max_terms + 3) & ~3u) + 4; }
uint32_t ring_lds(const MvPlan& p, uint32_t R, uint32_t np, uint32_t tj, uint32_t slots) {
  return plan_act_bytes(p) + plan_xf_bytes(p) + slots * R * ring_stride(p, np, tj) * 4;
}

uint32_t plan_blocks(const MvPlan& p, uint32_t R) {
  uint32_t b = 0;
  for (uint32_t s = 0; s < p.L.nseg; s++) b += (p.L.seg[s].w.rows + R - 1) / R;
  return b;
}

}  // namespace

void mv_plan_init(MvPlan& p, uint32_t cols, const Q8Mut& act) {
  p = MvPlan{};
  p.L.cols = cols;
  p.L.act = Q8Ptr{act.qs, act.d, act.s, act.s16};
}

void mv_plan_init_norm(MvPlan& p, uint32_t cols, const float* x, const float* w, float eps) {
  p = MvPlan{};
  p.L.cols = cols;
  p.L.nx = x ? x : w;  // a plan made only for its shape may pass null rows
  p.L.nw = w;
  p.L.eps = eps;
  p.norm = true;
}

void mv_plan_init_quant(MvPlan& p, uint32_t cols, const float* x) {
  p = MvPlan{};
  p.L.cols = cols;
  p.L.nx = x;
  p.L.nw = nullptr;
  p.norm = true;
  p.quant = true;
}

void mv_plan_set_f32(MvPlan& p, const float* xf) { p.L.xf = xf; }

void mv_plan_add(MvPlan& p, const DevMat& w, float* y, float* resid) {
  MvSeg& g = p.L.seg[p.L.nseg++];
  g = MvSeg{};
  g.w = w;
  g.y = y;
  g.resid = resid;
  p.rows += w.rows;
  p.max_terms = std::max(p.max_terms, mv_terms_per_sb(w.ty));
}

void mv_plan_add_pair(MvPlan& p, const DevMat& gate, const DevMat& up, const Q8Mut& hq, float* h) {
  MvSeg& g = p.L.seg[p.L.nseg++];
  g = MvSeg{};
  g.w = gate;
  g.w2 = up;
  g.y = h;
  g.hq = hq;
  g.pair = 1;
  p.rows += gate.rows;
  p.max_terms = std::max(p.max_terms, std::max(mv_terms_per_sb(gate.ty), mv_terms_per_sb(up.ty)));
}

void mv_plan_argmax(MvPlan& p, const MvArgmax& am) {
  p.L.has_argmax = 1;
  p.L.am = am;
}

// Block shape: R rows = whole row-tiles, one wave per tile (at most 8
// waves; a block with more tiles loops). Single launches take one row-tile
// per block, launches with the norm prologue two (half the blocks repeat
// it; the quantize-only prologue is cheap and keeps one); a PAIR launch takes 64 rows (its epilogue emits whole Q8 blocks of h,
// one row per lane). Measured on Qwen3-8B shapes against 1-4 tiles per wave
// and 16-64 rows per block.
bool mv_plan_finish(MvPlan& p) {
  const uint32_t nm = (p.L.nseg == 1 && p.L.seg[0].pair) ? 2u : 1u;
  const uint32_t nsb = p.L.cols / 256;
  if (p.L.nseg == 0 || nsb == 0) return false;
  // tiled segments share one tile shape (equal row lengths give equal
  // shapes); float segments (rows as stored) may sit beside them, and then
  // every block takes 64 rows (a whole number of tiles of any shape)
  bool fl = false;
  uint32_t tr = 0, ntj = 1, slots = 0;
  for (uint32_t s = 0; s < p.L.nseg; s++) {
    const DevMat& w = p.L.seg[s].w;
    if (w.cols != p.L.cols) return false;
    if (mv_is_float(w.ty)) {
      fl = true;
      slots = std::max(slots, mv_float_slots(w.ty));
    } else {
      if (!is_tiled(w.ty) || (tr != 0 && w.tr != tr)) return false;
      tr = w.tr;
      ntj = w.ntj;
    }
  }
  const bool tiled_any = tr != 0;
  if (tr == 0) tr = 64;  // float segments only
  if (nm == 2 && (p.L.seg[0].w2.ty != p.L.seg[0].w.ty || p.L.seg[0].w2.rows != p.L.seg[0].w.rows ||
                  p.L.seg[0].w.rows % 32 != 0))
    return false;
  // the epilogue runs one row per lane: R <= 64. Float segments alone take
  // few rows per block (many blocks stream the rows) with whole stages (a
  // row's part of a stage, 32768 / R bytes, must divide the row): 16 rows
  // when the row length is a multiple of 1024 values, 32 for 512, else 64;
  // 32 in PAIR mode (16 KB stages; the Q8 blocks of h); 64 beside tiled
  // segments
  uint32_t R;
  if (fl && !tiled_any)
    R = nm == 2 ? 32u : (p.L.cols % 1024 == 0 ? 16u : (p.L.cols % 512 == 0 ? 32u : 64u));
  else
    R = nm == 2 || fl ? 64u : std::min<uint32_t>(p.norm && !p.quant ? 2 * tr : tr, 64);
  p.L.need_xf = 0;
  for (uint32_t s = 0; s < p.L.nseg; s++)
    if (mv_needs_f32(p.L.seg[s].w.ty) || (p.L.seg[s].pair && mv_needs_f32(p.L.seg[s].w2.ty))) p.L.need_xf = 1;
  if (p.L.need_xf && !p.norm && !p.L.xf) return false;  // f32 products need the f32 activation
  // a launch whose tiled segments all multiply the f32 row stages no Q8 row
  p.L.need_q8 = 1;
  if (!p.norm && !fl) {
    bool all_f32 = true;
    for (uint32_t s = 0; s < p.L.nseg; s++)
      all_f32 = all_f32 && mv_needs_f32(p.L.seg[s].w.ty) && (!p.L.seg[s].pair || mv_needs_f32(p.L.seg[s].w2.ty));
    if (all_f32) p.L.need_q8 = 0;
  }
  p.slot_stride = slots + 1;  // float plans: a row's chain results
  p.float_stage = fl ? mv_float_stage_bytes(nm, R) : 0u;
  // a whole-row plan that exceeds the LDS may still run as a ring plan below
  const bool whole_fits = plan_lds(p, R, nm) <= kMaxLds;
  // A grid just above the blocks the GPU holds at once would run a second,
  // short round of blocks after the first (every block pays its prologue and
  // tail again, and most CUs idle meanwhile): then blocks of twice the rows,
  // when those fit in one round (the 32B q/k/v launch: 320 blocks of 32 rows
  // at one block per CU, 160 of 64)
  if (whole_fits && tiled_any && !fl && nm == 1 && 2 * R <= 64 && plan_lds(p, 2 * R, nm) <= kMaxLds) {
    const uint32_t b0 = plan_blocks(p, R), b1 = plan_blocks(p, 2 * R);
    const uint32_t s0 = mv_resident_blocks(p, R, tr, ntj), s1 = mv_resident_blocks(p, 2 * R, tr, ntj);
    if (s0 && s1 && b0 > s0 && b0 <= 2 * s0 && b1 <= s1) R *= 2;
  }
  if (p.norm && (p.L.cols > (p.quant ? kMvMaxQuantCols : kMvMaxNormCols) || p.L.cols % 256 != 0)) return false;
  // Still more blocks than the GPU holds (rows so long that their whole-row
  // terms leave one block per CU: the 32B ffn_down, 5120 rows of 25600
  // values in 320 blocks of 143 KB): a ring plan keeps two rounds of the
  // producers' tiles instead of whole rows, with the most producer waves
  // (two to seven, plus the chain wave) that let every block be resident at
  // once (32B ffn_down: four producers, 74 KB, two blocks per CU)
  // (RLH_MV_RING=1 in the environment takes a ring plan wherever one
  // applies, with the most producers that fit the LDS: the tests run the
  // ring on small shapes and every tiled type with it). Rows whose whole-row
  // terms do not fit the LDS at all (the f32-product types past ~12288
  // values: the f32 row alone takes 1 KB per 256 values) take the ring plan
  // with the most producers that fit.
  // Launches whose input is a finished Q8 row (no norm or quantize
  // prologue: ffn_down after the SwiGLU kernel) take a ring plan too when
  // all its blocks are resident: the chain wave then adds each round as it
  // completes instead of after the other waves' first tiles (8B decode
  // 433.1 -> 434.6, 4B 503.4 -> 506.8, 0.6B 995.3 -> 997.9 tok/s); with a
  // quantize prologue (attn_output) the ring measured slower.
  uint32_t ring_np = 0;
  const uint32_t tj = tiled_any ? p.L.seg[0].w.tj : 1u;
  if (tiled_any && !fl && nm == 1 && !p.norm && R == tr && ntj >= 2) {
    const char* env = std::getenv("RLH_MV_RING");
    const bool force = (env && env[0] == '1') || !whole_fits;
    const uint32_t b = plan_blocks(p, R), s = force ? 0u : mv_resident_blocks(p, R, tr, ntj);
    if (force || (s && b > s) || !p.quant)
      for (uint32_t np = std::min<uint32_t>(7, ntj); np >= 2 && !ring_np; np--)  // np + 1 <= 8 waves (launch bound)
        if (ring_lds(p, R, np, tj, 2) <= kMaxLds &&
            (force || mv_resident(p, 64 * (np + 1), ring_lds(p, R, np, tj, 2), true) >= b))
          ring_np = np;
  }
  if (!ring_np && !whole_fits) return false;
  p.L.rows_per_blk = R;
  p.L.ring = ring_np ? 2u : 0u;
  // The ring waits end because a producer waits only for round r - ring to
  // be consumed before writing round r, and wave 0 consumes the rounds in
  // order: this needs 1 <= ring <= 3 (the LDS counters the kernel keeps), at
  // least one producer wave beside wave 0 within the 8-wave launch bound, and
  // one row tile per block (equal rounds in every block).
  if (ring_np && !(p.L.ring >= 1 && p.L.ring <= 3 && ring_np + 1 <= 8 && R == tr)) return false;
  p.L.tile_stride = ring_np ? ring_stride(p, ring_np, tj) : std::max(nsb * p.max_terms + 4, p.slot_stride);
  p.L.xf_off = plan_act_bytes(p);
  p.L.region_off = p.L.xf_off + plan_xf_bytes(p);
  p.lds = ring_np ? ring_lds(p, R, ring_np, tj, 2) : plan_lds(p, R, nm);
  const uint32_t ntiles = (R / tr) * ntj;
  // a quantize prologue is VALU work on the whole row in every block: all
  // eight waves take part even where fewer carry tiles (measured 6.3 -> 5.8
  // us for the 8B attn_output)
  p.waves = ring_np ? ring_np + 1 : (p.quant || fl ? 8u : std::max<uint32_t>(nm, std::min<uint32_t>(8, ntiles)));
  if (p.waves > 8) return false;  // k_mv's launch bound: 512 threads
  p.blocks = 0;
  for (uint32_t s = 0; s < p.L.nseg; s++) {
    p.L.seg[s].blk_begin = p.blocks;
    p.blocks += (p.L.seg[s].w.rows + R - 1) / R;
  }
  return true;
}

uint32_t mv_blocks_for(uint32_t ty, uint32_t rows, uint32_t cols) {
  MvPlan p;
  mv_plan_init(p, cols, Q8Mut{});
  DevMat w{};
  w.ty = ty;
  w.rows = rows;
  w.cols = cols;
  w.ib = item_bytes(ty);
  w.tj = tile_width(cols / 256);
  w.tr = 64 / w.tj;
  w.ntj = cols / 256 / w.tj;
  mv_plan_add(p, w, nullptr, nullptr);
  if (!mv_plan_finish(p)) return 0;
  return p.blocks;
}

void mv_launch(hipStream_t st, const MvPlan& p, uint32_t* err, hipEvent_t ev_start, hipEvent_t ev_stop) {
  MvLaunch L = p.L;
  L.err = err;
  const bool pair = p.L.nseg == 1 && p.L.seg[0].pair;
  uint32_t ty = p.L.seg[0].w.ty;
  for (uint32_t s = 1; s < p.L.nseg; s++)
    if (p.L.seg[s].w.ty != ty) ty = 0;
  const MvKernel k = pair ? mv_kernel<2>(ty) : (p.L.ring ? mv_kernel<1, true>(ty) : mv_kernel<1>(ty));
  if (ev_start || ev_stop)
    hipExtLaunchKernelGGL(k, dim3(p.blocks), dim3(64 * p.waves), p.lds, st, ev_start, ev_stop, 0, L);
  else
    hipLaunchKernelGGL(k, dim3(p.blocks), dim3(64 * p.waves), p.lds, st, L);
}

bool mv_set_max_lds(size_t bytes) {
  const uint32_t tys[] = {0,           RLH_TYPE_Q4_K, RLH_TYPE_Q6_K, RLH_TYPE_Q8_0, RLH_TYPE_Q4_0,
                          RLH_TYPE_Q5_K, RLH_TYPE_Q4_1, RLH_TYPE_Q5_0, RLH_TYPE_Q5_1, RLH_TYPE_F16,
                          RLH_TYPE_F32,  RLH_TYPE_BF16};
  for (uint32_t ty : tys) {
    const void* fns[] = {(const void*)mv_kernel<1>(ty), (const void*)mv_kernel<2>(ty), (const void*)mv_kernel<1, true>(ty)};
    for (const void* f : fns)
      if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) return false;
  }
  return true;
}

}  // namespace rlh
