// attention.hip — GQA attention over the device f32 KV cache, exact in the
// reference order (model.rs:658-711 decode, 508-545 prefill):
//   s_j  = dot_f32_avx2(q_h, K_j) * scale            (simd.rs:328-377)
//   p    = softmax_inplace(s)                        (ops.rs:398-419:
//          max, e_j = expf(s_j - max), sum = sequential sum of e_j,
//          p_j = e_j * (1/sum) when sum > 0)
//   o_d  = sequential over j of (p_j * V_j[d]) + o_d (saxpy, simd.rs:674-691)
//
// k_attn_qk (decode): one block per (KV head, 64-position tile). The
// tile's K rows are staged in LDS once; each lane owns a position and holds
// its K row in registers for its wave's query head, whose q vector is an LDS
// broadcast. K rows and q are stored slot-major (element e = 8m + l + 32k at
// 16l + 4m + k): the FMA chains, A_l = (a0+a1)+(a2+a3) and the reduction
// tree then follow the reference exactly. The kernel also applies QK-norm
// (rmsnorm_head) and NeoX RoPE to the q heads and, in the block whose tile
// holds the new position, to k, and writes K/V at pos (model.rs:642-656);
// all of it in registers.
// k_attn_qk_pre (prefill): one block per (KV head, 64-position tile, tile of
// query tokens); lanes own positions as above, q reaches every lane by DPP
// row broadcasts (below). Tiles above the causal diagonal exit at once.
// k_attn_qk_pre_p (prefill, few blocks per CU): the same work items taken
// by resident blocks in turn, the next item's K tile and q loaded while
// the current one is computed.
// k_attn_softmax: one block per (head, token): the row in LDS, max and exp
// in parallel, the sequential sum in one lane, probabilities written back
// over the scores.
// k_attn_softmax_rows (prefill rows up to 4032 positions): 4, 8 or 16
// consecutive tokens of a head per block, one wave per 1, 2 or 4 rows for the
// parallel parts and the sequential sums of all rows side by side in the
// lanes of one wave.
// k_attn_pv_dec (decode): one block per (KV head, 32-wide slice of the head
// dimension). V slices and probabilities stream through double-buffered LDS
// chunks while one lane per (head, dimension) runs its ordered saxpy chain.
// k_attn_pv_pre (prefill): one block per (KV head, tile of query tokens);
// each V chunk staged in LDS serves every token and head of the tile, and
// each thread runs eight independent chains. The 32 outputs of a half wave
// are one Q8 block of the attn_output input in both variants.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "attention.h"
#include "rlh_device.h"
#define RLH_MONO_QUAL __device__ __forceinline__
#include "monosum.h"
#include "monosum_wave.h"

namespace rlh {

namespace {

constexpr int kHd = 128;
constexpr int kPosTile = 64;    // positions per scores block
// k_attn_softmax_rows: row stride in floats (t_max rounded up to 64, plus 4)
__host__ __device__ constexpr uint32_t softmax_rows_stride(uint32_t t_max) { return ((t_max + 63) & ~63u) + 4; }
constexpr int kKStride = 132;   // floats per staged K row (permuted + 4 pad)
constexpr int kQkComb = 16;     // (token, head) combinations per scores block
constexpr int kDecChunk = 256;  // positions per LDS chunk, decode PV
constexpr int kPreChunk = 64;   // positions per LDS chunk, prefill PV
constexpr int kPreComb = 32;    // (token, head) combinations per prefill PV block
// dynamic LDS of the fused decode kernel's score rows (its V chunks take
// 66.5 KB of static LDS)
constexpr size_t kDecFusedLds = 88u * 1024u;
typedef RLH_LDS float lfloat;
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef RLH_LDS f32x4_t lf32x4;

__device__ __forceinline__ int perm(int e) { return (e & 7) * 16 + ((e >> 3) & 3) * 4 + (e >> 5); }

// rmsnorm_head + NeoX RoPE of one 128-value head held by a whole wave:
// lane l owns elements l (x0) and l + 64 (x1). Slot s of rmsnorm_core's
// 32 FMA chains takes elements s, s+32, s+64, s+96 in that order; lanes
// 0..31 build them with the partner lane l ^ 32, then the exact AVX2 tree.
// out = (x * s) * w; RoPE pair (l, l + 64) with the glibc-built cos/sin.
__device__ __forceinline__ void norm_rope_regs(float& x0, float& x1, bool norm, float w0, float w1, float c, float sn,
                                               float eps) {
  if (norm) {
    const float y0 = __shfl_xor(x0, 32), y1 = __shfl_xor(x1, 32);
    float acc = __builtin_fmaf(x0, x0, 0.0f);
    acc = __builtin_fmaf(y0, y0, acc);
    acc = __builtin_fmaf(x1, x1, acc);
    acc = __builtin_fmaf(y1, y1, acc);
    const float ss = avx2_tree32(acc);
    const float s = 1.0f / sqrtf(ss / (float)kHd + eps);
    x0 = x0 * s * w0;
    x1 = x1 * s * w1;
  }
  const float r0 = x0 * c - x1 * sn;
  const float r1 = x0 * sn + x1 * c;
  x0 = r0;
  x1 = r1;
}

// grid: (KVH * ntiles, 1); block 256.
__global__ void __launch_bounds__(256, 2) k_attn_qk(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float kt_g[kPosTile * kKStride];
  __shared__ __attribute__((aligned(16))) float qv_g[kQkComb * kHd];
  lfloat* kt = (lfloat*)kt_g;
  lfloat* qv = (lfloat*)qv_g;
  const int G = a.H / a.KVH;
  const uint32_t TT = 1u;  // one token
  const uint32_t ntiles = (a.t_max + kPosTile - 1) / kPosTile;
  const uint32_t g = blockIdx.x / ntiles, tile = blockIdx.x % ntiles;
  const uint32_t tok0 = blockIdx.y * TT;
  const uint32_t ntok = a.n_tok - tok0 < TT ? a.n_tok - tok0 : TT;
  const uint32_t pos_first = a.pos0[0] + tok0, pos_last = pos_first + ntok - 1;
  const uint32_t j0 = tile * kPosTile;
  if (j0 > pos_last) return;  // whole tile above the causal diagonal
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qd = a.H * kHd, kvd = a.KVH * kHd;
  const int ncomb = (int)ntok * G;
  const int nmine = ncomb > wave ? (ncomb - wave + 3) / 4 : 0;  // combinations wave, wave+4, ...
  const bool own_pos = pos_last < j0 + kPosTile;

  // every global load first: K tile rows (the new position's row, in
  // decode, is produced below), q heads, and the decode norm/rope operands
  // every global load first and unconditionally (indices clamped into
  // bounds, absent optional vectors replaced by a valid row whose values are
  // then not used): a load under a branch gets a wait for every load before
  // it. K tile rows (the new position's row, in decode, is produced below),
  // q heads, and the decode norm/rope operands.
  float4 kr[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t c = (uint32_t)(tid + 256 * i), jl = c >> 5, f4 = c & 31, j = min(j0 + jl, pos_last);
    kr[i] = ld_gf4(a.kcache + (size_t)j * kvd + g * kHd + 4 * f4);
  }
  const bool hb = a.bq != nullptr;
  const float* bq = hb ? a.bq : a.q;
  float q0[4], q1[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int cb = min(wave + 4 * i, ncomb - 1), tt = cb / G, h = g * G + cb % G;
    const float* src = a.q + (size_t)(tok0 + tt) * qd + h * kHd;
    q0[i] = ld_gf(src + lane);
    q1[i] = ld_gf(src + lane + 64);
    {
      const float b0 = ld_gf(bq + h * kHd + lane), b1 = ld_gf(bq + h * kHd + lane + 64);
      if (hb) {
        q0[i] = q0[i] + b0;
        q1[i] = q1[i] + b1;
      }
    }
  }
  {
    const float c = ld_gf(a.rope_cs + (size_t)pos_first * kHd + 2 * lane);
    const float sn = ld_gf(a.rope_cs + (size_t)pos_first * kHd + 2 * lane + 1);
    const bool nq = a.qn != nullptr;
    const float* qn = nq ? a.qn : a.rope_cs;
    const float w0 = ld_gf(qn + lane), w1 = ld_gf(qn + lane + 64);
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (i < nmine) norm_rope_regs(q0[i], q1[i], nq, w0, w1, c, sn, a.eps);
    if (own_pos && wave == 3) {  // k and v of the new position (model.rs:642-656)
      const uint32_t pos = pos_last;
      const bool hbk = a.bk != nullptr, hbv = a.bv != nullptr, nk = a.kn != nullptr;
      const float* bk = hbk ? a.bk : a.k;
      const float* bv = hbv ? a.bv : a.v;
      const float* kn = nk ? a.kn : a.rope_cs;
      float k0 = ld_gf(a.k + g * kHd + lane), k1 = ld_gf(a.k + g * kHd + lane + 64);
      float v0 = ld_gf(a.v + g * kHd + lane), v1 = ld_gf(a.v + g * kHd + lane + 64);
      const float bk0 = ld_gf(bk + g * kHd + lane), bk1 = ld_gf(bk + g * kHd + lane + 64);
      const float bv0 = ld_gf(bv + g * kHd + lane), bv1 = ld_gf(bv + g * kHd + lane + 64);
      const float u0 = ld_gf(kn + lane), u1 = ld_gf(kn + lane + 64);
      if (hbk) {
        k0 = k0 + bk0;
        k1 = k1 + bk1;
      }
      if (hbv) {
        v0 = v0 + bv0;
        v1 = v1 + bv1;
      }
      norm_rope_regs(k0, k1, nk, u0, u1, c, sn, a.eps);
      float* kd = a.kcache + (size_t)pos * kvd + g * kHd;
      kd[lane] = k0;
      kd[lane + 64] = k1;
      float* vd = a.vcache + (size_t)pos * kvd + g * kHd;
      vd[lane] = v0;
      vd[lane + 64] = v1;
      lfloat* row = kt + (pos - j0) * kKStride;
      row[perm(lane)] = k0;
      row[perm(lane + 64)] = k1;
    }
  }
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t c = (uint32_t)(tid + 256 * i), jl = c >> 5, f4 = c & 31, j = j0 + jl;
    if (j < pos_last) {
      lfloat* row = kt + jl * kKStride;
      row[perm(4 * f4)] = kr[i].x;
      row[perm(4 * f4 + 1)] = kr[i].y;
      row[perm(4 * f4 + 2)] = kr[i].z;
      row[perm(4 * f4 + 3)] = kr[i].w;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (i < nmine) {
      const int cb = wave + 4 * i;
      qv[cb * kHd + perm(lane)] = q0[i];
      qv[cb * kHd + perm(lane + 64)] = q1[i];
    }
  }
  __syncthreads();
  if (nmine == 0) return;
  // lane = position: the K row sits in registers for all the wave's
  // combinations; q is read from LDS as a broadcast
  const uint32_t j = j0 + (uint32_t)lane;
  const lf32x4* krow = (const lf32x4*)(kt + lane * kKStride);
  f32x4_t kreg[32];
#pragma unroll
  for (int i = 0; i < 32; i++) kreg[i] = krow[i];
#pragma unroll 1
  for (int c = 0; c < nmine; c++) {
    const int cb = wave + 4 * c, tt = cb / G, h = g * G + cb % G;
    const lf32x4* qc = (const lf32x4*)(qv + cb * kHd);
    float A[8];
#pragma unroll
    for (int l = 0; l < 8; l++) {
      float acc[4];
#pragma unroll
      for (int m = 0; m < 4; m++) {
        const f32x4_t x = qc[l * 4 + m];
        const f32x4_t y = kreg[l * 4 + m];
        float s = __builtin_fmaf(x.x, y.x, 0.0f);
        s = __builtin_fmaf(x.y, y.y, s);
        s = __builtin_fmaf(x.z, y.z, s);
        acc[m] = __builtin_fmaf(x.w, y.w, s);
      }
      A[l] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    if (j <= pos_first + (uint32_t)tt) {
      const float d = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
      a.scores[((size_t)(tok0 + tt) * a.H + h) * a.t_stride + j] = d * a.scale;
    }
  }
}

// Prefill scores (q already normed and roped): k_attn_qk_pre (a block per
// work item) or k_attn_qk_pre_p (persistent), below; a work item is (KV
// head, 64-position tile, tile of combinations / G query tokens).
constexpr int kPreQkComb = 64;  // k_attn_qk_pre: combinations per block (a multiple of 8)
constexpr int kPreQkItem = 32;  // k_attn_qk_pre_p: combinations per work item (a multiple of 8)
// k_attn_qk_pre_p runs when k_attn_qk_pre's blocks would fill at most this
// many rounds of the resident blocks: it loads an item's K tile and q while
// the previous item is computed, but each item waits for the previous one's
// score stores to drain (one memory counter covers both), which costs more
// than it saves once a block has many items (8B 512-token chunk, 2.25
// rounds: 58 -> 43 us; 32B 4096-token chunks, 12-60 rounds: 468 -> 646 us)
constexpr uint32_t kQkPersistRounds = 6;
// blocks of k_attn_qk_pre_p the GPU holds at once (attn_init)
uint32_t g_qk_pre_resident = 0;

// acc[i] = fma(q_e, k_i, acc[i]) for the 8 elements e = 16m + R0 + i, whose
// q_e is lane R0 + i of every row of 16 lanes in qm (v_fmac_f32 takes it by
// DPP row_newbcast; one instruction per FMA, no broadcast copies). The
// leading s_nop covers the DPP read-after-VALU-write hazard on qm.
template <int R0>
__device__ __forceinline__ void fmac8_bcast(float (&acc)[32], int s0, float qm, const f32x4_t& k0, const f32x4_t& k1) {
  asm("s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %8, %9 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %8, %10 row_newbcast:%18 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %8, %11 row_newbcast:%19 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %8, %12 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %4, %8, %13 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %5, %8, %14 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %6, %8, %15 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %7, %8, %16 row_newbcast:%24 row_mask:0xf bank_mask:0xf"
      : "+v"(acc[s0]), "+v"(acc[s0 + 1]), "+v"(acc[s0 + 2]), "+v"(acc[s0 + 3]), "+v"(acc[s0 + 4]), "+v"(acc[s0 + 5]),
        "+v"(acc[s0 + 6]), "+v"(acc[s0 + 7])
      : "v"(qm), "v"(k0.x), "v"(k0.y), "v"(k0.z), "v"(k0.w), "v"(k1.x), "v"(k1.y), "v"(k1.z), "v"(k1.w), "i"(R0),
        "i"(R0 + 1), "i"(R0 + 2), "i"(R0 + 3), "i"(R0 + 4), "i"(R0 + 5), "i"(R0 + 6), "i"(R0 + 7));
}
// step K of the 32 slot chains (elements s + 32K): slots 0..15 take qm[2K],
// slots 16..31 qm[2K + 1]
template <int K>
__device__ __forceinline__ void qk_step(float (&acc)[32], const float (&qm)[8], const f32x4_t (&kreg)[32]) {
  fmac8_bcast<0>(acc, 0, qm[2 * K], kreg[8 * K], kreg[8 * K + 1]);
  fmac8_bcast<8>(acc, 8, qm[2 * K], kreg[8 * K + 2], kreg[8 * K + 3]);
  fmac8_bcast<0>(acc, 16, qm[2 * K + 1], kreg[8 * K + 4], kreg[8 * K + 5]);
  fmac8_bcast<8>(acc, 24, qm[2 * K + 1], kreg[8 * K + 6], kreg[8 * K + 7]);
}

// Work item of the persistent prefill scores kernel: KV head g, token tile y
// (tokens y TP .. y TP + TP - 1) and a 64-position tile at or below the
// tile's causal diagonal; per KV head the items run y-major. count(y) is
// the number of position tiles token tile y sees.
struct QkItem {
  uint32_t g, tile, tok0, ntok;
};
__host__ __device__ inline uint32_t qk_tiles_seen(uint32_t p0, uint32_t n_tok, uint32_t TP, uint32_t y) {
  const uint32_t last = p0 + (n_tok < (y + 1) * TP ? n_tok : (y + 1) * TP) - 1;
  return last / kPosTile + 1;
}
__host__ __device__ inline uint32_t qk_items_per_head(uint32_t p0, uint32_t n_tok, uint32_t TP) {
  uint32_t n = 0;
  for (uint32_t y = 0; y * TP < n_tok; y++) n += qk_tiles_seen(p0, n_tok, TP, y);
  return n;
}
__device__ inline QkItem qk_item(uint32_t it, uint32_t per_g, uint32_t p0, uint32_t n_tok, uint32_t TP) {
  QkItem q;
  q.g = it / per_g;
  uint32_t r = it % per_g, y = 0;
  for (;; y++) {  // r < per_g: some token tile holds it
    const uint32_t c = qk_tiles_seen(p0, n_tok, TP, y);
    if (r < c) break;
    r -= c;
  }
  q.tile = r;
  q.tok0 = y * TP;
  q.ntok = n_tok - q.tok0 < TP ? n_tok - q.tok0 : TP;
  return q;
}

// Prefill scores (q already normed and roped): one block per (KV head,
// 64-position tile, tile of kPreQkComb / G query tokens). The K tile is
// staged in LDS once and each lane (= position) keeps its K row in
// registers. The wave walks its (token, head) combinations with q held in
// every row of 16 lanes (lane r of a row holds elements 16m + r in qm[m])
// and broadcast to the row by DPP (row_newbcast), so no q element passes
// through LDS; the next combination's q is loaded while the current one is
// computed. Slot s (0..31) of dot_f32_avx2 is the FMA chain over elements s,
// s+32, s+64, s+96, A_l = (slot l + slot l+8) + (slot l+16 + slot l+24),
// then the AVX2 tree (simd.rs:328-377).
// grid: (KVH * ntiles, ceil(n_tok / TP)), TP = kPreQkComb / G; block 256.
__global__ void __launch_bounds__(256, 2) k_attn_qk_pre(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float kt_g[kPosTile * kKStride];
  __shared__ __attribute__((aligned(16))) float qv_g[kPreQkComb * kHd];
  lfloat* kt = (lfloat*)kt_g;
  lfloat* qv = (lfloat*)qv_g;
  const uint32_t G = (uint32_t)(a.H / a.KVH), TP = (uint32_t)kPreQkComb / G;
  const uint32_t ntiles = (a.t_max + kPosTile - 1) / kPosTile;
  const uint32_t g = blockIdx.x / ntiles, tile = blockIdx.x % ntiles;
  const uint32_t tok0 = blockIdx.y * TP;
  const uint32_t ntok = a.n_tok - tok0 < TP ? a.n_tok - tok0 : TP;
  const uint32_t pos_first = a.pos0[0] + tok0, pos_last = pos_first + ntok - 1;
  const uint32_t j0 = tile * kPosTile;
  if (j0 > pos_last) return;  // whole tile above the causal diagonal
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t qd = (uint32_t)a.H * kHd, kvd = (uint32_t)a.KVH * kHd;
  // K tile rows in natural element order (rows past pos_last repeat it)
  float4 kr[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t c = tid + 256u * i, jl = c >> 5, f4 = c & 31, j = min(j0 + jl, pos_last);
    kr[i] = ld_gf4(a.kcache + (size_t)j * kvd + g * kHd + 4 * f4);
  }
  // combinations of tokens that see at least one position of the tile;
  // the wave's first q is loaded with the K tile
  const uint32_t tt0 = j0 > pos_first ? j0 - pos_first : 0u;
  const uint32_t ncomb = ntok * G;
  // the block's q vectors are staged in LDS with the K tile, element
  // 16 m + r of a combination at r * 8 + m, so that lane r of every row of
  // 16 lanes reads its eight elements in two 16-byte reads
  constexpr int kQv = kPreQkComb / 8;  // float4s of q per thread (32 per combination)
  float4 qr[kQv];
#pragma unroll
  for (int i = 0; i < kQv; i++) {
    const uint32_t ci = tid + 256u * i, cb = min(ci >> 5, ncomb - 1), f4 = ci & 31;
    qr[i] = ld_gf4(a.q + (size_t)(tok0 + cb / G) * qd + (g * G + cb % G) * kHd + 4 * f4);
  }
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t ci = tid + 256u * i, jl = ci >> 5, f4 = ci & 31;
    *(lf32x4*)(kt + jl * kKStride + 4 * f4) = f32x4_t{kr[i].x, kr[i].y, kr[i].z, kr[i].w};
  }
#pragma unroll
  for (int i = 0; i < kQv; i++) {
    const uint32_t ci = tid + 256u * i, cb = ci >> 5, f4 = ci & 31;  // cb < kPreQkComb
    lfloat* qd0 = qv + cb * kHd + 4 * (f4 & 3) * 8 + (f4 >> 2);
    qd0[0] = qr[i].x;
    qd0[8] = qr[i].y;
    qd0[16] = qr[i].z;
    qd0[24] = qr[i].w;
  }
  auto q_load = [&](float (&qm)[8], uint32_t c) {
    const lf32x4* qp = (const lf32x4*)(qv + min(c, ncomb - 1) * kHd + (lane & 15) * 8);
    const f32x4_t u0 = qp[0], u1 = qp[1];
    qm[0] = u0.x, qm[1] = u0.y, qm[2] = u0.z, qm[3] = u0.w;
    qm[4] = u1.x, qm[5] = u1.y, qm[6] = u1.z, qm[7] = u1.w;
  };
  float qa[8], qb[8];
  uint32_t c = tt0 * G + wave;
  __syncthreads();
  q_load(qa, c);
  const uint32_t j = j0 + lane;
  f32x4_t kreg[32];
#pragma unroll
  for (int i = 0; i < 32; i++) kreg[i] = *(const lf32x4*)(kt + lane * kKStride + 4 * i);
  auto one = [&](const float (&qm)[8], uint32_t cc) {
    const uint32_t tt = cc / G, h = g * G + cc % G;
    float acc[32];
#pragma unroll
    for (int s = 0; s < 32; s++) acc[s] = 0.0f;  // fma(q, k, +0) starts each chain, as the reference
    qk_step<0>(acc, qm, kreg);
    qk_step<1>(acc, qm, kreg);
    qk_step<2>(acc, qm, kreg);
    qk_step<3>(acc, qm, kreg);
    float A[8];
#pragma unroll
    for (int l = 0; l < 8; l++) A[l] = (acc[l] + acc[l + 8]) + (acc[l + 16] + acc[l + 24]);
    const float d = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
    if (j <= pos_first + tt) a.scores[((size_t)(tok0 + tt) * a.H + h) * a.t_stride + j] = d * a.scale;
  };
#pragma unroll 1
  for (; c < ncomb; c += 8) {
    q_load(qb, c + 4);
    one(qa, c);
    if (c + 4 >= ncomb) break;
    q_load(qa, c + 8);
    one(qb, c + 4);
  }
}

// grid: the resident blocks (at most the items); block 256. Block b takes
// items b, b + gridDim.x, ... (exits are uniform, no waits between blocks).
// Per item the K tile is staged in LDS and each lane (= position) keeps its
// K row in registers; the item's q vectors sit in one of two LDS buffers in
// their natural element order, copied there by DMA. While an item is
// computed, the next item's K tile is loaded into registers and its q
// vectors are copied into the other buffer, so the loads' latency is paid
// once per block instead of once per item; the combination loop issues no
// global loads (nothing it waits for queues behind the next item's). Lane
// r of every row of 16 lanes reads elements 16 m + r of q (conflict-free
// 4-byte reads) into qm[m], which the FMAs take by DPP row broadcasts
// (fmac8_bcast). Slot s (0..31) of dot_f32_avx2 is the FMA chain over
// elements s, s+32, s+64, s+96, A_l = (slot l + slot l+8) + (slot l+16 +
// slot l+24), then the AVX2 tree (simd.rs:328-377).
__global__ void __launch_bounds__(256, 2) k_attn_qk_pre_p(AttnArgs a, uint32_t per_g) {
  __shared__ __attribute__((aligned(16))) float kt_g[kPosTile * kKStride];
  __shared__ __attribute__((aligned(16))) float qv_g[2][kPreQkItem * kHd];
  lfloat* kt = (lfloat*)kt_g;
  const uint32_t G = (uint32_t)(a.H / a.KVH), TP = (uint32_t)kPreQkItem / G;
  const uint32_t p0h = a.t_max - a.n_tok;  // the chunk's first position (the host's view of pos0)
  const uint32_t n_items = (uint32_t)a.KVH * per_g;
  uint32_t it = blockIdx.x;
  if (it >= n_items) return;  // whole block, before any barrier
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t qd = (uint32_t)a.H * kHd, kvd = (uint32_t)a.KVH * kHd;
  const uint32_t p0 = a.pos0[0];
  // an item's K tile rows in natural element order (rows past its last
  // token's position repeat that row)
  auto load_k = [&](float4 (&kr)[8], const QkItem& q) {
    const uint32_t pos_last = p0 + q.tok0 + q.ntok - 1, j0 = q.tile * kPosTile;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t c = tid + 256u * i, jl = c >> 5, f4 = c & 31, j = min(j0 + jl, pos_last);
      kr[i] = ld_gf4(a.kcache + (size_t)j * kvd + q.g * kHd + 4 * f4);
    }
  };
  // an item's q vectors into buffer b by DMA: one 1 KB copy per wave and
  // step holds two combinations (lanes 0..31 and 32..63, 16 bytes each);
  // combinations past the last token repeat the last one
  auto dma_q = [&](uint32_t b, const QkItem& q) {
    const uint32_t ncomb = q.ntok * G;
#pragma unroll
    for (uint32_t k = 0; k < (uint32_t)kPreQkItem / 8; k++) {
      const uint32_t pair = wave + 4 * k, cb = min(2 * pair + lane / 32, ncomb - 1);
      __builtin_amdgcn_global_load_lds(
          (const RLH_GLOBAL void*)(a.q + (size_t)(q.tok0 + cb / G) * qd + (q.g * G + cb % G) * kHd + 4 * (lane % 32)),
          (RLH_LDS void*)((lfloat*)qv_g[b] + 2 * pair * kHd), 16, 0, 0);
    }
  };
  QkItem cur = qk_item(it, per_g, p0h, a.n_tok, TP);
  float4 kr[8];
  load_k(kr, cur);
  dma_q(0, cur);
  for (uint32_t n = 0;; n++) {
    wait_vmcnt<0>();  // this wave's K rows and q copies of the item have landed
    __syncthreads();  // ... everyone's; every wave is done with the previous kt
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t ci = tid + 256u * i, jl = ci >> 5, f4 = ci & 31;
      *(lf32x4*)(kt + jl * kKStride + 4 * f4) = f32x4_t{kr[i].x, kr[i].y, kr[i].z, kr[i].w};
    }
    __syncthreads();
    f32x4_t kreg[32];
#pragma unroll
    for (int i = 0; i < 32; i++) kreg[i] = *(const lf32x4*)(kt + lane * kKStride + 4 * i);
    const lfloat* qv = (const lfloat*)qv_g[n & 1];
    const uint32_t nit = it + gridDim.x;
    const bool more = nit < n_items;
    QkItem nxt = cur;
    if (more) {  // uniform: the next item's K tile and q vectors in flight
      nxt = qk_item(nit, per_g, p0h, a.n_tok, TP);
      load_k(kr, nxt);
      dma_q((n + 1) & 1, nxt);  // that buffer's last reader was the item before this one
    }
    const uint32_t j0 = cur.tile * kPosTile, pos_first = p0 + cur.tok0, ncomb = cur.ntok * G;
    const uint32_t j = j0 + lane;
    auto q_load = [&](float (&qm)[8], uint32_t c) {
      const lfloat* qp = qv + min(c, ncomb - 1) * kHd + (lane & 15);
#pragma unroll
      for (int m = 0; m < 8; m++) qm[m] = qp[16 * m];
    };
    auto one = [&](const float (&qm)[8], uint32_t cc) {
      const uint32_t tt = cc / G, h = cur.g * G + cc % G;
      float acc[32];
#pragma unroll
      for (int s = 0; s < 32; s++) acc[s] = 0.0f;  // fma(q, k, +0) starts each chain, as the reference
      qk_step<0>(acc, qm, kreg);
      qk_step<1>(acc, qm, kreg);
      qk_step<2>(acc, qm, kreg);
      qk_step<3>(acc, qm, kreg);
      float A[8];
#pragma unroll
      for (int l = 0; l < 8; l++) A[l] = (acc[l] + acc[l + 8]) + (acc[l + 16] + acc[l + 24]);
      const float d = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
      if (j <= pos_first + tt) a.scores[((size_t)(cur.tok0 + tt) * a.H + h) * a.t_stride + j] = d * a.scale;
    };
    // tokens before tt0 see no position of the tile
    uint32_t c = (j0 > pos_first ? j0 - pos_first : 0u) * G + wave;
    float qa[8], qb[8];
    q_load(qa, c);
#pragma unroll 1
    for (; c < ncomb; c += 8) {
      q_load(qb, c + 4);
      one(qa, c);
      if (c + 4 >= ncomb) break;
      q_load(qa, c + 8);
      one(qb, c + 4);
    }
    if (!more) break;
    it = nit;
    cur = nxt;
  }
}

// One wave walks nr runs of K terms in order (run r: e[r K, min(t, (r + 1) K)),
// its pair A0[r], A1[r] made at binade U[r]): a DPP scan of 64 runs' pairs
// at a time from the exact state; the first run whose binade was mispredicted
// or whose increments leave the binade is added with f32 adds from its exact
// start and the scan resumes after it. Every lane returns the sum. Each
// pass either ends its 64 runs or moves l0 past the replayed run, so the
// walk ends.
__device__ float wave_walk_runs(const lfloat* e, uint32_t t, uint32_t K, uint32_t nr, const RLH_LDS uint32_t* A0,
                                const RLH_LDS uint32_t* A1, const RLH_LDS int* U) {
  const uint32_t lane = threadIdx.x & 63;
  int u = -149;  // the state of the sum 0
  uint32_t N = 0;
  for (uint32_t gb = 0; gb < nr; gb += 64) {
    const uint32_t r = gb + lane;
    const bool live = r < nr;
    const uint32_t rc = live ? r : nr - 1;
    const MonoFn fr{A0[rc], A1[rc]};
    const int urr = U[rc];
    uint32_t l0 = 0;
    for (;;) {
      const bool mine = live && lane >= l0;
      const bool hit = urr == u;
      const MonoFn g = mine && hit ? fr : mono_identity();
      const MonoFn incl = wave_scan_fn(g);
      const uint32_t nl = N + mono_apply(wave_excl_fn(incl), N);
      const bool stop = mine && (!hit || mono_inc_leaves(nl, mono_apply(fr, nl)));
      const uint64_t mask = __ballot(stop);
      if (mask == 0) {
        N += mono_apply(MonoFn{readlane_u32(incl.a0, 63), readlane_u32(incl.a1, 63)}, N);
        break;
      }
      const uint32_t lc = (uint32_t)__builtin_ctzll(mask);
      const uint32_t k0 = (gb + lc) * K;
      const float sv = seq_sum_lds(e + k0, min(t, k0 + K) - k0, mono_value(u, readlane_u32(nl, (int)lc)));
      mono_state(sv, &u, &N);
      u = __builtin_amdgcn_readfirstlane(u);
      N = (uint32_t)__builtin_amdgcn_readfirstlane((int)N);
      if (lc == 63) break;
      l0 = lc + 1;
    }
  }
  return mono_value(u, N);
}

// grid: (H, n_tok); block kSoftmaxWalkThreads (decode) or 256 (prefill);
// dynamic LDS: one row of t_max floats.
// The softmax sum ((0 + e_0) + e_1) + ... of the t non-negative terms in LDS
// (16-byte aligned), bit for bit as the sequential loop rounds it
// (ops.rs:408-412), by a block of kSoftmaxWalkThreads threads. Thread r takes run r (K
// consecutive terms, K a multiple of 4), predicts the binade of the running
// sum at the run's start from an approximate f32 prefix and forms the run's
// increment pair there (monosum.h). Wave 0 then takes the runs 64 at a
// time: one scan of their pairs gives every run's exact start inside the
// current binade; the first run whose prediction misses that binade or
// whose increments leave it is added with f32 adds from its exact start,
// and the scan resumes after it (a few runs per row: about one per doubling
// of the sum). The prediction only chooses between the two paths. Rows with
// a NaN or infinite term take the plain loop, and so do short rows. Only
// the decode launch (one row per head) uses it: in prefill the blocks'
// chains overlap each other, and the walk's LDS and extra work per term
// made the 32B 4096-token prefill slower (1931 -> 1957 ms); decode at 4.1 K
// positions gains (96.1 -> 97.6 tok/s). Every thread gets the sum.
constexpr uint32_t kSoftmaxWalkMin = 1024;  // shorter rows: the plain chain
constexpr uint32_t kSoftmaxWalkThreads = 1024;  // the decode launch's block: one run per thread
struct SoftmaxSumLds {
  uint32_t a0[kSoftmaxWalkThreads], a1[kSoftmaxWalkThreads];
  int u[kSoftmaxWalkThreads];
  float wsum[kSoftmaxWalkThreads / 64];
  float out;
};
// shift (a test knob, 0 in use): 1 / 2 move every run's predicted binade
// one up / down, 3 every third run's one up (scans that pass runs, then
// stop); a shifted prediction never equals the exact state's binade, so
// each such run is replayed from its exact start, and the sum must not
// change.
__device__ float block_softmax_sum(const lfloat* e, uint32_t t, SoftmaxSumLds* sl, int shift) {
  RLH_LDS SoftmaxSumLds* L = (RLH_LDS SoftmaxSumLds*)sl;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (t < kSoftmaxWalkMin) {
    if (tid == 0) L->out = seq_sum_lds(e, t);
    __syncthreads();
    return L->out;
  }
  const uint32_t K = (((t + kSoftmaxWalkThreads - 1) / kSoftmaxWalkThreads) + 3) & ~3u;
  const uint32_t j0 = min(tid * K, t), j1 = min(j0 + K, t);
  float a = 0.0f;
  bool bad = false;
  for (uint32_t j = j0; j < j1; j++) {
    const float v = e[j];
    a += v;
    bad |= !(v < __int_as_float(0x7f800000));
  }
  float inc = a;  // the approximate prefix: any order serves
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float v = __shfl_up(inc, o);
    if ((int)lane >= o) inc += v;
  }
  if (lane == 63) L->wsum[wave] = inc;
  if (__syncthreads_or(bad)) {
    if (tid == 0) L->out = seq_sum_lds(e, t);
    __syncthreads();
    return L->out;
  }
  float base = 0.0f;
  for (uint32_t w = 0; w < wave; w++) base += L->wsum[w];
  int ur = mono_binade(base + inc - a);
  if (shift) ur += shift == 1 ? 1 : (shift == 2 ? -1 : (tid % 3 == 0 ? 1 : 0));
  const MonoFn f = mono_run_pair(e + j0, j1 - j0, ur);
  L->a0[tid] = f.a0;
  L->a1[tid] = f.a1;
  L->u[tid] = ur;
  __syncthreads();
  if (wave == 0) {
    const float sum = wave_walk_runs(e, t, K, (t + K - 1) / K, L->a0, L->a1, L->u);
    if (lane == 0) L->out = sum;
  }
  __syncthreads();
  return L->out;
}

// WALK: the decode launch (block of kSoftmaxWalkThreads), whose sum is
// block_softmax_sum's; the prefill launch takes 256 threads per row.
template <bool WALK>
__global__ void __launch_bounds__(WALK ? kSoftmaxWalkThreads : 256) k_attn_softmax(AttnArgs a) {
  constexpr uint32_t NT = WALK ? kSoftmaxWalkThreads : 256;
  extern __shared__ __attribute__((aligned(16))) float lds_generic[];
  __shared__ float red[NT / 64];
  __shared__ uint64_t tab_g[32];
  __shared__ float s_inv;
  __shared__ int s_on;
  lu64* tab = (lu64*)tab_g;
  lfloat* e = (lfloat*)lds_generic;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t t = a.pos0[0] + blockIdx.y + 1;
  float* row = a.scores + ((size_t)blockIdx.y * a.H + blockIdx.x) * a.t_stride;
  // max: the reference keeps x[0] and takes every later v > max, so a NaN
  // first score gives NaN and later NaNs are skipped, as fmaxf does
  // the row in batches of eight loads per thread in flight together (a
  // load per iteration would make each LDS store wait for its own load in
  // turn); a -inf stand-in past t leaves the max unchanged
  float mx = -__int_as_float(0x7f800000);
  for (uint32_t b = 0; b < t; b += NT * 8) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t j = b + tid + NT * k;
      v[k] = j < t ? ld_gf(row + j) : -__int_as_float(0x7f800000);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t j = b + tid + NT * k;
      if (j < t) e[j] = v[k];
      mx = fmaxf(mx, v[k]);
    }
  }
  exp_tab_to_lds(tab);  // after the row loads: its store waits for its load
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
#pragma unroll
  for (uint32_t w = 0; w < NT / 64; w++) mx = fmaxf(mx, red[w]);
  const float x0 = e[0];
  if (x0 != x0) mx = x0;
  // four terms per thread and step (16-byte LDS accesses: the row and its
  // LDS stride are 16-byte aligned and cover t rounded up to 4); words past
  // t keep their contents
  const uint32_t nq = (t + 3) / 4;
  for (uint32_t q = tid; q < nq; q += NT) {
    const uint32_t j = 4 * q;
    const f32x4_t x = *(const lf32x4*)(e + j);
    const float y0 = expf_glibc_t(x.x - mx, tab), y1 = expf_glibc_t(x.y - mx, tab);
    const float y2 = expf_glibc_t(x.z - mx, tab), y3 = expf_glibc_t(x.w - mx, tab);
    *(lf32x4*)(e + j) = f32x4_t{y0, j + 1 < t ? y1 : x.y, j + 2 < t ? y2 : x.z, j + 3 < t ? y3 : x.w};
  }
  __syncthreads();
  bool on;
  float inv;
  if constexpr (WALK) {
    __shared__ SoftmaxSumLds ssl;  // only in the decode instantiation
    const float sum = block_softmax_sum(e, t, &ssl, a.walk_shift);  // the sequential sum of softmax_inplace
    on = sum > 0.0f;
    inv = 1.0f / sum;
  } else {
    if (tid == 0) {  // the sequential sum of softmax_inplace
      const float sum = seq_sum_lds(e, t);
      s_on = sum > 0.0f;
      s_inv = 1.0f / sum;
    }
    __syncthreads();
    on = s_on;
    inv = s_inv;
  }
  for (uint32_t q = tid; q < nq; q += NT) {
    const uint32_t j = 4 * q;
    const f32x4_t v = *(const lf32x4*)(e + j);
    row[j] = on ? v.x * inv : v.x;
    if (j + 1 < t) row[j + 1] = on ? v.y * inv : v.y;
    if (j + 2 < t) row[j + 2] = on ? v.z * inv : v.z;
    if (j + 3 < t) row[j + 3] = on ? v.w * inv : v.w;
  }
}

// grid: (H, ceil(n_tok / (4 RW))); block 256; dynamic LDS: 4 RW rows of
// softmax_rows_stride(t_max) floats. The prefill softmax of 4 RW consecutive
// tokens of one head, with k_attn_softmax<false>'s arithmetic: wave w loads
// rows w RW .. w RW + RW - 1 (max, exponentials) and scales them; the
// sequential sums of all rows run side by side in the first 4 RW lanes of
// wave 0, one dependent add per term for all rows at once. Every row is
// padded with +0 terms to T, the block's longest row rounded up to 4: the
// sum starts at +0 and its terms are never negative, so a +0 term leaves it
// unchanged. The row stride is 4 words above a multiple of 64, so the
// lanes' 16-byte reads fall in distinct banks. A row past the last token has
// t = 0: no loads, no stores, and every wave reaches the block's barriers.
template <int RW>
__global__ void __launch_bounds__(256) k_attn_softmax_rows(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds_generic[];
  __shared__ uint64_t tab_g[32];
  __shared__ float s_inv[4 * RW];
  __shared__ int s_on[4 * RW];
  lu64* tab = (lu64*)tab_g;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t S = softmax_rows_stride(a.t_max), p0 = a.pos0[0], y0 = blockIdx.y * (4 * RW);
  const uint32_t T = (p0 + min(y0 + 4 * RW, a.n_tok) + 3) & ~3u;
  constexpr int KL = 16 / RW;  // loads per lane and row in flight together
  uint32_t t[RW];
  float mx[RW];
  const float* rows[RW];
#pragma unroll
  for (int i = 0; i < RW; i++) {
    const uint32_t y = y0 + wave * RW + i;
    t[i] = y < a.n_tok ? p0 + y + 1 : 0;
    rows[i] = a.scores + ((size_t)min(y, a.n_tok - 1) * a.H + blockIdx.x) * a.t_stride;
    mx[i] = -__int_as_float(0x7f800000);
  }
  // the wave's longest row is its last valid one; a -inf stand-in past a
  // row's end leaves its max unchanged (fmaxf never returns NaN from a
  // non-NaN max, so the max is never NaN)
  const uint32_t tw = t[0] ? p0 + min(y0 + wave * RW + RW, a.n_tok) : 0;
  for (uint32_t b = 0; b < tw; b += 64 * KL) {
    float v[RW][KL];
#pragma unroll
    for (int i = 0; i < RW; i++)
#pragma unroll
      for (int k = 0; k < KL; k++) {
        const uint32_t j = b + lane + 64 * k;
        v[i][k] = j < t[i] ? ld_gf(rows[i] + j) : -__int_as_float(0x7f800000);
      }
#pragma unroll
    for (int i = 0; i < RW; i++) {
      lfloat* e = (lfloat*)lds_generic + (wave * RW + i) * S;
#pragma unroll
      for (int k = 0; k < KL; k++) {
        const uint32_t j = b + lane + 64 * k;
        if (j < t[i]) e[j] = v[i][k];
        mx[i] = fmaxf(mx[i], v[i][k]);
      }
    }
  }
  exp_tab_to_lds(tab);
#pragma unroll
  for (int i = 0; i < RW; i++) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], m));
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < RW; i++) {
    lfloat* e = (lfloat*)lds_generic + (wave * RW + i) * S;
    float m = mx[i];
    if (t[i]) {  // a NaN first score gives NaN (the reference's max loop)
      const float x0 = e[0];
      if (x0 != x0) m = x0;
    }
    // four terms per lane (16-byte LDS accesses); the words past t hold
    // nothing loaded, and their exponentials are replaced by +0
    for (uint32_t j = 4 * lane; j < T; j += 256) {
      const f32x4_t x = *(const lf32x4*)(e + j);
      const float y0 = expf_glibc_t(x.x - m, tab), y1 = expf_glibc_t(x.y - m, tab);
      const float y2 = expf_glibc_t(x.z - m, tab), y3 = expf_glibc_t(x.w - m, tab);
      *(lf32x4*)(e + j) = f32x4_t{j < t[i] ? y0 : 0.0f, j + 1 < t[i] ? y1 : 0.0f, j + 2 < t[i] ? y2 : 0.0f,
                                  j + 3 < t[i] ? y3 : 0.0f};
    }
  }
  __syncthreads();
  if (tid < 4 * RW) {  // the sequential sums of softmax_inplace (ops.rs:408-412)
    const float sum = seq_sum_lds((lfloat*)lds_generic + tid * S, T);
    s_on[tid] = sum > 0.0f;
    s_inv[tid] = 1.0f / sum;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < RW; i++) {
    const uint32_t r = wave * RW + i;
    const lfloat* e = (const lfloat*)lds_generic + r * S;
    float* row = (float*)rows[i];
    const bool on = s_on[r];
    const float inv = s_inv[r];
    for (uint32_t j = lane; j < t[i]; j += 64) {
      const float v = e[j];
      row[j] = on ? v * inv : v;
    }
  }
}

// grid: (KVH, 4 slices of 32 dimensions); block 512. Lanes tid < G*32 run
// the chains of (head tid/32, dimension d0 + tid%32); every thread loads.
__global__ void __launch_bounds__(512) k_attn_pv_dec(AttnArgs a) {
  constexpr int CS = kDecChunk + 4;
  __shared__ __attribute__((aligned(16))) float vs_g[2 * 32 * CS];
  __shared__ __attribute__((aligned(16))) float ps_g[2 * kAttnMaxGroup * CS];
  lfloat* vs = (lfloat*)vs_g;
  lfloat* ps = (lfloat*)ps_g;
  const int G = a.H / a.KVH;
  const uint32_t g = blockIdx.x, d0 = blockIdx.y * 32;
  const int tid = threadIdx.x, hl = tid >> 5, dd = tid & 31;
  const int kvd = a.KVH * kHd;
  const uint32_t t = a.pos0[0] + 1;
  const uint32_t nch = (t + kDecChunk - 1) / kDecChunk;
  const float* vsrc = a.vcache + g * kHd + d0;
  const float* prow = a.scores + (size_t)g * G * a.t_stride;
  float4 vr[4];
  float pr[4];
  // chunk k: V rows (8 float4 of the slice each) and G probability rows
  auto load = [&](uint32_t k) {
    const uint32_t jb = k * kDecChunk;
#pragma unroll
    for (int i = 0; i < 4; i++) {  // unconditional: indices clamped into bounds
      const uint32_t c = (uint32_t)(tid + 512 * i), jl = c >> 3, f4 = c & 7;
      vr[i] = ld_gf4(vsrc + (size_t)min(jb + jl, t - 1) * kvd + 4 * f4);
      const uint32_t h = min(c / kDecChunk, (uint32_t)G - 1), pl = c % kDecChunk;
      pr[i] = ld_gf(prow + (size_t)h * a.t_stride + min(jb + pl, t - 1));
    }
  };
  auto store = [&](uint32_t k) {
    const uint32_t jb = k * kDecChunk;
    lfloat* vb = vs + (k & 1) * 32 * CS;
    lfloat* pb = ps + (k & 1) * kAttnMaxGroup * CS;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t c = (uint32_t)(tid + 512 * i), jl = c >> 3, f4 = c & 7;
      if (jb + jl < t) {
        vb[(4 * f4 + 0) * CS + jl] = vr[i].x;
        vb[(4 * f4 + 1) * CS + jl] = vr[i].y;
        vb[(4 * f4 + 2) * CS + jl] = vr[i].z;
        vb[(4 * f4 + 3) * CS + jl] = vr[i].w;
      }
      const uint32_t h = c / kDecChunk, pl = c % kDecChunk;
      if ((int)h < G && jb + pl < t) pb[h * CS + pl] = pr[i];
    }
  };
  const bool chain = tid < G * 32;
  float o = 0.0f;
  load(0);
  store(0);
  __syncthreads();
  for (uint32_t k = 0; k < nch; k++) {
    if (k + 1 < nch) load(k + 1);
    if (chain) {
      const uint32_t rem = t - k * kDecChunk;
      const uint32_t jn = rem < (uint32_t)kDecChunk ? rem : (uint32_t)kDecChunk;
      o = seq_saxpy_lds(ps + (k & 1) * kAttnMaxGroup * CS + hl * CS, vs + (k & 1) * 32 * CS + dd * CS, jn, o);
    }
    if (k + 1 < nch) store(k + 1);
    __syncthreads();
  }
  if (chain) {
    const uint32_t col = (uint32_t)(g * G + hl) * kHd + d0 + dd;
    ((RLH_GLOBAL float*)a.out)[col] = o;
    q8_quant_block32(o, a.out_q8, col / 32);
  }
}

// LDS row stride of the decode kernels' score rows: whole 64-position
// pieces plus 4 floats, so that the same position of different heads' rows
// falls in different banks (the G-lane sums and the product reads touch
// several rows per instruction)
__host__ __device__ inline uint32_t dec_row_stride(uint32_t t_max) { return ((t_max + 63) & ~63u) + 4; }

// Decode with the softmax fused: grid (KVH, 4 slices of 32 dimensions),
// block 512, dynamic LDS: the group's G score rows (stride RS =
// dec_row_stride). Each block computes softmax_inplace of the G rows itself
// (the same arithmetic as k_attn_softmax): the rows arrive by
// global_load_lds while the first V chunk's loads are in flight, max and exp
// run over head groups of threads, lanes 0..G-1 run the G sequential sums
// side by side, and the probabilities stay in LDS for the saxpy chains (as
// in k_attn_pv_dec).

__global__ void __launch_bounds__(512) k_attn_smpv_dec(AttnArgs a) {
  constexpr int CS = kDecChunk + 4;
  __shared__ __attribute__((aligned(16))) float vs_g[2 * 32 * CS];
  __shared__ float red[8 * kAttnMaxGroup];
  __shared__ float s_mx[kAttnMaxGroup], s_inv[kAttnMaxGroup];
  __shared__ int s_on[kAttnMaxGroup];
  __shared__ uint64_t tab_g[32];
  extern __shared__ __attribute__((aligned(16))) float lds_generic[];
  lu64* tab = (lu64*)tab_g;
  lfloat* vs = (lfloat*)vs_g;
  lfloat* e = (lfloat*)lds_generic;
  const int G = a.H / a.KVH;
  const uint32_t RS = dec_row_stride(a.t_max);
  const uint32_t g = blockIdx.x, d0 = blockIdx.y * 32;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hl = tid >> 5, dd = tid & 31;
  const int kvd = a.KVH * kHd;
  const uint32_t t = a.pos0[0] + 1;
  const uint32_t nch = (t + kDecChunk - 1) / kDecChunk;
  const float* vsrc = a.vcache + g * kHd + d0;
  const float* srow = a.scores + (size_t)g * G * a.t_stride;
  // score rows -> LDS, 64 positions per wave instruction (positions past t
  // repeat the last score; their slots lie inside the row stride)
  const uint32_t pieces = (t + 63) / 64;
  for (uint32_t pc = wave; pc < (uint32_t)G * pieces; pc += 8) {
    const uint32_t h = pc / pieces, j0 = (pc % pieces) * 64;
    __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)(srow + (size_t)h * a.t_stride + min(j0 + lane, t - 1)),
                                     (RLH_LDS void*)(e + h * RS + j0), 4, 0, 0);
  }
  // first V chunk to registers (unconditional, indices clamped)
  float4 vr[4];
  auto load = [&](uint32_t k) {
    const uint32_t jb = k * kDecChunk;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t c = (uint32_t)(tid + 512 * i), jl = c >> 3, f4 = c & 7;
      vr[i] = ld_gf4(vsrc + (size_t)min(jb + jl, t - 1) * kvd + 4 * f4);
    }
  };
  auto store = [&](uint32_t k) {
    const uint32_t jb = k * kDecChunk;
    lfloat* vb = vs + (k & 1) * 32 * CS;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t c = (uint32_t)(tid + 512 * i), jl = c >> 3, f4 = c & 7;
      if (jb + jl < t) {
        vb[(4 * f4 + 0) * CS + jl] = vr[i].x;
        vb[(4 * f4 + 1) * CS + jl] = vr[i].y;
        vb[(4 * f4 + 2) * CS + jl] = vr[i].z;
        vb[(4 * f4 + 3) * CS + jl] = vr[i].w;
      }
    }
  };
  load(0);
  exp_tab_to_lds(tab);  // after the bulk loads: its store waits for its load
  __syncthreads();
  // softmax_inplace of the G rows (ops.rs:398-419); head hg is taken by
  // TPH = 64 * floor(8 / G) threads
  const uint32_t TPH = 64u * (8u / (uint32_t)G), WPH = TPH / 64;
  const uint32_t hg = tid / TPH, lt = tid % TPH;
  lfloat* eh = e + min(hg, (uint32_t)G - 1) * RS;
  float mx = -__int_as_float(0x7f800000);
  if (hg < (uint32_t)G)
    for (uint32_t j = lt; j < t; j += TPH) mx = fmaxf(mx, eh[j]);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  if (tid < G) {  // NaN first score: the reference's max stays NaN
    float m = red[tid * WPH];
    for (uint32_t w = 1; w < WPH; w++) m = fmaxf(m, red[tid * WPH + w]);
    const float x0 = e[tid * RS];
    s_mx[tid] = x0 != x0 ? x0 : m;
  }
  __syncthreads();
  if (hg < (uint32_t)G) {
    const float m = s_mx[hg];
    for (uint32_t j = lt; j < t; j += TPH) eh[j] = expf_glibc_t(eh[j] - m, tab);
  }
  __syncthreads();
  if (tid < G) {  // the G sequential sums side by side, one lane each
    const float sum = seq_sum_lds(e + tid * RS, t);
    s_on[tid] = sum > 0.0f;
    s_inv[tid] = 1.0f / sum;
  }
  __syncthreads();
  if (hg < (uint32_t)G && s_on[hg]) {
    const float inv = s_inv[hg];
    for (uint32_t j = lt; j < t; j += TPH) eh[j] = eh[j] * inv;
  }
  store(0);
  __syncthreads();
  // the ordered saxpy chains over double-buffered V chunks
  const bool chain = tid < G * 32;
  float o = 0.0f;
  for (uint32_t k = 0; k < nch; k++) {
    if (k + 1 < nch) load(k + 1);
    if (chain) {
      const uint32_t rem = t - k * kDecChunk;
      const uint32_t jn = rem < (uint32_t)kDecChunk ? rem : (uint32_t)kDecChunk;
      o = seq_saxpy_lds(e + hl * RS + k * kDecChunk, vs + (k & 1) * 32 * CS + dd * CS, jn, o);
    }
    if (k + 1 < nch) store(k + 1);
    __syncthreads();
  }
  if (chain) {
    const uint32_t col = (uint32_t)(g * G + hl) * kHd + d0 + dd;
    ((RLH_GLOBAL float*)a.out)[col] = o;
    q8_quant_block32(o, a.out_q8, col / 32);
  }
}

// Max over the 64 lanes of a wave (order-free) with DPP row shifts and row
// broadcasts: a lane whose DPP source is outside its row keeps its own value.
__device__ __forceinline__ float wave_max(float x) {
  auto dpp = [](float v, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), decltype(ctrl)::value, 0xf,
                                                      0xf, false));
  };
  x = fmaxf(x, dpp(x, std::integral_constant<int, 0x111>{}));  // row_shr:1
  x = fmaxf(x, dpp(x, std::integral_constant<int, 0x112>{}));  // row_shr:2
  x = fmaxf(x, dpp(x, std::integral_constant<int, 0x114>{}));  // row_shr:4
  x = fmaxf(x, dpp(x, std::integral_constant<int, 0x118>{}));  // row_shr:8
  x = fmaxf(x, dpp(x, std::integral_constant<int, 0x142>{}));  // row_bcast:15
  x = fmaxf(x, dpp(x, std::integral_constant<int, 0x143>{}));  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// Decode softmax + PV with the block's V slice resident in LDS.
// grid (KVH, 16 slices of kVsW = 8 dimensions), block 512 (8 waves); G <= 4.
// Dynamic LDS: score rows e[G][RS] | V slice vs[RS][kVsW] | product ring
// pr[3][64 chain lanes][kPrStride]. (8-wide slices: twice the blocks of
// 16-wide ones, each with half the product traffic through LDS; measured
// 8B 421.0 -> 422.3, 4B 490.2 -> 491.3, 0.6B 946.9 -> 952.5 tok/s.)
// * At entry every wave issues its DMA copies: the G score rows, then exactly
//   kVDma 1 KB pieces of the V slice (kVRows rows x 4 kVsW bytes each; a
//   piece index past the last is clamped, so a repeated piece rewrites the
//   same bytes).
//   The softmax runs while the V slice lands.
// * softmax_inplace of the G rows as in k_attn_smpv_dec.
// * PV: chain lane l < G*kVsW of wave 0 owns (head l / kVsW, dimension
//   l % kVsW) and adds its products in position order, o = prod_j + o (the saxpy's
//   add); the products prod_j = p_j * v_j[d] are formed by waves 1..7 one
//   64-position chunk ahead into a ring of three chunk slots, so the chain
//   wave issues one add per position and a 16-byte LDS read per four (a
//   multiply on the chain wave would cost an issue slot per position).
//   One block barrier per chunk: at chunk c the chain reads slot c % 3 while
//   the producers fill slot (c + 2) % 3.
// The output is written in f32; its Q8 blocks are made by the attn_output
// matvec's prologue.
constexpr int kVsW = 8;               // dimensions per block
constexpr int kPrC = 64;              // positions per product chunk
constexpr int kPrStride = kPrC + 4;   // floats per chain lane in a chunk slot
constexpr int kPrSlots = 3;
constexpr int kVRows = 256 / kVsW;    // V-slice rows per 1 KB DMA piece
constexpr int kVDma = 1536 / (8 * kVRows);  // V-slice DMA pieces per wave
constexpr uint32_t kDecVMaxCtx = 8u * kVDma * kVRows;  // 1536 positions
constexpr size_t kDecVLdsMax = 150u * 1024u;

// The chain wave's part of a product ring (chunk c of kPrC positions in
// slot c % kPrSlots of slot_floats floats, chain lane l's kPrC products at
// l * kPrStride in the slot, one block barrier per chunk): o = prod_j + o
// in position order for chain lane lc. Chunk c + 1 is complete while chunk
// c is added (it was made before the previous barrier), so the reads run
// one 32-position batch ahead across chunk boundaries; the chain wave
// writes no LDS and meets the producers at a plain s_barrier. Lanes past the
// chain count pass a clamped lc and run a copy of a chain (uniform control
// flow).
__device__ __forceinline__ float chain_products(const lfloat* pr, uint32_t lc, uint32_t t, uint32_t nch,
                                                uint32_t slot_floats) {
  const lfloat* base = pr + lc * kPrStride;
  auto slotp = [&](uint32_t c) { return (const lf32x4d*)(base + (c % kPrSlots) * slot_floats); };
  float o = 0.0f;
  f32x4d_t xa[8], xb[8];
#pragma unroll
  for (int i = 0; i < 8; i++) xa[i] = slotp(0)[i];
  for (uint32_t c = 0; c < nch; c++) {
    const lf32x4d* sc = slotp(c);
    const lf32x4d* sn = slotp(c + 1);  // past the last chunk: read, never added
    const uint32_t n = t - c * kPrC;
    if (n >= (uint32_t)kPrC) {
#pragma unroll
      for (int i = 0; i < 8; i++) xb[i] = sc[8 + i];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; i++) o = (((o + xa[i].x) + xa[i].y) + xa[i].z) + xa[i].w;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; i++) xa[i] = sn[i];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; i++) o = (((o + xb[i].x) + xb[i].y) + xb[i].z) + xb[i].w;
      __builtin_amdgcn_sched_barrier(0);
    } else {
      o = seq_sum_lds((const lfloat*)sc, n, o);
    }
    asm volatile("s_barrier" ::: "memory");
  }
  return o;
}

__global__ void __launch_bounds__(512) k_attn_dec_v(AttnArgs a) {
  __shared__ float red[8 * kAttnMaxGroup];
  __shared__ float s_mx[kAttnMaxGroup], s_inv[kAttnMaxGroup];
  __shared__ int s_on[kAttnMaxGroup];
  __shared__ uint32_t s_exp_done[kDecVMaxCtx / 256];
  __shared__ uint64_t tab_g[32];
  extern __shared__ __attribute__((aligned(16))) float lds_generic[];
  lu64* tab = (lu64*)tab_g;
  const int G = a.H / a.KVH;
  const uint32_t RS = dec_row_stride(a.t_max);
  lfloat* e = (lfloat*)lds_generic;
  lfloat* vs = e + (size_t)G * RS;
  lfloat* pr = vs + (size_t)RS * kVsW;
  const uint32_t g = blockIdx.x, d0 = blockIdx.y * kVsW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kvd = a.KVH * kHd;
  const uint32_t t = a.pos0[0] + 1;
  if (tid < kDecVMaxCtx / 256) s_exp_done[tid] = 0u;  // seen by all after the first barrier
  const float* srow = a.scores + (size_t)g * G * a.t_stride;
  // score rows -> LDS (positions past t repeat the last score; their slots
  // lie inside the row stride), the exp table, then the V slice
  const uint32_t pieces = (t + 63) / 64;
  for (uint32_t pc = wave; pc < (uint32_t)G * pieces; pc += 8) {
    const uint32_t h = pc / pieces, j0 = (pc % pieces) * 64;
    __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)(srow + (size_t)h * a.t_stride + min(j0 + lane, t - 1)),
                                     (RLH_LDS void*)(e + h * RS + j0), 4, 0, 0);
  }
  if (wave == 0) exp_tab_dma(tab);
  {
    const uint32_t nvp = (t + kVRows - 1) / kVRows;
    const float* vsrc = a.vcache + g * kHd + d0 + (lane % (kVsW / 4)) * 4;
#pragma unroll
    for (int i = 0; i < kVDma; i++) {
      const uint32_t pc = min((uint32_t)(wave + 8 * i), nvp - 1);
      const uint32_t row = min(pc * kVRows + (uint32_t)lane / (kVsW / 4), t - 1);
      __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)(vsrc + (size_t)row * kvd),
                                       (RLH_LDS void*)(vs + pc * kVRows * kVsW), 16, 0, 0);
    }
  }
  wait_vmcnt<kVDma>();  // this wave's score rows (and table) have landed
  lds_barrier();
  // softmax_inplace of the G rows (ops.rs:398-419); head hg is taken by
  // TPH = 64 * floor(8 / G) threads, four consecutive positions at a time
  // (the positions from t to the next multiple of 4 hold copies of the last
  // score: they leave the max unchanged and are never summed)
  const uint32_t TPH = 64u * (8u / (uint32_t)G), WPH = TPH / 64;
  const uint32_t hg = tid / TPH, lt = tid % TPH;
  const bool hon = hg < (uint32_t)G;
  lfloat* eh = e + min(hg, (uint32_t)G - 1) * RS;
  const uint32_t nq4 = (t + 3) / 4;
  float mx = -__int_as_float(0x7f800000), my = mx;
  if (hon)
    for (uint32_t q = lt; q < nq4; q += 2 * TPH) {
      const f32x4_t x = *(const lf32x4*)(eh + 4 * q);
      const f32x4_t y = *(const lf32x4*)(eh + 4 * min(q + TPH, nq4 - 1));
      mx = fmaxf(fmaxf(mx, x.x), fmaxf(x.y, fmaxf(x.z, x.w)));
      my = fmaxf(fmaxf(my, y.x), fmaxf(y.y, fmaxf(y.z, y.w)));
    }
  mx = wave_max(fmaxf(mx, my));
  if (lane == 0) red[wave] = mx;
  lds_barrier();
  if (tid < G) {  // NaN first score: the reference's max stays NaN
    float m = red[tid * WPH];
    for (uint32_t w = 1; w < WPH; w++) m = fmaxf(m, red[tid * WPH + w]);
    const float x0 = e[tid * RS];
    s_mx[tid] = x0 != x0 ? x0 : m;
  }
  lds_barrier();
  // The exponentials, 256 positions of every row at a time, by waves 1..3
  // and 5..7; each of waves 1..7 announces a finished chunk on that chunk's counter, and lanes
  // 0..G-1 of wave 0 run the G sequential sums right behind them, each chunk
  // once all seven waves have announced it (every wave finishes every chunk,
  // so each wait ends). One counter per chunk: waves without work in a chunk
  // run ahead, so a single running total would not say which chunks are done.
  constexpr uint32_t kExpC = 256;
  RLH_LDS uint32_t* exp_done = (RLH_LDS uint32_t*)s_exp_done;
  const uint32_t nek = (t + kExpC - 1) / kExpC;
  if (wave != 0) {
    // wave 4 runs on wave 0's SIMD: it takes no exponentials (they would
    // take issue cycles from the sums) and only announces the chunks
    const uint32_t xw = wave < 4 ? wave - 1 : wave - 2;
    for (uint32_t k = 0; k < nek; k++) {
      for (uint32_t i = wave == 4 ? ~0u : xw * 64 + lane; i < (uint32_t)G * (kExpC / 4); i += 384) {
        const uint32_t h = i / (kExpC / 4), q = k * (kExpC / 4) + i % (kExpC / 4);
        if (q < nq4) {
          lfloat* x4 = e + h * RS + 4 * q;
          const float m = s_mx[h];
          const f32x4_t x = *(const lf32x4*)x4;
          *(lf32x4*)x4 = f32x4_t{expf_glibc_t(x.x - m, tab), expf_glibc_t(x.y - m, tab),
                                 expf_glibc_t(x.z - m, tab), expf_glibc_t(x.w - m, tab)};
        }
      }
      // LDS-only hand-over: a wave's LDS operations complete in order, so
      // lgkmcnt(0) before a relaxed add publishes the chunk (release/acquire
      // atomics would also wait for the wave's in-flight global copies);
      // the asm statements keep the compiler from moving accesses across
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0): the chunk is in LDS
      asm volatile("" ::: "memory");
      if (lane == 0) __hip_atomic_fetch_add(exp_done + k, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  } else if (tid < G) {  // the G sequential sums side by side, one lane each
    float sum = 0.0f;
    for (uint32_t k = 0; k < nek; k++) {
      wait_lds_count(exp_done + k, 7u, a.err, kErrAttnExp);
      const uint32_t n = t - k * kExpC < kExpC ? t - k * kExpC : kExpC;
      sum = seq_sum_lds(e + tid * RS + k * kExpC, n, sum);
    }
    s_on[tid] = sum > 0.0f;
    s_inv[tid] = 1.0f / sum;
  }
  wait_vmcnt<0>();  // this wave's V pieces have landed
  lds_barrier();
  // PV. Chain lane l < NL = G * 8 (head h = l / 8, dimension l % 8). The
  // producers (waves 1..7) are bound by their instruction issue, so both
  // half-waves work: lane l of wave w forms chain l % 32's products of the
  // position quad 2 (w - 1) + l / 32 of a chunk (wave 1 also quad 14 +
  // l / 32): p_j = e_j * (1 / sum) when sum > 0 (softmax_inplace's last
  // loop), then p_j * v_j[d], both rounded as the reference rounds them.
  const uint32_t NL = (uint32_t)G * kVsW;  // chain lanes (at most 32)
  const uint32_t nch = (t + kPrC - 1) / kPrC;
  const uint32_t cl = (uint32_t)lane & 31, hq = (uint32_t)lane >> 5;
  const uint32_t ph = min(cl, NL - 1) / kVsW;
  const bool pon = s_on[ph];
  const float pinv = s_inv[ph];
  auto produce = [&](uint32_t c) {
    if (cl >= NL) return;
    lfloat* slot = pr + (c % kPrSlots) * (64 * kPrStride) + cl * kPrStride;
    const lfloat* ec = e + ph * RS + c * kPrC;  // < RS: chunks never pass the row stride
    const lfloat* vc = vs + c * kPrC * kVsW + cl % kVsW;
    for (uint32_t q = 2 * ((uint32_t)wave - 1) + hq; q < (uint32_t)kPrC / 4; q += 14) {
      f32x4_t x = *(const lf32x4*)(ec + 4 * q);
      if (pon) x = f32x4_t{x.x * pinv, x.y * pinv, x.z * pinv, x.w * pinv};
      const lfloat* v = vc + 4 * q * kVsW;
      *(lf32x4*)(slot + 4 * q) = f32x4_t{x.x * v[0], x.y * v[kVsW], x.z * v[2 * kVsW], x.w * v[3 * kVsW]};
    }
  };
  if (wave != 0 && cl < NL) {
    // chunks 0 and 1 before the chain starts: all their reads first
    f32x4_t px[2][2];
    float vx[2][2][4];
#pragma unroll
    for (int cc = 0; cc < 2; cc++) {
      const uint32_t c = min((uint32_t)cc, nch - 1);
      const lfloat* ec = e + ph * RS + c * kPrC;
      const lfloat* vc = vs + c * kPrC * kVsW + cl % kVsW;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t q = min(2 * ((uint32_t)wave - 1) + hq + 14u * i, (uint32_t)kPrC / 4 - 1);
        px[cc][i] = *(const lf32x4*)(ec + 4 * q);
#pragma unroll
        for (int r = 0; r < 4; r++) vx[cc][i][r] = vc[(4 * q + r) * kVsW];
      }
    }
#pragma unroll
    for (int cc = 0; cc < 2; cc++) {
      if ((uint32_t)cc >= nch) break;
      lfloat* slot = pr + cc * (64 * kPrStride) + cl * kPrStride;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t q = 2 * ((uint32_t)wave - 1) + hq + 14u * i;
        if (q >= (uint32_t)kPrC / 4) break;
        f32x4_t x = px[cc][i];
        if (pon) x = f32x4_t{x.x * pinv, x.y * pinv, x.z * pinv, x.w * pinv};
        *(lf32x4*)(slot + 4 * q) =
            f32x4_t{x.x * vx[cc][i][0], x.y * vx[cc][i][1], x.z * vx[cc][i][2], x.w * vx[cc][i][3]};
      }
    }
  }
  lds_barrier();
  if (wave != 0) {
    for (uint32_t c = 0; c < nch; c++) {
      if (c + 2 < nch) produce(c + 2);
      lds_barrier();
    }
    return;
  }
  const float o = chain_products(pr, min((uint32_t)lane, NL - 1), t, nch, 64 * kPrStride);
  if ((uint32_t)lane < NL)
    ((RLH_GLOBAL float*)a.out)[(g * G + lane / kVsW) * kHd + d0 + lane % kVsW] = o;
}


// Decode PV over any context (after k_attn_softmax wrote the probabilities
// over the scores), V and p streamed through LDS. grid (128 / W slices of W
// dimensions, KVH), W = 8 (4 when more than 4 query heads share a KV head,
// so a block never has more than 32 chains), block 512. Wave 0 lane l < NL
// = G * W (head l / W, dimension l % W) adds the products in position order
// (chain_products); waves 1..7 (producers) stream each 64-position chunk's
// p rows and V slice into an 8-slot input ring by DMA, and form the products
// two chunks ahead of the chain into the 3-slot product ring. The producers
// are bound by their instruction issue (two share most SIMDs), so both
// half-waves of a producer work: lane l forms chain l % 32's products of
// quad 2 (w - 1) + l / 32 of a chunk (and producer 1 also quad 14 + l / 32).
// Every producer wave issues
// exactly two DMA copies per chunk (duplicates of its last job where a chunk
// has fewer jobs: the same bytes to the same place), so its vector-memory
// count says when a chunk it is about to use has landed: at the end of
// iteration c it waits for chunk c + 3 (the copies of chunks c + 4 .. c + 8
// may stay in flight), and the block barrier then makes every wave's copies
// visible. The output is written in f32 (attn_output quantizes the row).
constexpr int kRingSlots = 8;  // input ring: chunks c .. c + 7 resident or in flight

__host__ __device__ inline uint32_t pv_ring_width(uint32_t group) { return group > 4 ? 4u : 8u; }

__host__ __device__ inline size_t pv_ring_lds(uint32_t group) {
  const size_t w = pv_ring_width(group);
  const size_t prod = (size_t)kPrSlots * 64 * kPrStride * 4;
  const size_t in_slot = ((size_t)group * kPrStride + (size_t)kPrC * w) * 4;
  return prod + kRingSlots * in_slot;
}

__global__ void __launch_bounds__(512) k_attn_pv_ring(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds_generic[];
  const uint32_t G = (uint32_t)(a.H / a.KVH);
  const uint32_t W = pv_ring_width(G), NL = G * W;
  // p rows [G][64] at a stride of kPrStride floats (a producer's 16-byte
  // reads of G rows fall in distinct banks), then V rows [64][W]
  const uint32_t in_floats = G * kPrStride + kPrC * W;
  lfloat* pr = (lfloat*)lds_generic;
  lfloat* in = pr + kPrSlots * 64 * kPrStride;
  const uint32_t d0 = blockIdx.x * W, g = blockIdx.y;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t kvd = (uint32_t)a.KVH * kHd;
  const uint32_t t = a.pos0[0] + 1;
  const uint32_t nch = (t + kPrC - 1) / kPrC;
  const uint32_t nvj = W / 4;       // V copies per chunk: 16 B per lane, 256 / W rows each
  const uint32_t njobs = nvj + G;   // + one copy per p row (4 B per lane)
  const uint32_t pw = wave - 1;     // producer index (waves 1..7)
  auto fetch = [&](uint32_t c) {
    lfloat* slot = in + (c % kRingSlots) * in_floats;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const uint32_t j = min(2 * pw + (uint32_t)k, njobs - 1);
      if (j < nvj) {
        const uint32_t rpi = 256 / W;  // rows per copy
        const uint32_t row = min(c * kPrC + rpi * j + lane / (W / 4), t - 1);
        __builtin_amdgcn_global_load_lds(
            (const RLH_GLOBAL void*)(a.vcache + (size_t)row * kvd + g * kHd + d0 + (lane % (W / 4)) * 4),
            (RLH_LDS void*)(slot + G * kPrStride + rpi * j * W), 16, 0, 0);
      } else {
        const uint32_t h = j - nvj, pos = min(c * kPrC + lane, t - 1);
        __builtin_amdgcn_global_load_lds(
            (const RLH_GLOBAL void*)(a.scores + (size_t)(g * G + h) * a.t_stride + pos),
            (RLH_LDS void*)(slot + h * kPrStride), 4, 0, 0);
      }
    }
  };
  // lane l of a producer forms chain l % 32's products of the quads
  // 2 pw + l / 32 and (producer 0 only) 14 + l / 32 of the chunk: the two
  // half-waves split the 16 quads, at most two per lane
  const uint32_t cl = lane & 31, hq = lane >> 5;
  auto produce = [&](uint32_t c) {
    if (cl >= NL) return;
    const lfloat* slot = in + (c % kRingSlots) * in_floats;
    lfloat* ps = pr + (c % kPrSlots) * (64 * kPrStride) + cl * kPrStride;
    const lfloat* pc = slot + (cl / W) * kPrStride;
    const lfloat* vc = slot + G * kPrStride + cl % W;
    for (uint32_t q = 2 * pw + hq; q < (uint32_t)kPrC / 4; q += 14) {
      const f32x4_t p = *(const lf32x4*)(pc + 4 * q);
      const lfloat* v = vc + 4 * q * W;
      *(lf32x4*)(ps + 4 * q) = f32x4_t{p.x * v[0], p.y * v[W], p.z * v[2 * W], p.w * v[3 * W]};
    }
  };
  // every wave meets the two set-up barriers, then the nch barriers of the
  // chunk loop (wave 0 inside chain_products)
  if (wave != 0) {
    for (uint32_t c = 0; c < (uint32_t)kRingSlots; c++) fetch(c);
    wait_vmcnt<2 * (kRingSlots - 2)>();  // chunks 0 and 1 have landed
  }
  lds_barrier();
  if (wave != 0) {
    produce(0);
    if (nch > 1) produce(1);
    wait_vmcnt<2 * (kRingSlots - 3)>();  // chunk 2
  }
  lds_barrier();
  if (wave == 0) {
    const float o = chain_products(pr, min(lane, NL - 1), t, nch, 64 * kPrStride);
    if (lane < NL) ((RLH_GLOBAL float*)a.out)[(g * G + lane / W) * kHd + d0 + lane % W] = o;
    return;
  }
  for (uint32_t c = 0; c < nch; c++) {
    if (c + 2 < nch) produce(c + 2);
    fetch(c + kRingSlots);               // into chunk c's input slot (its products were made at c - 2)
    wait_vmcnt<2 * (kRingSlots - 3)>();  // chunk c + 3 has landed
    lds_barrier();
  }
}

// grid: (KVH, ceil(n_tok / TT)), TT = 32 / G tokens per block, latest (most
// positions) token tiles first; block 512: thread (d = tid % 128, quarter
// tid / 128) runs the chains of combinations quarter + 4i.
__global__ void __launch_bounds__(512) k_attn_pv_pre(AttnArgs a) {
  constexpr int CS = kPreChunk + 4;
  constexpr int NC = kPreComb / 4;  // chains per thread
  __shared__ __attribute__((aligned(16))) float vs_g[kPreChunk * kHd];
  __shared__ __attribute__((aligned(16))) float ps_g[kPreComb * CS];
  lfloat* vs = (lfloat*)vs_g;
  lfloat* ps = (lfloat*)ps_g;
  const int G = a.H / a.KVH;
  const uint32_t TT = (uint32_t)(kPreComb / G);
  const int ncomb = (int)TT * G;
  const uint32_t g = blockIdx.x;
  const uint32_t tok0 = (gridDim.y - 1 - blockIdx.y) * TT;
  const uint32_t ntok = a.n_tok - tok0 < TT ? a.n_tok - tok0 : TT;
  const int tid = threadIdx.x, d = tid & 127, qtr = tid >> 7;
  const int qd = a.H * kHd, kvd = a.KVH * kHd;
  const uint32_t p0 = a.pos0[0];
  const uint32_t t_lo = p0 + tok0 + 1, t_hi = p0 + tok0 + ntok;
  float o[NC];
  uint32_t tlim[NC];  // positions chain i takes (0 for combinations past the last token)
#pragma unroll
  for (int i = 0; i < NC; i++) {
    o[i] = 0.0f;
    const int cb = qtr + 4 * i;
    const uint32_t tt = (uint32_t)(cb / G);
    tlim[i] = cb < ncomb && tt < ntok ? p0 + tok0 + tt + 1 : 0u;
  }
  // chunk loads go to registers one chunk ahead and into LDS after the
  // chunk in use is consumed
  float4 vr[4];
  float pr[4];
  auto load = [&](uint32_t j0) {
    const uint32_t jn = t_hi - j0 < (uint32_t)kPreChunk ? t_hi - j0 : (uint32_t)kPreChunk;
#pragma unroll
    for (int i = 0; i < 4; i++) {  // unconditional: indices clamped into bounds
      const uint32_t c = (uint32_t)(tid + 512 * i), jl = c >> 5, f4 = c & 31;
      vr[i] = ld_gf4(a.vcache + (size_t)(j0 + min(jl, jn - 1)) * kvd + g * kHd + 4 * f4);
      const uint32_t cb = min(c / kPreChunk, (uint32_t)ncomb - 1), pl = c % kPreChunk;
      const uint32_t tt = min(cb / G, ntok - 1);
      pr[i] = ld_gf(a.scores + ((size_t)(tok0 + tt) * a.H + g * G + cb % G) * a.t_stride +
                    min(j0 + pl, p0 + tok0 + tt));
    }
  };
  auto store = [&](uint32_t j0) {
    const uint32_t jn = t_hi - j0 < (uint32_t)kPreChunk ? t_hi - j0 : (uint32_t)kPreChunk;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t c = (uint32_t)(tid + 512 * i), jl = c >> 5, f4 = c & 31;
      if (jl < jn) *(lf32x4*)(vs + jl * kHd + 4 * f4) = f32x4_t{vr[i].x, vr[i].y, vr[i].z, vr[i].w};
      const uint32_t cb = c / kPreChunk, pl = c % kPreChunk, tt = cb / G;
      if ((int)cb < ncomb && tt < ntok && j0 + pl < p0 + tok0 + tt + 1) ps[cb * CS + pl] = pr[i];
    }
  };
  load(0);
  store(0);
  __syncthreads();
  for (uint32_t j0 = 0; j0 < t_hi; j0 += kPreChunk) {
    const uint32_t jn = t_hi - j0 < (uint32_t)kPreChunk ? t_hi - j0 : (uint32_t)kPreChunk;
    const bool more = j0 + kPreChunk < t_hi;
    if (more) load(j0 + kPreChunk);
    // positions below t_lo are taken by every chain
    const uint32_t jf = t_lo > j0 ? (t_lo - j0 < jn ? t_lo - j0 : jn) : 0u;
    // every chain runs here, branch-free, with all its p reads issued before
    // the arithmetic (a chain past the last token reads rows of ps that hold
    // nothing and is never stored)
    uint32_t jj = 0;
    for (; jj + 4 <= jf; jj += 4) {
      const float v0 = vs[jj * kHd + d], v1 = vs[(jj + 1) * kHd + d];
      const float v2 = vs[(jj + 2) * kHd + d], v3 = vs[(jj + 3) * kHd + d];
      f32x4_t p[NC];
#pragma unroll
      for (int i = 0; i < NC; i++) p[i] = *(const lf32x4*)(ps + (qtr + 4 * i) * CS + jj);
#pragma unroll
      for (int i = 0; i < NC; i++) {
        o[i] = p[i].x * v0 + o[i];
        o[i] = p[i].y * v1 + o[i];
        o[i] = p[i].z * v2 + o[i];
        o[i] = p[i].w * v3 + o[i];
      }
    }
    for (; jj < jn; jj++) {
      const uint32_t j = j0 + jj;
      const float v = vs[jj * kHd + d];
#pragma unroll
      for (int i = 0; i < NC; i++)
        if (j < tlim[i]) o[i] = ps[(qtr + 4 * i) * CS + jj] * v + o[i];
    }
    __syncthreads();  // the chunk is consumed
    if (more) {
      store(j0 + kPreChunk);
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < NC; i++) {
    if (tlim[i]) {
      const int cb = qtr + 4 * i;
      const uint32_t tok = tok0 + (uint32_t)(cb / G);
      const uint32_t col = (uint32_t)(g * G + cb % G) * kHd + d;
      ((RLH_GLOBAL float*)a.out)[(size_t)tok * qd + col] = o[i];
      const uint32_t nbq = (uint32_t)qd / 32;
      Q8Out ot{a.out_q8.qs + (size_t)tok * qd, a.out_q8.d + (size_t)tok * nbq, a.out_q8.s + (size_t)tok * nbq,
               a.out_q8.s16 + (size_t)tok * nbq * 2};
      q8_quant_block32(o[i], ot, col / 32);
    }
  }
}

size_t softmax_lds(uint32_t t_max) { return (size_t)((t_max + 3) & ~3u) * 4; }

// k_attn_softmax_rows: at most this much LDS per block for 16 rows (up to
// 960 positions) and 8 rows (up to 1984); 4 rows take up to
// kSoftmaxRows1Lds (4988 positions: two blocks and their static arrays fit
// one CU's 160 KB); longer rows take k_attn_softmax<false>.
constexpr size_t kSoftmaxRowsLds = 65536;
constexpr size_t kSoftmaxRows1Lds = 80896;
size_t softmax_rows_lds(uint32_t t_max, int rw) { return (size_t)4 * rw * softmax_rows_stride(t_max) * 4; }

}  // namespace

void launch_attn_scores(hipStream_t st, const AttnArgs& a, bool fused) {
  const uint32_t ntiles = (a.t_max + kPosTile - 1) / kPosTile;
  if (fused) {
    hipLaunchKernelGGL(k_attn_qk, dim3(a.KVH * ntiles, a.n_tok), dim3(256), 0, st, a);
  } else {
    const uint32_t G = (uint32_t)(a.H / a.KVH), p0 = a.t_max - a.n_tok;
    const uint32_t TP = (uint32_t)kPreQkComb / G, blocks = (uint32_t)a.KVH * qk_items_per_head(p0, a.n_tok, TP);
    const char* env = std::getenv("RLH_QK_PRE_GRID");  // '1': always the grid kernel (tests)
    const bool grid_only = env && env[0] == '1';
    if (!grid_only && g_qk_pre_resident && blocks <= kQkPersistRounds * g_qk_pre_resident) {
      const uint32_t per_g = qk_items_per_head(p0, a.n_tok, (uint32_t)kPreQkItem / G);
      const uint32_t n_items = (uint32_t)a.KVH * per_g;
      hipLaunchKernelGGL(k_attn_qk_pre_p, dim3(std::min(n_items, g_qk_pre_resident)), dim3(256), 0, st, a, per_g);
    } else {
      hipLaunchKernelGGL(k_attn_qk_pre, dim3(a.KVH * ntiles, (a.n_tok + TP - 1) / TP), dim3(256), 0, st, a);
    }
  }
}

void launch_attn_softmax(hipStream_t st, const AttnArgs& a) {
  if (a.n_tok == 1)
    hipLaunchKernelGGL(k_attn_softmax<true>, dim3(a.H, 1), dim3(kSoftmaxWalkThreads), softmax_lds(a.t_max), st, a);
  else if (softmax_rows_lds(a.t_max, 4) <= kSoftmaxRowsLds)
    hipLaunchKernelGGL(k_attn_softmax_rows<4>, dim3(a.H, (a.n_tok + 15) / 16), dim3(256),
                       softmax_rows_lds(a.t_max, 4), st, a);
  else if (softmax_rows_lds(a.t_max, 2) <= kSoftmaxRowsLds)
    hipLaunchKernelGGL(k_attn_softmax_rows<2>, dim3(a.H, (a.n_tok + 7) / 8), dim3(256), softmax_rows_lds(a.t_max, 2),
                       st, a);
  else if (softmax_rows_lds(a.t_max, 1) <= kSoftmaxRows1Lds)
    hipLaunchKernelGGL(k_attn_softmax_rows<1>, dim3(a.H, (a.n_tok + 3) / 4), dim3(256), softmax_rows_lds(a.t_max, 1),
                       st, a);
  else
    hipLaunchKernelGGL(k_attn_softmax<false>, dim3(a.H, a.n_tok), dim3(256), softmax_lds(a.t_max), st, a);
}

size_t attn_dec_fused_lds(uint32_t t_max, uint32_t group) {
  const size_t b = (size_t)group * dec_row_stride(t_max) * 4;
  return b <= kDecFusedLds ? b : 0;
}

size_t attn_dec_v_lds(uint32_t t_max, uint32_t group) {
  if (group < 1 || group > 4 || t_max > kDecVMaxCtx) return 0;
  const size_t rs = dec_row_stride(t_max);
  const size_t b = (size_t)group * rs * 4 + rs * kVsW * 4 + (size_t)kPrSlots * 64 * kPrStride * 4;
  return b <= kDecVLdsMax ? b : 0;
}

void launch_attn_decode(hipStream_t st, const AttnArgs& a, bool f32_out) {
  const uint32_t G = (uint32_t)(a.H / a.KVH);
  if (f32_out) {
    const size_t lv = attn_dec_v_lds(a.t_max, G);
    if (lv) {
      hipLaunchKernelGGL(k_attn_dec_v, dim3(a.KVH, kHd / kVsW), dim3(512), lv, st, a);
    } else {
      launch_attn_softmax(st, a);
      hipLaunchKernelGGL(k_attn_pv_ring, dim3(kHd / pv_ring_width(G), a.KVH), dim3(512), pv_ring_lds(G), st, a);
    }
    return;
  }
  const size_t lds = attn_dec_fused_lds(a.t_max, (uint32_t)(a.H / a.KVH));
  if (lds) {
    hipLaunchKernelGGL(k_attn_smpv_dec, dim3(a.KVH, 4), dim3(512), lds, st, a);
  } else {
    launch_attn_softmax(st, a);
    hipLaunchKernelGGL(k_attn_pv_dec, dim3(a.KVH, 4), dim3(512), 0, st, a);
  }
}

void launch_attn_pv(hipStream_t st, const AttnArgs& a, bool decode) {
  if (decode) {
    hipLaunchKernelGGL(k_attn_pv_dec, dim3(a.KVH, 4), dim3(512), 0, st, a);
  } else {
    const uint32_t TT = (uint32_t)(kPreComb / (a.H / a.KVH));
    hipLaunchKernelGGL(k_attn_pv_pre, dim3(a.KVH, (a.n_tok + TT - 1) / TT), dim3(512), 0, st, a);
  }
}

bool attn_init(uint32_t max_ctx) {
  if (max_ctx > kAttnMaxCtx) return false;
  if (!g_qk_pre_resident) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)k_attn_qk_pre_p, 256, 0) == hipSuccess &&
        cus > 0 && per_cu > 0)
      g_qk_pre_resident = (uint32_t)(cus * per_cu);
  }
  size_t ring_lds = 0;
  for (uint32_t gq = 1; gq <= (uint32_t)kAttnMaxGroup; gq++) ring_lds = std::max(ring_lds, pv_ring_lds(gq));
  return hipFuncSetAttribute((const void*)k_attn_softmax<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)softmax_lds(kAttnMaxCtx)) == hipSuccess &&
         hipFuncSetAttribute((const void*)k_attn_softmax<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)softmax_lds(kAttnMaxCtx)) == hipSuccess &&
         hipFuncSetAttribute((const void*)k_attn_softmax_rows<1>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)kSoftmaxRows1Lds) == hipSuccess &&
         hipFuncSetAttribute((const void*)k_attn_softmax_rows<2>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)kSoftmaxRowsLds) == hipSuccess &&
         hipFuncSetAttribute((const void*)k_attn_softmax_rows<4>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)kSoftmaxRowsLds) == hipSuccess &&
         hipFuncSetAttribute((const void*)k_attn_smpv_dec, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)kDecFusedLds) == hipSuccess &&
         hipFuncSetAttribute((const void*)k_attn_dec_v, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)kDecVLdsMax) == hipSuccess &&
         hipFuncSetAttribute((const void*)k_attn_pv_ring, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)ring_lds) == hipSuccess;
}

}  // namespace rlh
