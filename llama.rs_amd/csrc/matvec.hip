// matvec.hip — decode matvec (ops.rs:67-141, integer path) for gfx950.
//
// Exactness: every row's f32 total is the sequential sum, in the reference's
// index order, of the per-group terms of dot_q4k_q8_avx2 (simd.rs:581),
// dot_q6k_q8_avx2 (simd.rs:663), dot_q80_q8_avx2 (simd.rs:891) or
// dot_q40_q8_avx2 (simd.rs:863), each term evaluated with the reference's
// expression and rounding.
//
// Structure (HBM-bound): a block of 256 threads owns R = 4 * NS * P rows of
// one matrix. The row is walked in chunks of 64/P "units" per lane group (a
// unit = the weights behind one term, or four consecutive terms for Q6_K).
// Per chunk every lane first issues the loads of its unit for all NS of its
// rows (memory-level parallelism), then computes the terms into an LDS tile
// [row][term]. The in-order per-row sum (one lane per row) of chunk k-1 runs
// while chunk k's loads are in flight, from a double-buffered tile. Rows
// narrower than 64 units pack P rows per wave instruction.
//
// One launch covers up to three matrices (the q/k/v projections) of mixed
// ggml types; a segment in PAIR mode computes the same rows of two matrices
// (ffn_gate, ffn_up) and fuses SwiGLU + Q8 quantisation of the 32-row block
// (model.rs:720-724, ops.rs:393-395, simd.rs:116-203).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"
#include "matvec.h"
#include "rlh_device.h"

namespace rlh {

namespace {

constexpr int kThreads = 256;
typedef RLH_LDS float lfloat;
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef RLH_LDS f32x4_t lf32x4;

// ---- per-type unit loaders and term evaluators ------------------------------
template <uint32_t TY>
struct MU;

template <>
struct MU<RLH_TYPE_Q4_K> {
  static constexpr int kT = 1;
  struct W {
    uint4 hdr, q0, q1;
  };
  struct A {
    uint4 a0, a1, b0, b1;
    float da, db, sa, sb;
  };
  __device__ __forceinline__ static uint32_t units(uint32_t cols) { return cols >> 6; }
  __device__ __forceinline__ static A act(const Q8Ptr& q, uint32_t u) {
    uint32_t ab = (u >> 2) * 8 + 2 * (u & 3);
    const int8_t* p = q.qs + (size_t)ab * 32;
    A a;
    a.a0 = ld_g16(p);
    a.a1 = ld_g16(p + 16);
    a.b0 = ld_g16(p + 32);
    a.b1 = ld_g16(p + 48);
    a.da = ld_gf(q.d + ab);
    a.db = ld_gf(q.d + ab + 1);
    a.sa = (float)ld_gi(q.s + ab);
    a.sb = (float)ld_gi(q.s + ab + 1);
    return a;
  }
  __device__ __forceinline__ static W load(const DevMat& w, uint32_t row, uint32_t u) {
    const uint8_t* sb = w.a + (size_t)row * w.row_bytes + (size_t)(u >> 2) * 144;
    uint32_t g = u & 3;
    W r;
    r.hdr = ld_nt16(sb);
    r.q0 = ld_nt16(sb + 16 + 32 * g);
    r.q1 = ld_nt16(sb + 32 + 32 * g);
    return r;
  }
  __device__ __forceinline__ static void terms(const W r, const A& a, uint32_t u, lfloat* t) {
    const uint32_t m = 0x0F0F0F0Fu;
    uint32_t g = u & 3;
    int i1 = 0, i2 = 0;
    i1 = sdot4(r.q0.x & m, a.a0.x, i1); i1 = sdot4(r.q0.y & m, a.a0.y, i1);
    i1 = sdot4(r.q0.z & m, a.a0.z, i1); i1 = sdot4(r.q0.w & m, a.a0.w, i1);
    i1 = sdot4(r.q1.x & m, a.a1.x, i1); i1 = sdot4(r.q1.y & m, a.a1.y, i1);
    i1 = sdot4(r.q1.z & m, a.a1.z, i1); i1 = sdot4(r.q1.w & m, a.a1.w, i1);
    i2 = sdot4((r.q0.x >> 4) & m, a.b0.x, i2); i2 = sdot4((r.q0.y >> 4) & m, a.b0.y, i2);
    i2 = sdot4((r.q0.z >> 4) & m, a.b0.z, i2); i2 = sdot4((r.q0.w >> 4) & m, a.b0.w, i2);
    i2 = sdot4((r.q1.x >> 4) & m, a.b1.x, i2); i2 = sdot4((r.q1.y >> 4) & m, a.b1.y, i2);
    i2 = sdot4((r.q1.z >> 4) & m, a.b1.z, i2); i2 = sdot4((r.q1.w >> 4) & m, a.b1.w, i2);
    float d = f16_to_f32(r.hdr.x & 0xffff);
    float dmin = f16_to_f32(r.hdr.x >> 16);
    // get_scale_min_k4 (quant.rs:176-185) for j = 2g and 2g+1 on the 12
    // scale bytes held in hdr.y, hdr.z, hdr.w
    const uint32_t s0 = r.hdr.y, s1 = r.hdr.z, s2 = r.hdr.w;
    uint32_t sc1, m1, sc2, m2;
    if (g < 2) {  // j = 2g, 2g+1 < 4: low 6 bits of bytes j (scale) and j+4 (min)
      uint32_t sh1 = 16 * g, sh2 = 16 * g + 8;
      sc1 = (s0 >> sh1) & 63;
      m1 = (s1 >> sh1) & 63;
      sc2 = (s0 >> sh2) & 63;
      m2 = (s1 >> sh2) & 63;
    } else {  // j >= 4: nibbles of byte j+4, top bits of bytes j-4 and j
      uint32_t sh1 = 16 * (g - 2), sh2 = sh1 + 8;
      sc1 = ((s2 >> sh1) & 0xF) | (((s0 >> sh1) >> 6 & 3) << 4);
      m1 = ((s2 >> sh1) >> 4 & 0xF) | (((s1 >> sh1) >> 6 & 3) << 4);
      sc2 = ((s2 >> sh2) & 0xF) | (((s0 >> sh2) >> 6 & 3) << 4);
      m2 = ((s2 >> sh2) >> 4 & 0xF) | (((s1 >> sh2) >> 6 & 3) << 4);
    }
    float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
    float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
    t[0] = a.da * (d1 * (float)i1 - mm1 * a.sa) + a.db * (d2 * (float)i2 - mm2 * a.sb);
  }
};

template <>
struct MU<RLH_TYPE_Q6_K> {
  static constexpr int kT = 4;
  struct W {
    uint4 ql0, ql1, qh;
    uint2 sc;
    uint32_t d;
  };
  struct A {
    uint4 a[4];
    float da[4], sa[4];
  };
  __device__ __forceinline__ static uint32_t units(uint32_t cols) { return cols >> 6; }
  __device__ __forceinline__ static A act(const Q8Ptr& q, uint32_t u) {
    uint32_t bi = u >> 2, half = (u >> 1) & 1, sub = u & 1;
    uint32_t ab = bi * 8 + half * 4;
    A a;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      a.a[c] = ld_g16(q.qs + (size_t)(ab + c) * 32 + sub * 16);
      a.da[c] = ld_gf(q.d + ab + c);
      a.sa[c] = (float)ld_gi(q.s16 + (size_t)(ab + c) * 2 + sub);
    }
    return a;
  }
  __device__ __forceinline__ static W load(const DevMat& w, uint32_t row, uint32_t u) {
    uint32_t nsb = w.cols >> 8;
    uint32_t bi = u >> 2, half = (u >> 1) & 1, sub = u & 1;
    size_t sbi = (size_t)row * nsb + bi;
    const uint8_t* ql = w.a + sbi * 128 + half * 64 + sub * 16;
    W r;
    r.ql0 = ld_nt16(ql);
    r.ql1 = ld_nt16(ql + 32);
    r.qh = ld_nt16(w.b + sbi * 64 + half * 32 + sub * 16);
    r.sc = ld_g8(w.c + sbi * 16 + half * 8);
    r.d = ld_g2(w.d + sbi * 2);
    return r;
  }
  __device__ __forceinline__ static void terms(const W r, const A& a, uint32_t u, lfloat* t) {
    uint32_t sub = u & 1;
    const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x03030303u;
    const uint32_t l0[4] = {r.ql0.x, r.ql0.y, r.ql0.z, r.ql0.w};
    const uint32_t l1[4] = {r.ql1.x, r.ql1.y, r.ql1.z, r.ql1.w};
    const uint32_t h[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    float d = f16_to_f32(r.d);
    float out[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint32_t av[4] = {a.a[c].x, a.a[c].y, a.a[c].z, a.a[c].w};
      int ss = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t lo = (c & 1) ? l1[k] : l0[k];
        uint32_t nib = (c < 2) ? (lo & m4) : ((lo >> 4) & m4);
        uint32_t uu = nib | (((h[k] >> (2 * c)) & m2) << 4);
        ss = sdot4(uu, av[k], ss);
      }
      // sc[sub + 2c] of the half's 8 scale bytes (simd.rs:626-629)
      uint32_t word = (c < 2) ? r.sc.x : r.sc.y;
      uint32_t shift = 8 * ((sub + 2 * c) & 3);
      float scf = (float)(int8_t)((word >> shift) & 0xff);
      out[c] = d * scf * ((float)ss - 32.0f * a.sa[c]) * a.da[c];
    }
    f32x4_t v = {out[0], out[1], out[2], out[3]};
    *(lf32x4*)t = v;
  }
};

template <>
struct MU<RLH_TYPE_Q8_0> {
  static constexpr int kT = 1;
  struct W {
    uint4 q0, q1;
    uint32_t d;
  };
  struct A {
    uint4 a0, a1;
    float da;
  };
  __device__ __forceinline__ static uint32_t units(uint32_t cols) { return cols >> 5; }
  __device__ __forceinline__ static A act(const Q8Ptr& q, uint32_t u) {
    const int8_t* p = q.qs + (size_t)u * 32;
    A a;
    a.a0 = ld_g16(p);
    a.a1 = ld_g16(p + 16);
    a.da = ld_gf(q.d + u);
    return a;
  }
  __device__ __forceinline__ static W load(const DevMat& w, uint32_t row, uint32_t u) {
    size_t b = (size_t)row * (w.cols >> 5) + u;
    const uint8_t* qp = w.a + b * 32;
    W r;
    r.q0 = ld_nt16(qp);
    r.q1 = ld_nt16(qp + 16);
    r.d = ld_g2(w.b + b * 2);
    return r;
  }
  __device__ __forceinline__ static void terms(const W r, const A& a, uint32_t, lfloat* t) {
    int i = 0;
    i = sdot4(r.q0.x, a.a0.x, i); i = sdot4(r.q0.y, a.a0.y, i); i = sdot4(r.q0.z, a.a0.z, i);
    i = sdot4(r.q0.w, a.a0.w, i); i = sdot4(r.q1.x, a.a1.x, i); i = sdot4(r.q1.y, a.a1.y, i);
    i = sdot4(r.q1.z, a.a1.z, i); i = sdot4(r.q1.w, a.a1.w, i);
    t[0] = f16_to_f32(r.d) * (float)i * a.da;
  }
};

template <>
struct MU<RLH_TYPE_Q4_0> {
  static constexpr int kT = 1;
  struct W {
    uint4 q;
    uint32_t d;
  };
  struct A {
    uint4 a0, a1;
    float da;
    int s;
  };
  __device__ __forceinline__ static uint32_t units(uint32_t cols) { return cols >> 5; }
  __device__ __forceinline__ static A act(const Q8Ptr& q, uint32_t u) {
    const int8_t* p = q.qs + (size_t)u * 32;
    A a;
    a.a0 = ld_g16(p);
    a.a1 = ld_g16(p + 16);
    a.da = ld_gf(q.d + u);
    a.s = ld_gi(q.s + u);
    return a;
  }
  __device__ __forceinline__ static W load(const DevMat& w, uint32_t row, uint32_t u) {
    size_t b = (size_t)row * (w.cols >> 5) + u;
    W r;
    r.q = ld_nt16(w.a + b * 16);
    r.d = ld_g2(w.b + b * 2);
    return r;
  }
  __device__ __forceinline__ static void terms(const W r, const A& a, uint32_t, lfloat* t) {
    const uint32_t m = 0x0F0F0F0Fu;
    int i0 = 0, i1 = 0;
    i0 = sdot4(r.q.x & m, a.a0.x, i0); i0 = sdot4(r.q.y & m, a.a0.y, i0);
    i0 = sdot4(r.q.z & m, a.a0.z, i0); i0 = sdot4(r.q.w & m, a.a0.w, i0);
    i1 = sdot4((r.q.x >> 4) & m, a.a1.x, i1); i1 = sdot4((r.q.y >> 4) & m, a.a1.y, i1);
    i1 = sdot4((r.q.z >> 4) & m, a.a1.z, i1); i1 = sdot4((r.q.w >> 4) & m, a.a1.w, i1);
    t[0] = f16_to_f32(r.d) * (float)(i0 + i1 - 8 * a.s) * a.da;
  }
};

// In-order sum of n terms (the per-row f32 chain).
__device__ __forceinline__ float chain(float acc, const lfloat* t, uint32_t n) {
  uint32_t k = 0;
  for (; k + 4 <= n; k += 4) {
    f32x4_t v = *(const lf32x4*)(t + k);
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
  }
  for (; k < n; k++) acc = acc + t[k];
  return acc;
}

// Rows [row0, row0 + nrows) of matrix `w` (nrows <= 4 * NS * P). Row r is
// summed by block thread chain_lane0 + r, which gets the total as result.
// Lane layout in P-packed groups: lane -> (sub = lane / (64/P), unit
// offset = lane % (64/P)); wave w owns rows [w*NS*P, (w+1)*NS*P).
template <uint32_t TY, int P, int NS>
__device__ __forceinline__ float mv_rows(const DevMat& w, const Q8Ptr& act, uint32_t row0, uint32_t nrows, uint32_t chain_lane0,
                         lfloat* tile) {
  using U = MU<TY>;
  constexpr int kT = U::kT;
  constexpr uint32_t kUnits = 64 / P;      // units of one row per wave instruction
  constexpr uint32_t kStride = 64 * kT + 4;  // floats per tile row
  constexpr uint32_t R = 4 * NS * P;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t sub = lane / kUnits, ul = lane % kUnits;
  const uint32_t nunits = U::units(w.cols);
  float acc = 0.0f;
  const bool chain_lane = threadIdx.x >= chain_lane0 && threadIdx.x < chain_lane0 + nrows;
  const uint32_t my_row = threadIdx.x - chain_lane0;
  uint32_t prev_cn = 0;
  uint32_t buf = 0;
  for (uint32_t c0 = 0; c0 < nunits; c0 += kUnits) {
    const uint32_t cn = nunits - c0 < kUnits ? nunits - c0 : kUnits;
    const uint32_t u = c0 + ul;
    const bool uok = ul < cn;
    typename U::W raw[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) {
      uint32_t r = wave * NS * P + (uint32_t)i * P + sub;
      if (uok && r < nrows) raw[i] = U::load(w, row0 + r, u);
    }
    // chain of the previous chunk while this chunk's loads are in flight
    if (prev_cn && chain_lane) acc = chain(acc, tile + ((buf ^ 1) * R + my_row) * kStride, prev_cn * kT);
    if (uok) {
      const typename U::A a = U::act(act, u);
#pragma unroll
      for (int i = 0; i < NS; i++) {
        uint32_t r = wave * NS * P + (uint32_t)i * P + sub;
        if (r < nrows) U::terms(raw[i], a, u, tile + (buf * R + r) * kStride + ul * kT);
      }
    }
    __syncthreads();
    prev_cn = cn;
    buf ^= 1;
  }
  if (prev_cn && chain_lane) acc = chain(acc, tile + ((buf ^ 1) * R + my_row) * kStride, prev_cn * kT);
  __syncthreads();
  return acc;
}

template <uint32_t TY, int NS>
__device__ __forceinline__ float mv_rows_p(const DevMat& w, const Q8Ptr& act, uint32_t row0, uint32_t nrows, uint32_t chain_lane0,
                           lfloat* tile) {
  uint32_t units = MU<TY>::units(w.cols);
  if (units <= 16) return mv_rows<TY, 4, NS>(w, act, row0, nrows, chain_lane0, tile);
  if (units <= 32) return mv_rows<TY, 2, NS>(w, act, row0, nrows, chain_lane0, tile);
  return mv_rows<TY, 1, NS>(w, act, row0, nrows, chain_lane0, tile);
}

template <int NS>
__device__ __forceinline__ float mv_dispatch(const DevMat& w, const Q8Ptr& act, uint32_t row0, uint32_t nrows, uint32_t chain_lane0,
                             lfloat* tile) {
  switch (w.ty) {
    case RLH_TYPE_Q4_K: return mv_rows_p<RLH_TYPE_Q4_K, NS>(w, act, row0, nrows, chain_lane0, tile);
    case RLH_TYPE_Q6_K: return mv_rows_p<RLH_TYPE_Q6_K, NS>(w, act, row0, nrows, chain_lane0, tile);
    case RLH_TYPE_Q8_0: return mv_rows_p<RLH_TYPE_Q8_0, NS>(w, act, row0, nrows, chain_lane0, tile);
    case RLH_TYPE_Q4_0: return mv_rows_p<RLH_TYPE_Q4_0, NS>(w, act, row0, nrows, chain_lane0, tile);
    default: return 0.0f;
  }
}

// All segments of one launch use the same NS; a segment's rows per block is
// R = 4 * NS * P with P from its row width (host computes the same).
template <int NS>
__global__ void __launch_bounds__(kThreads) k_mv(MvLaunch L) {
  extern __shared__ float tile_generic[];
  lfloat* tile = (lfloat*)tile_generic;
  uint32_t s = 0;
  if (L.nseg > 1 && blockIdx.x >= L.seg[1].wg_begin) s = 1;
  if (L.nseg > 2 && blockIdx.x >= L.seg[2].wg_begin) s = 2;
  const MvSeg& g = L.seg[s];
  const uint32_t wg = blockIdx.x - g.wg_begin;
  const uint32_t R = g.rows_per_wg;
  const uint32_t row0 = wg * R;
  const uint32_t nrows = g.w.rows - row0 < R ? g.w.rows - row0 : R;
  if (!g.pair) {
    float acc = mv_dispatch<NS>(g.w, g.act, row0, nrows, 0, tile);
    if (threadIdx.x < nrows) {
      uint32_t r = row0 + threadIdx.x;
      if (g.resid) {  // x += xb (model.rs:714-716, 726-728)
        RLH_GLOBAL float* x = (RLH_GLOBAL float*)g.resid;
        x[r] = x[r] + acc;
      }
      if (g.y) ((RLH_GLOBAL float*)g.y)[r] = acc;
    }
    return;
  }
  // PAIR (R == 32): gate rows summed in lanes [0, 32), up rows in [32, 64).
  float ag = mv_dispatch<NS>(g.w, g.act, row0, nrows, 0, tile);
  float au = mv_dispatch<NS>(g.w2, g.act, row0, nrows, 32, tile);
  float acc = threadIdx.x < 32 ? ag : au;
  if (threadIdx.x < 64) {
    float up = __shfl(acc, (int)(threadIdx.x + 32) & 63);
    if (threadIdx.x < 32) {
      float x = acc;
      float h = (x / (1.0f + expf_glibc(-x))) * up;  // silu(g) * u (ops.rs:393-395)
      if (g.y) ((RLH_GLOBAL float*)g.y)[row0 + threadIdx.x] = h;
      q8_quant_block32(h, g.hq, row0 / 32);
    }
  }
}

}  // namespace

void launch_mv(hipStream_t st, const MvLaunch& L, uint32_t total_wgs, uint32_t lds_bytes, uint32_t ns) {
  switch (ns) {
    case 1: hipLaunchKernelGGL(k_mv<1>, dim3(total_wgs), dim3(kThreads), lds_bytes, st, L); break;
    case 2: hipLaunchKernelGGL(k_mv<2>, dim3(total_wgs), dim3(kThreads), lds_bytes, st, L); break;
    case 4: hipLaunchKernelGGL(k_mv<4>, dim3(total_wgs), dim3(kThreads), lds_bytes, st, L); break;
    default: hipLaunchKernelGGL(k_mv<8>, dim3(total_wgs), dim3(kThreads), lds_bytes, st, L); break;
  }
}

bool mv_set_max_lds(size_t bytes) {
  const void* fns[] = {(const void*)k_mv<1>, (const void*)k_mv<2>, (const void*)k_mv<4>, (const void*)k_mv<8>};
  for (const void* f : fns)
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) return false;
  return true;
}

}  // namespace rlh
