// rlh_device.h — device-side building blocks shared by the gfx950 kernels.
//
// Everything here reproduces the arithmetic of the reference's AVX2 path
// operation for operation (one IEEE rounding per operator, FMAs exactly where
// the reference issues _mm256_fmadd_ps). Sources are built with
// -ffp-contract=off so the compiler never fuses a*b+c on its own.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlh_format.h"

// Explicit address spaces: pointers reaching a kernel inside a by-value
// struct are generic, and generic (flat) loads share the LDS wait counter,
// which would make every LDS access wait for all outstanding HBM loads.
#define RLH_GLOBAL __attribute__((address_space(1)))
#define RLH_LDS __attribute__((address_space(3)))

namespace rlh {

// ---------------------------------------------------------------------------
// f16 -> f32 (quant.rs:115-157 with F16C): exact for every half value.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float f16_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// ---------------------------------------------------------------------------
// expf with the host glibc expf's results (the reference's f32::exp in
// softmax_inplace ops.rs:410 and silu ops.rs:394): expf_glibc_t of
// expf_glibc.h, the same source the host tests check against glibc expf
// over every float (tests/test_host_expf.py).
// ---------------------------------------------------------------------------
#define RLH_EXPF_QUAL __device__ __forceinline__
#define RLH_EXPF_KEEP(v) __asm__ volatile("" : "+v"(v))
#include "expf_glibc.h"

__device__ __constant__ static const uint64_t kExp2Tab[32] = RLH_EXP2_TABLE_INIT;

__device__ __forceinline__ float expf_glibc(float x) { return expf_glibc_t(x, kExp2Tab); }

// ---------------------------------------------------------------------------
// Ordered f32 chains over LDS data, the reference's sequential loops:
//   seq_sum_lds   s = ((s0 + x0) + x1) + ...  s0 = 0 (the softmax sum,
//                 ops.rs:408-412; the per-row term chain of the matvec)
//   seq_saxpy_lds o = p_j * v_j + o for j in order     (saxpy, simd.rs:674-691)
// The chain is latency bound (one dependent add per element), so the LDS
// reads run one batch ahead in two register sets used alternately; no set
// is copied into the other, which would make every batch wait for the reads
// just issued. x, p and v are 16-byte aligned.
// ---------------------------------------------------------------------------
typedef float f32x4d_t __attribute__((ext_vector_type(4)));
typedef RLH_LDS f32x4d_t lf32x4d;

__device__ __forceinline__ float seq_sum_lds(const RLH_LDS float* x, uint32_t n, float s = 0.0f) {
  const lf32x4d* x4 = (const lf32x4d*)x;
  const uint32_t nq = n / 4, nb = nq / 8;  // float4s, full batches of 8
  if (nb) {
    // the next batch's reads are unconditional (index clamped to the last
    // full batch): with a branch around them the compiler assumes either
    // path and waits for the newest reads before using the older ones
    f32x4d_t a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; i++) a[i] = x4[i];
    for (uint32_t bi = 0;; bi += 2) {
      const uint32_t q1 = 8 * min(bi + 1, nb - 1);
#pragma unroll
      for (int i = 0; i < 8; i++) b[i] = x4[q1 + i];
      __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the adds
#pragma unroll
      for (int i = 0; i < 8; i++) s = (((s + a[i].x) + a[i].y) + a[i].z) + a[i].w;
      __builtin_amdgcn_sched_barrier(0);
      if (bi + 1 >= nb) break;
      const uint32_t q2 = 8 * min(bi + 2, nb - 1);
#pragma unroll
      for (int i = 0; i < 8; i++) a[i] = x4[q2 + i];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; i++) s = (((s + b[i].x) + b[i].y) + b[i].z) + b[i].w;
      __builtin_amdgcn_sched_barrier(0);
      if (bi + 2 >= nb) break;
    }
  }
  for (uint32_t q = 8 * nb; q < nq; q++) {
    const f32x4d_t v = x4[q];
    s = (((s + v.x) + v.y) + v.z) + v.w;
  }
  for (uint32_t j = 4 * nq; j < n; j++) s = s + x[j];
  return s;
}

__device__ __forceinline__ float seq_saxpy_lds(const RLH_LDS float* p, const RLH_LDS float* v, uint32_t n, float o) {
  const lf32x4d* p4 = (const lf32x4d*)p;
  const lf32x4d* v4 = (const lf32x4d*)v;
  const uint32_t nq = n / 4, nb = nq / 4;  // float4s, full batches of 4 (16 positions)
  if (nb) {
    f32x4d_t pa[4], va[4], pb[4], vb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) pa[i] = p4[i], va[i] = v4[i];
    for (uint32_t bi = 0;; bi += 2) {
      const uint32_t q1 = 4 * min(bi + 1, nb - 1);
#pragma unroll
      for (int i = 0; i < 4; i++) pb[i] = p4[q1 + i], vb[i] = v4[q1 + i];
      __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the chain
#pragma unroll
      for (int i = 0; i < 4; i++) {
        o = pa[i].x * va[i].x + o;
        o = pa[i].y * va[i].y + o;
        o = pa[i].z * va[i].z + o;
        o = pa[i].w * va[i].w + o;
      }
      __builtin_amdgcn_sched_barrier(0);
      if (bi + 1 >= nb) break;
      const uint32_t q2 = 4 * min(bi + 2, nb - 1);
#pragma unroll
      for (int i = 0; i < 4; i++) pa[i] = p4[q2 + i], va[i] = v4[q2 + i];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        o = pb[i].x * vb[i].x + o;
        o = pb[i].y * vb[i].y + o;
        o = pb[i].z * vb[i].z + o;
        o = pb[i].w * vb[i].w + o;
      }
      __builtin_amdgcn_sched_barrier(0);
      if (bi + 2 >= nb) break;
    }
  }
  for (uint32_t q = 4 * nb; q < nq; q++) {
    const f32x4d_t a = p4[q], b = v4[q];
    o = a.x * b.x + o;
    o = a.y * b.y + o;
    o = a.z * b.z + o;
    o = a.w * b.w + o;
  }
  for (uint32_t j = 4 * nq; j < n; j++) o = p[j] * v[j] + o;
  return o;
}

// LDS copy of kExp2Tab: every thread of the block calls it; visible to the
// block after the next barrier.
typedef RLH_LDS uint64_t lu64;
__device__ __forceinline__ void exp_tab_to_lds(lu64* tab) {
  if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Tab[threadIdx.x];
}

// The same copy as one wave's LDS DMA (global_load_lds, 4 bytes per lane): no
// register round trip, so nothing waits for it until the wave's vector-memory
// count says it has landed (wait_vmcnt), and the block's barrier after that.
__device__ __forceinline__ void exp_tab_dma(lu64* tab) {
  const uint32_t lane = threadIdx.x & 63;
  __builtin_amdgcn_global_load_lds((const RLH_GLOBAL void*)((const uint32_t*)(const void*)kExp2Tab + lane),
                                   (RLH_LDS void*)tab, 4, 0, 0);
}

// ---------------------------------------------------------------------------
// Waits and barriers that leave the wave's global loads in flight.
//
// __syncthreads() is a release/acquire fence plus s_barrier; in a kernel that
// copies HBM -> LDS with global_load_lds the fence waits for every
// outstanding vector-memory operation (vmcnt(0)), including register loads of
// weights meant to stay in flight. A prologue that stages its inputs by DMA
// therefore issues the DMA first, then the weight loads, then waits with
// wait_vmcnt<n> (n = loads issued after the DMA: the counter retires in
// issue order) and meets the other waves at lds_barrier().
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  // gfx9 s_waitcnt: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] at [15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// Block barrier for LDS traffic: this wave's LDS accesses have completed
// (lgkmcnt(0)); vector-memory operations are not waited for. The asm's memory
// clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
  asm volatile("s_barrier" ::: "memory");
}

// ---------------------------------------------------------------------------
// Bounded waits on an LDS counter written by other waves of the same block.
// Every such wait ends by construction (the producers it waits for never
// wait on it); the bound turns a broken invariant into an error instead of a
// hang or silently wrong values: once kWaitPolls polls (~1.8 s of sleeps)
// have passed, the wave gives up, lane 0 sets `bit` in the device error word
// `err` (nullable) and the host reports RLH_EDEVICE after the step. The wait
// is wave-uniform (every lane reads the same counter).
// ---------------------------------------------------------------------------
constexpr uint32_t kWaitPolls = 1u << 26;
constexpr uint32_t kErrMvRing = 1u, kErrMvSplit = 2u, kErrAttnExp = 4u;

__device__ __forceinline__ void wait_lds_count(const RLH_LDS uint32_t* ctr, uint32_t need, uint32_t* err,
                                               uint32_t bit) {
  for (uint32_t spin = 0;; spin++) {
    if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= need) break;
    if (spin == kWaitPolls) {
      if (err && (threadIdx.x & 63) == 0)
        __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// Exact AVX2 reduction tree over 32 "slot" accumulators held in lanes 0..31
// of a wave: slot 8k+l is lane l of the reference's accumulator a_k.
//   A_l = (a0_l + a1_l) + (a2_l + a3_l)            (simd.rs:308, 370)
//   hsum(A) = ((A0+A4)+(A2+A6)) + ((A1+A5)+(A3+A7)) (simd.rs:261-270)
// Every lane returns the result.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float avx2_tree32(float a) {
  // the partner lanes read below (l + 8, l + 16, l + 4, l + 2, l + 1 for the
  // lanes whose sums are used) stay inside the groups the DPP row shift and
  // the 32-lane swizzle address, so the operands match the shuffle-down tree
  const float b = a + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x108, 0xf, 0xf, false));
  const float A = b + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(b), 0x401F));  // lane ^ 16
  const float s = A + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(A), 0x104, 0xf, 0xf, false));
  const float t = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x102, 0xf, 0xf, false));
  const float r = t + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x101, 0xf, 0xf, false));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
}

// Sum of squares of rmsnorm_core (simd.rs:285-313) for one wave: lanes 0..31
// own the 32 FMA chains; the 8-wide remainder loop feeds slots 0..7; the
// scalar tail is added last, in order. Returns ss in every lane.
__device__ __forceinline__ float rms_sumsq_wave(const float* x, int n) {
  int lane = threadIdx.x & 63;
  int n32 = (n / 32) * 32;
  int n8 = n32 + ((n - n32) / 8) * 8;
  float acc = 0.0f;
  if (lane < 32) {
    for (int i = lane; i < n32; i += 32) acc = __builtin_fmaf(x[i], x[i], acc);
    if (lane < 8)
      for (int i = n32 + lane; i < n8; i += 8) acc = __builtin_fmaf(x[i], x[i], acc);
  }
  float ss = avx2_tree32(acc);
  for (int i = n8; i < n; i++) ss = ss + x[i] * x[i];
  return ss;
}

// ---------------------------------------------------------------------------
// quantize_q8 of one 32-value block (simd.rs:126-195), one value per lane of
// a 32-lane half wave (lane & 31 = position in the block).
// amax -> d = amax/127 -> inv = 1/d -> q = RNE(v*inv) (_mm256_cvtps_epi32) with
// packs saturation: out-of-range conversions give INT_MIN -> -128.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int cvtps_packs_i8(float r) {
  // r is already rounded to an integer value (or NaN/inf).
  if (!(r >= -2147483648.0f && r < 2147483648.0f)) return -128;  // INT_MIN -> -128
  int v = (int)r;
  return v > 127 ? 127 : (v < -128 ? -128 : v);
}

using Q8Out = Q8Mut;

__device__ __forceinline__ void q8_quant_block32(float v, Q8Out o, uint32_t blk) {
  int l = threadIdx.x & 31;
  float a = fabsf(v);
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) a = fmaxf(a, __shfl_xor(a, m, 32));
  float d = a / 127.0f;
  float inv = d > 0.0f ? 1.0f / d : 0.0f;
  int q = cvtps_packs_i8(__builtin_rintf(v * inv));
  int s = q;
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) s += __shfl_xor(s, m, 16);  // half sums
  int tot = s + __shfl_xor(s, 16, 32);
  o.qs[(size_t)blk * 32 + l] = (int8_t)q;
  if (l == 0) {
    o.d[blk] = d;
    o.s[blk] = tot;
    o.s16[(size_t)blk * 2] = s;
  } else if (l == 16) {
    o.s16[(size_t)blk * 2 + 1] = s;
  }
}

// The same for a whole wave holding two blocks, lanes 0..31 = block blk and
// 32..63 = block blk + 1 (every lane active; the stores of half h happen
// when store[h]). The reductions use DPP instead of LDS-routed shuffles:
// inclusive prefix steps (row_shr 1, 2, 4, 8) leave each 16-lane row's
// result in its lane 15, row_bcast:15 on rows 1 and 3 folds row 0 into row
// 1 and row 2 into row 3, and readlane fetches the per-row / per-block
// values. amax is order-free and the sums are exact integers.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dpp_keep_f(float v) {  // invalid source: keep own value
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_zero_i(int v) {  // invalid source: 0
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ void q8_quant_wave2(float v, Q8Out o, uint32_t blk, bool store0, bool store1) {
  const uint32_t lane = threadIdx.x & 63, l = lane & 31;
  float a = fabsf(v);
  a = fmaxf(a, dpp_keep_f<0x111>(a));
  a = fmaxf(a, dpp_keep_f<0x112>(a));
  a = fmaxf(a, dpp_keep_f<0x114>(a));
  a = fmaxf(a, dpp_keep_f<0x118>(a));
  a = fmaxf(a, dpp_keep_f<0x142, 0xa>(a));  // rows 1, 3 take rows 0, 2
  const float amax_lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 31));  // lane index: uniform
  const float amax_hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 63));
  const float amax = lane < 32 ? amax_lo : amax_hi;
  const float d = amax / 127.0f;
  const float inv = d > 0.0f ? 1.0f / d : 0.0f;
  const int q = cvtps_packs_i8(__builtin_rintf(v * inv));
  int s = q;
  s += dpp_zero_i<0x111>(s);
  s += dpp_zero_i<0x112>(s);
  s += dpp_zero_i<0x114>(s);
  s += dpp_zero_i<0x118>(s);
  const int r0 = __builtin_amdgcn_readlane(s, 15), r1 = __builtin_amdgcn_readlane(s, 31);
  const int r2 = __builtin_amdgcn_readlane(s, 47), r3 = __builtin_amdgcn_readlane(s, 63);
  const bool hi = lane >= 32;
  if (hi ? store1 : store0) {
    const uint32_t b = blk + (hi ? 1u : 0u);
    o.qs[(size_t)b * 32 + l] = (int8_t)q;
    if (l == 0) {
      o.d[b] = d;
      o.s[b] = hi ? r2 + r3 : r0 + r1;
      o.s16[(size_t)b * 2] = hi ? r2 : r0;
      o.s16[(size_t)b * 2 + 1] = hi ? r3 : r1;
    }
  }
}

// Cross-lane moves inside groups of 8 lanes with DPP (no LDS round trip):
// lane ^ 1 and lane ^ 2 within a quad, and the mirror 7 - i of the 8-lane
// half-row, which pairs every lane of one quad with a lane of the other.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141;

// quantize_q8 of one 32-value block held as 4 consecutive values per lane in
// 8 consecutive lanes (lane & 7 = which 4 values; the group starts at a lane
// multiple of 8 and all 8 lanes are active). Same arithmetic as
// q8_quant_block32; amax is order-free and the sums are exact integers, so
// the DPP reduction order does not matter. Stores 4 packed bytes per lane.
struct Q8Blk8x4 {
  uint32_t packed;  // this lane's 4 quants
  float d;          // block scale
  int tot;          // sum of the 32 quants
  int s;            // sum of this lane's 16-value half
};
__device__ __forceinline__ Q8Blk8x4 q8_block8x4(float v0, float v1, float v2, float v3) {
  const float a0 = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
  float a = fmaxf(a0, dpp_f<kDppXor1>(a0));
  a = fmaxf(a, dpp_f<kDppXor2>(a));
  a = fmaxf(a, dpp_f<kDppHalfMirror>(a));
  const float d = a / 127.0f;
  const float inv = d > 0.0f ? 1.0f / d : 0.0f;
  const int q0 = cvtps_packs_i8(__builtin_rintf(v0 * inv));
  const int q1 = cvtps_packs_i8(__builtin_rintf(v1 * inv));
  const int q2 = cvtps_packs_i8(__builtin_rintf(v2 * inv));
  const int q3 = cvtps_packs_i8(__builtin_rintf(v3 * inv));
  int s = q0 + q1 + q2 + q3;
  s = s + dpp_i<kDppXor1>(s);
  s = s + dpp_i<kDppXor2>(s);  // sum of the 16-value half (lanes 0-3 / 4-7)
  Q8Blk8x4 r;
  r.tot = s + dpp_i<kDppHalfMirror>(s);
  r.s = s;
  r.d = d;
  r.packed =
      (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)q3 << 24);
  return r;
}

__device__ __forceinline__ void q8_quant_block8x4(float v0, float v1, float v2, float v3, Q8Out o, uint32_t blk) {
  const int l = threadIdx.x & 7;
  const Q8Blk8x4 r = q8_block8x4(v0, v1, v2, v3);
  *(RLH_GLOBAL uint32_t*)(o.qs + (size_t)blk * 32 + 4 * l) = r.packed;
  if (l == 0) {
    ((RLH_GLOBAL float*)o.d)[blk] = r.d;
    ((RLH_GLOBAL int32_t*)o.s)[blk] = r.tot;
    ((RLH_GLOBAL int32_t*)o.s16)[(size_t)blk * 2] = r.s;
  } else if (l == 4) {
    ((RLH_GLOBAL int32_t*)o.s16)[(size_t)blk * 2 + 1] = r.s;
  }
}

// Sum of squares of rmsnorm_core (simd.rs:285-313) over a row staged in LDS,
// computed by one wave: lanes 0..31 run the 32 FMA chains (8 independent
// loads in flight per step), remainder loop into slots 0..7, then the AVX2
// tree and the in-order scalar tail. Returns ss in every lane.
__device__ __forceinline__ float rms_sumsq_lds(const RLH_LDS float* x, int n) {
  const int lane = threadIdx.x & 63;
  const int n32 = (n / 32) * 32;
  const int n8 = n32 + ((n - n32) / 8) * 8;
  float acc = 0.0f;
  if (lane < 32) {
    int i = lane;
    // batches of 32 elements per lane, the next batch's reads issued before
    // the current batch's chain (two register sets used alternately, the
    // reads unconditional with the batch index clamped, as in seq_sum_lds)
    const int nb = n32 / (32 * 32);
    if (nb > 0) {
      float a[32], b[32];
#pragma unroll
      for (int k = 0; k < 32; k++) a[k] = x[i + 32 * k];
      for (int bi = 0;; bi += 2) {
        const int o1 = (bi + 1 < nb ? bi + 1 : nb - 1) * 1024;
#pragma unroll
        for (int k = 0; k < 32; k++) b[k] = x[i + o1 + 32 * k];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 32; k++) acc = __builtin_fmaf(a[k], a[k], acc);
        __builtin_amdgcn_sched_barrier(0);
        if (bi + 1 >= nb) break;
        const int o2 = (bi + 2 < nb ? bi + 2 : nb - 1) * 1024;
#pragma unroll
        for (int k = 0; k < 32; k++) a[k] = x[i + o2 + 32 * k];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 32; k++) acc = __builtin_fmaf(b[k], b[k], acc);
        __builtin_amdgcn_sched_barrier(0);
        if (bi + 2 >= nb) break;
      }
      i += nb * 1024;
    }
    for (; i + 32 * 7 < n32; i += 32 * 8) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; k++) v[k] = x[i + 32 * k];
#pragma unroll
      for (int k = 0; k < 8; k++) acc = __builtin_fmaf(v[k], v[k], acc);
    }
    for (; i < n32; i += 32) acc = __builtin_fmaf(x[i], x[i], acc);
    if (lane < 8)
      for (int j = n32 + lane; j < n8; j += 8) acc = __builtin_fmaf(x[j], x[j], acc);
  }
  float ss = avx2_tree32(acc);
  for (int i = n8; i < n; i++) ss = ss + x[i] * x[i];
  return ss;
}

// get_scale_min_k4 (quant.rs:176-185) on the 12 scale bytes.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Load helpers that force global_load_* instructions.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld_g16(const void* p) {
  u32x4_t v = *(const RLH_GLOBAL u32x4_t*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
// 16-byte streaming load (weights are read once per token).
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  u32x4_t v = __builtin_nontemporal_load((const RLH_GLOBAL u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_g8(const void* p) {
  u32x2_t v = *(const RLH_GLOBAL u32x2_t*)p;
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld_g4(const void* p) { return *(const RLH_GLOBAL uint32_t*)p; }
__device__ __forceinline__ uint32_t ld_g2(const void* p) { return *(const RLH_GLOBAL uint16_t*)p; }
__device__ __forceinline__ float ld_gf(const float* p) { return *(const RLH_GLOBAL float*)p; }
typedef float f32x4v_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_gf4(const float* p) {
  f32x4v_t v = *(const RLH_GLOBAL f32x4v_t*)p;
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ int ld_gi(const int32_t* p) { return *(const RLH_GLOBAL int32_t*)p; }

// ---------------------------------------------------------------------------
// Element dequantisation in the device layout (quant.rs:191-385).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t item_u8(const DevMat& w, uint32_t row, uint32_t j, uint32_t o) {
  return w.a[item_offset(w, row, j, o)];
}
__device__ __forceinline__ uint32_t item_u16(const DevMat& w, uint32_t row, uint32_t j, uint32_t o) {
  return item_u8(w, row, j, o) | (item_u8(w, row, j, o + 1) << 8);
}

__device__ __forceinline__ float dq_elem(const DevMat& w, uint32_t row, uint32_t i) {
  const uint32_t j = i >> 8, p = i & 255;
  switch (w.ty) {
    case RLH_TYPE_Q4_K: {
      const uint32_t g = p >> 6, hi = (p >> 5) & 1, l = p & 31;
      const float d = f16_to_f32(item_u16(w, row, j, 0));
      const float dmin = f16_to_f32(item_u16(w, row, j, 2));
      uint8_t sb[12];
      for (int k = 0; k < 12; k++) sb[k] = (uint8_t)item_u8(w, row, j, 4 + k);
      uint32_t sc, m;
      scale_min_k4((int)(2 * g + hi), sb, sc, m);
      const float d1 = d * (float)sc;
      const float mm1 = dmin * (float)m;
      const uint32_t q = (item_u8(w, row, j, 16 + 32 * g + l) >> (4 * hi)) & 0xF;
      return d1 * (float)q - mm1;
    }
    case RLH_TYPE_Q5_K: {  // quant.rs:313-349: d1 * (q + 16 * hbit) - mm1
      const uint32_t g = p >> 6, hi = (p >> 5) & 1, l = p & 31, sub = 2 * g + hi;
      const float d = f16_to_f32(item_u16(w, row, j, 0));
      const float dmin = f16_to_f32(item_u16(w, row, j, 2));
      uint8_t sb[12];
      for (int k = 0; k < 12; k++) sb[k] = (uint8_t)item_u8(w, row, j, 4 + k);
      uint32_t sc, m;
      scale_min_k4((int)sub, sb, sc, m);
      const float d1 = d * (float)sc;
      const float mm1 = dmin * (float)m;
      const uint32_t q = (item_u8(w, row, j, 48 + 32 * g + l) >> (4 * hi)) & 0xF;
      const uint32_t h = (item_u8(w, row, j, 16 + l) >> sub) & 1;
      return d1 * (float)(q + 16 * h) - mm1;
    }
    case RLH_TYPE_Q6_K: {
      const uint32_t half = p >> 7, pp = p & 127, quarter = pp >> 5, l = pp & 31;
      const float d = f16_to_f32(item_u16(w, row, j, 208));
      const uint32_t byte = item_u8(w, row, j, half * 64 + (quarter & 1) * 32 + l);
      const uint32_t nib = quarter < 2 ? (byte & 0xF) : (byte >> 4);
      const uint32_t h2 = (item_u8(w, row, j, 128 + half * 32 + l) >> (2 * quarter)) & 3;
      const int q = (int)(nib | (h2 << 4)) - 32;
      const float sc = (float)(int8_t)item_u8(w, row, j, 192 + half * 8 + (l >> 4) + 2 * quarter);
      return d * sc * (float)q;
    }
    case RLH_TYPE_Q8_0: {
      const uint32_t k = p >> 5;
      const float d = f16_to_f32(item_u16(w, row, j, 256 + 2 * k));
      return (float)(int8_t)item_u8(w, row, j, p) * d;
    }
    case RLH_TYPE_Q4_0: {
      const uint32_t k = p >> 5, t = p & 31;
      const float d = f16_to_f32(item_u16(w, row, j, 128 + 2 * k));
      const uint32_t byte = item_u8(w, row, j, k * 16 + (t & 15));
      const float x = (float)((int)(t < 16 ? (byte & 0xF) : (byte >> 4)) - 8);
      return x * d;
    }
    case RLH_TYPE_Q4_1:  // quant.rs:222-236: q * d + m
    case RLH_TYPE_Q5_0:  // quant.rs:237-254: (q5 - 16) * d
    case RLH_TYPE_Q5_1: {  // quant.rs:255-272: q5 * d + m
      const uint32_t k = p >> 5, t = p & 31;
      const uint32_t byte = item_u8(w, row, j, k * 16 + (t & 15));
      uint32_t q = t < 16 ? (byte & 0xF) : (byte >> 4);
      const uint32_t sc0 = w.ty == RLH_TYPE_Q4_1 ? 128 : 160;  // the scales follow the quants (and qh)
      if (w.ty != RLH_TYPE_Q4_1) {
        const uint32_t qh = item_u16(w, row, j, 128 + 4 * k) | (item_u16(w, row, j, 130 + 4 * k) << 16);
        q |= ((qh >> t) & 1) << 4;  // bit t of qh is the 5th bit of value t
      }
      if (w.ty == RLH_TYPE_Q5_0) return (float)((int)q - 16) * f16_to_f32(item_u16(w, row, j, sc0 + 2 * k));
      const float d = f16_to_f32(item_u16(w, row, j, sc0 + 4 * k));
      const float m = f16_to_f32(item_u16(w, row, j, sc0 + 4 * k + 2));
      return (float)q * d + m;
    }
    case RLH_TYPE_F32:
      return ((const float*)(w.a + (size_t)row * w.row_bytes))[i];
    case RLH_TYPE_F16: {
      const uint8_t* q = w.a + (size_t)row * w.row_bytes + 2 * (size_t)i;
      return f16_to_f32(q[0] | (q[1] << 8));
    }
    case RLH_TYPE_BF16: {
      const uint8_t* q = w.a + (size_t)row * w.row_bytes + 2 * (size_t)i;
      return __uint_as_float((uint32_t)(q[0] | (q[1] << 8)) << 16);
    }
    default:
      return 0.0f;
  }
}

}  // namespace rlh
