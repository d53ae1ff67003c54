// attention.hip — GQA attention over the device f32 KV cache, exact in the
// reference order (model.rs:658-711 decode, 508-545 prefill):
//   s_j  = dot_f32_avx2(q_h, K_j) * scale            (simd.rs:328-377)
//   p    = softmax_inplace(s)                        (ops.rs:398-419:
//          max, e_j = expf(s_j - max), sum = sequential sum of e_j,
//          p_j = e_j * (1/sum))
//   o_d  = sequential over j of (p_j * V_j[d]) + o_d (saxpy, simd.rs:674-691)
//
// Kernel A (k_attn_scores) is wide: one block per (kv head, 64-position
// chunk, token); each thread evaluates whole 128-dim dot products with the
// reference's 32-slot FMA tree. In decode it also applies QK-norm
// (rmsnorm_head) and NeoX RoPE to the group's q heads and, in the block that
// owns the new position, to k, and writes K/V at pos (model.rs:642-656).
// Kernel B (k_attn_out) runs one block per (head, 32-wide slice of the head
// dimension, token). The softmax sum is one sequential chain; while it runs
// the V slice streams into LDS; the products p_j * V_j[d] are formed in LDS
// and 32 lanes run the ordered saxpy chains over double-buffered V tiles.
// The 32 outputs of a slice are one Q8 block of the attn_output input.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attention.h"
#include "rlh_device.h"

namespace rlh {

namespace {

constexpr int kHd = 128;
constexpr int kChunk = 64;  // positions per scores block
typedef RLH_LDS float lfloat;
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// One head of 128 values in LDS: (+bias), rmsnorm_head (exact tree, one
// wave), then NeoX RoPE at `pos` from the glibc-built cos/sin table. The
// calling wave must be whole (64 lanes).
__device__ __forceinline__ void norm_rope_head(lfloat* hb, const float* nw, const float* rope_cs, uint32_t pos,
                                               float eps) {
  const int lane = threadIdx.x & 63;
  if (nw) {
    const int n = kHd;
    float acc = 0.0f;
    if (lane < 32)
      for (int i = lane; i < n; i += 32) acc = __builtin_fmaf(hb[i], hb[i], acc);
    float ss = avx2_tree32(acc);
    float s = 1.0f / sqrtf(ss / (float)n + eps);
    float a0 = hb[lane] * s * ld_gf(nw + lane);
    float a1 = hb[lane + 64] * s * ld_gf(nw + lane + 64);
    hb[lane] = a0;
    hb[lane + 64] = a1;
  }
  const float c = ld_gf(rope_cs + (size_t)pos * kHd + 2 * lane);
  const float sn = ld_gf(rope_cs + (size_t)pos * kHd + 2 * lane + 1);
  float x0 = hb[lane], x1 = hb[lane + 64];
  hb[lane] = x0 * c - x1 * sn;
  hb[lane + 64] = x0 * sn + x1 * c;
}

// grid: (KVH * nchunks, n_tok); block 256; static LDS.
template <bool FUSED>
__global__ void __launch_bounds__(256) k_attn_scores(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float qv[8 * kHd];
  __shared__ __attribute__((aligned(16))) float kpos[kHd];
  const int G = a.H / a.KVH;
  const uint32_t nchunks = (a.t_max + kChunk - 1) / kChunk;
  const uint32_t g = blockIdx.x / nchunks, chunk = blockIdx.x % nchunks;
  const uint32_t tok = blockIdx.y;
  const uint32_t pos = a.pos0[0] + tok;
  const uint32_t t = pos + 1;
  const uint32_t j0 = chunk * kChunk;
  if (j0 >= t) return;
  const uint32_t jn = t - j0 < (uint32_t)kChunk ? t - j0 : (uint32_t)kChunk;
  const int qd = a.H * kHd, kvd = a.KVH * kHd;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool own_pos = pos >= j0 && pos < j0 + kChunk;
  // q heads of the group -> LDS (normalised + roped here in decode)
  for (int h = wave; h < G; h += 4) {
    lfloat* hb = (lfloat*)qv + h * kHd;
    const float* src = a.q + (size_t)tok * qd + (g * G + h) * kHd;
    float v0 = ld_gf(src + lane), v1 = ld_gf(src + lane + 64);
    if (FUSED && a.bq) {
      v0 = v0 + ld_gf(a.bq + (g * G + h) * kHd + lane);
      v1 = v1 + ld_gf(a.bq + (g * G + h) * kHd + lane + 64);
    }
    hb[lane] = v0;
    hb[lane + 64] = v1;
    if (FUSED) norm_rope_head(hb, a.qn, a.rope_cs, pos, a.eps);
  }
  if (FUSED && own_pos && wave == 0) {
    lfloat* kb = (lfloat*)kpos;
    const float* ks = a.k + (size_t)tok * kvd + g * kHd;
    float v0 = ld_gf(ks + lane), v1 = ld_gf(ks + lane + 64);
    if (a.bk) {
      v0 = v0 + ld_gf(a.bk + g * kHd + lane);
      v1 = v1 + ld_gf(a.bk + g * kHd + lane + 64);
    }
    kb[lane] = v0;
    kb[lane + 64] = v1;
    norm_rope_head(kb, a.kn, a.rope_cs, pos, a.eps);
    float* kd = a.kcache + (size_t)pos * kvd + g * kHd;
    kd[lane] = kb[lane];
    kd[lane + 64] = kb[lane + 64];
    const float* vs = a.v + (size_t)tok * kvd + g * kHd;
    float* vd = a.vcache + (size_t)pos * kvd + g * kHd;
    float w0 = ld_gf(vs + lane), w1 = ld_gf(vs + lane + 64);
    if (a.bv) {
      w0 = w0 + ld_gf(a.bv + g * kHd + lane);
      w1 = w1 + ld_gf(a.bv + g * kHd + lane + 64);
    }
    vd[lane] = w0;
    vd[lane + 64] = w1;
  }
  __syncthreads();
  // one (position, head) dot per thread: 32 slot FMA chains + AVX2 tree
  for (uint32_t idx = threadIdx.x; idx < jn * (uint32_t)G; idx += 256) {
    const uint32_t jl = idx % jn, h = idx / jn, j = j0 + jl;
    const lfloat* qh = (const lfloat*)qv + h * kHd;
    const float* kr = (FUSED && j == pos) ? nullptr : a.kcache + (size_t)j * kvd + g * kHd;
    float acc[32];
#pragma unroll
    for (int s = 0; s < 32; s++) acc[s] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int s4 = 0; s4 < 8; s4++) {
        float4 kk;
        if (kr) {
          kk = ld_gf4(kr + i * 32 + s4 * 4);
        } else {
          const lfloat* kp = (const lfloat*)kpos + i * 32 + s4 * 4;
          kk = make_float4(kp[0], kp[1], kp[2], kp[3]);
        }
        const int s = s4 * 4, e = i * 32 + s;
        acc[s] = __builtin_fmaf(qh[e], kk.x, acc[s]);
        acc[s + 1] = __builtin_fmaf(qh[e + 1], kk.y, acc[s + 1]);
        acc[s + 2] = __builtin_fmaf(qh[e + 2], kk.z, acc[s + 2]);
        acc[s + 3] = __builtin_fmaf(qh[e + 3], kk.w, acc[s + 3]);
      }
    }
    float A[8];
#pragma unroll
    for (int l = 0; l < 8; l++) A[l] = (acc[l] + acc[8 + l]) + (acc[16 + l] + acc[24 + l]);
    const float dot = ((A[0] + A[4]) + (A[2] + A[6])) + ((A[1] + A[5]) + (A[3] + A[7]));
    a.scores[((size_t)tok * a.H + g * G + h) * a.t_stride + j] = dot * a.scale;
  }
}

// grid: (H, 4 slices, n_tok); block 256; dynamic LDS: e[t_max] + 2 V tiles of
// vtile positions x 32 floats.
__global__ void __launch_bounds__(256) k_attn_out(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds_generic[];
  lfloat* lds = (lfloat*)lds_generic;
  __shared__ float red[256];
  __shared__ float s_inv;
  __shared__ int s_on;
  const int h = blockIdx.x, slice = blockIdx.y, tok = blockIdx.z;
  const int G = a.H / a.KVH;
  const int kvh = h / G;
  const int qd = a.H * kHd, kvd = a.KVH * kHd;
  const uint32_t t = a.pos0[0] + tok + 1;
  const uint32_t vt = a.vtile;
  lfloat* e = lds;                                          // [t_max] (rounded to 4)
  lfloat* vb = lds + ((a.t_max + 3) & ~3u);                 // [2][vt][32]
  const float* srow = a.scores + ((size_t)tok * a.H + h) * a.t_stride;
  // V slice rows: vcache[j][kvh*128 + slice*32 .. +32]
  const float* vbase = a.vcache + kvh * kHd + slice * 32;
  // thread -> (position in tile, float4 of the 32-float row)
  const uint32_t vq = threadIdx.x & 7, vj = threadIdx.x >> 3;  // 8 float4 per row, 32 rows per pass
  const uint32_t passes = vt / 32;
  float4 pre[16];  // V of one tile (vt <= 512): passes <= 16
  auto load_tile = [&](uint32_t j0) {
#pragma unroll
    for (int p = 0; p < 16; p++) {
      uint32_t j = j0 + (uint32_t)p * 32 + vj;
      if ((uint32_t)p < passes && j < t) pre[p] = ld_gf4(vbase + (size_t)j * kvd + vq * 4);
    }
  };
  // V tile 0 starts streaming now; it lands while the softmax sum runs.
  load_tile(0);
  // scores -> e, max
  float mx = -__int_as_float(0x7f800000);
  for (uint32_t j = threadIdx.x; j < t; j += 256) {
    float s = ld_gf(srow + j);
    e[j] = s;
    mx = fmaxf(mx, s);
  }
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + st]);
    __syncthreads();
  }
  mx = red[0];
  for (uint32_t j = threadIdx.x; j < t; j += 256) e[j] = expf_glibc(e[j] - mx);
  __syncthreads();
  if (threadIdx.x == 0) {  // sequential sum of softmax_inplace
    float sum = 0.0f;
    uint32_t j = 0;
    for (; j + 4 <= t; j += 4) {
      f32x4_t v = *(const RLH_LDS f32x4_t*)(e + j);
      sum = sum + v.x;
      sum = sum + v.y;
      sum = sum + v.z;
      sum = sum + v.w;
    }
    for (; j < t; j++) sum = sum + e[j];
    s_on = sum > 0.0f;
    s_inv = 1.0f / sum;
  }
  __syncthreads();
  if (s_on) {  // p_j = e_j * inv
    const float inv = s_inv;
    for (uint32_t j = threadIdx.x; j < t; j += 256) e[j] = e[j] * inv;
    __syncthreads();
  }
  // products of tile 0
  auto store_tile = [&](uint32_t j0, lfloat* dst) {
#pragma unroll
    for (int p = 0; p < 16; p++) {
      uint32_t jl = (uint32_t)p * 32 + vj, j = j0 + jl;
      if ((uint32_t)p < passes && j < t) {
        const float pj = e[j];
        lfloat* d = dst + jl * 32 + vq * 4;
        d[0] = pj * pre[p].x;
        d[1] = pj * pre[p].y;
        d[2] = pj * pre[p].z;
        d[3] = pj * pre[p].w;
      }
    }
  };
  store_tile(0, vb);
  __syncthreads();
  float o = 0.0f;
  uint32_t buf = 0;
  for (uint32_t j0 = 0; j0 < t; j0 += vt) {
    const uint32_t jn = t - j0 < vt ? t - j0 : vt;
    const bool more = j0 + vt < t;
    if (more) load_tile(j0 + vt);
    if (threadIdx.x < 32) {  // the ordered saxpy chains
      const lfloat* pr = vb + buf * vt * 32 + threadIdx.x;
      for (uint32_t jl = 0; jl < jn; jl++) o = pr[jl * 32] + o;
    }
    if (more) store_tile(j0 + vt, vb + (buf ^ 1) * vt * 32);
    __syncthreads();
    buf ^= 1;
  }
  if (threadIdx.x < 32) {
    const uint32_t d = (uint32_t)h * kHd + (uint32_t)slice * 32 + threadIdx.x;
    ((RLH_GLOBAL float*)a.out)[(size_t)tok * qd + d] = o;
    const uint32_t nbq = (uint32_t)qd / 32;
    Q8Out ot{a.out_q8.qs + (size_t)tok * qd, a.out_q8.d + (size_t)tok * nbq, a.out_q8.s + (size_t)tok * nbq,
             a.out_q8.s16 + (size_t)tok * nbq * 2};
    q8_quant_block32(o, ot, d / 32);
  }
}

}  // namespace

uint32_t attn_vtile(uint32_t t_max) {
  // LDS budget ~150 KB: e[t_max] + 2 tiles x vt x 32 floats
  uint32_t avail = 150u * 1024u - ((t_max + 3) & ~3u) * 4u;
  uint32_t vt = 512;
  while (vt > 32 && 2u * vt * 32u * 4u > avail) vt /= 2;
  return vt;
}

size_t attn_out_lds(uint32_t t_max, uint32_t vtile) { return (size_t)((t_max + 3) & ~3u) * 4 + 2 * (size_t)vtile * 32 * 4; }

void launch_attn_scores(hipStream_t st, const AttnArgs& a, uint32_t n_tok, bool fused) {
  uint32_t nchunks = (a.t_max + kChunk - 1) / kChunk;
  dim3 grid(a.KVH * nchunks, n_tok);
  if (fused)
    hipLaunchKernelGGL(k_attn_scores<true>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(k_attn_scores<false>, grid, dim3(256), 0, st, a);
}

void launch_attn_out(hipStream_t st, const AttnArgs& a, uint32_t n_tok) {
  hipLaunchKernelGGL(k_attn_out, dim3(a.H, 4, n_tok), dim3(256), attn_out_lds(a.t_max, a.vtile), st, a);
}

bool attn_set_max_lds(size_t bytes) {
  return hipFuncSetAttribute((const void*)k_attn_out, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) ==
         hipSuccess;
}

}  // namespace rlh
